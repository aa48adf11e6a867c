"""GPU parity of the fused offset/mask path (``dcn2_forward_om`` /
``dcn2_backward_om``, ``DCN(fused_offset_mask=True)``).

The operator reads the offset-and-mask predictor's raw output ``om``: offsets
are its first ``2*G*kh*kw`` channels and the mask is ``sigmoid`` of the rest,
the split the reference's ``DCN.forward`` makes (``dcn_v2_mm.py:133-137``).
Checks, to the tolerances of ``north_star`` (``tests/util.py::TOL``):

* against the CPU oracle in fp64 with ``offset = om[:, :2GK]`` and
  ``mask = sigmoid(om[:, 2GK:])``; the expected ``grad_om`` is
  ``cat(grad_offset, grad_mask * mask * (1 - mask))`` (chain rule through the
  sigmoid), in every dtype and at several geometries;
* against the separate-tensor path of the same library at the c1/c2 shape
  (B8 C64 128x128 Cout256, fp16), where the fused forward kernel runs the
  warp-specialised tile loop;
* the ``DCN`` module, fused against ``fused_offset_mask=False``, on outputs and
  every parameter gradient (fp32).
"""
from __future__ import annotations

import pytest
import torch

from dcnv2_amd import _C
from dcnv2_amd.dcn_v2_mm import DCN
from dcnv2_amd.workloads import CONFIGS
from oracle import oracle
from util import TOL, check

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def _om_case(B, C, H, W, Cout, k, s, p, d, G, dtype, seed, off_sd=2.0, logit_sd=1.5):
    g = torch.Generator().manual_seed(seed)
    Ho = (H + 2 * p - (d * (k - 1) + 1)) // s + 1
    Wo = (W + 2 * p - (d * (k - 1) + 1)) // s + 1
    kk = G * k * k
    om = torch.cat([torch.randn(B, 2 * kk, Ho, Wo, generator=g) * off_sd,
                    torch.randn(B, kk, Ho, Wo, generator=g) * logit_sd], dim=1)
    t = dict(input=torch.randn(B, C, H, W, generator=g),
             weight=torch.randn(Cout, C, k, k, generator=g) * (2.0 / (C * k * k)) ** 0.5,
             bias=torch.randn(Cout, generator=g) * 0.1, om=om,
             grad_output=torch.randn(B, Cout, Ho, Wo, generator=g))
    t = {key: v.to(dtype) for key, v in t.items()}
    geo = dict(stride=s, padding=p, dilation=d, deformable_groups=G)
    return t, geo, 2 * kk


def _args(geo):
    s, p, d, G = geo["stride"], geo["padding"], geo["dilation"], geo["deformable_groups"]
    return (s, s, p, p, d, d, G)


def _split(om, n_off):
    """offset, mask of the reference's split, in fp64 (om's stored values)."""
    o = om.double()
    return o[:, :n_off], torch.sigmoid(o[:, n_off:])


GEOMS = {
    "b2_c16_dg2_3x3": (2, 16, 12, 10, 24, 3, 1, 1, 1, 2),
    "b1_c64_s2_d2": (1, 64, 20, 18, 40, 3, 2, 2, 2, 1),
    "b2_c80_cout300": (2, 80, 9, 11, 300, 3, 1, 1, 1, 1),
    # fused backward with two 64-channel chunks per group (the chunks' corner
    # sums finished in a second launch, through the sigmoid of the logits)
    "b2_c128_cout96": (2, 128, 14, 16, 96, 3, 1, 1, 1, 1),
}


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("geom", list(GEOMS), ids=list(GEOMS))
def test_om_forward_backward_vs_oracle(geom, dtype):
    t, geo, n_off = _om_case(*GEOMS[geom], dtype=dtype, seed=11)
    tol = TOL[dtype]
    dev = {k: v.to(DEV) for k, v in t.items()}
    y = _C.dcn_v2_forward_om(dev["input"], dev["weight"], dev["om"], dev["bias"], *_args(geo))
    gi, gom, gw, gb = _C.dcn_v2_backward_om(dev["input"], dev["weight"], dev["om"], dev["bias"],
                                            dev["grad_output"], *_args(geo))
    torch.cuda.synchronize()
    offset, mask = _split(t["om"], n_off)
    x64 = {k: t[k].double() for k in ("input", "weight", "bias", "grad_output")}
    y_ref = oracle.dcn_forward(x64["input"], x64["weight"], mask, offset, x64["bias"],
                               pos_f32=True, **geo)
    r_gi, r_goff, r_gmask, r_gw, r_gb = oracle.dcn_backward(
        x64["input"], x64["weight"], mask, offset, x64["bias"], x64["grad_output"],
        pos_f32=True, **geo)
    m = mask.numpy()
    r_gom = torch.cat([torch.from_numpy(r_goff), torch.from_numpy(r_gmask * m * (1.0 - m))], 1)
    check("output", y, y_ref, tol)
    check("grad_input", gi, r_gi, tol)
    check("grad_om", gom, r_gom, tol)
    check("grad_om[offsets]", gom[:, :n_off], r_goff, tol)
    check("grad_om[logits]", gom[:, n_off:], r_gom[:, n_off:], tol)
    check("grad_weight", gw, r_gw, tol)
    check("grad_bias", gb, r_gb, tol)


def test_om_matches_separate_path_c2_shape():
    """Full c2 shape, fp16: fused against the separate-tensor entry points fed
    with the same split (the mask is rounded to fp16 there, not here)."""
    w = CONFIGS[2]
    t, geo, n_off = _om_case(w.B, w.C, w.H, w.W, w.Cout, w.k, w.stride, w.pad, w.dil, w.groups,
                             dtype=torch.float16, seed=5)
    tol = TOL[torch.float16]
    dev = {k: v.to(DEV) for k, v in t.items()}
    om = dev["om"]
    offset = om[:, :n_off].contiguous()
    mask = torch.sigmoid(om[:, n_off:].float()).half().contiguous()
    y = _C.dcn_v2_forward_om(dev["input"], dev["weight"], om, dev["bias"], *_args(geo))
    y_sep = _C.dcn_v2_forward(dev["input"], dev["weight"], mask, offset, dev["bias"], *_args(geo))
    check("output", y, y_sep, tol)
    gi, gom, gw, gb = _C.dcn_v2_backward_om(dev["input"], dev["weight"], om, dev["bias"],
                                            dev["grad_output"], *_args(geo))
    s_gi, s_goff, s_gmask, s_gw, s_gb = _C.dcn_v2_backward(
        dev["input"], dev["weight"], mask, offset, dev["bias"], dev["grad_output"], *_args(geo))
    mf = mask.float()
    check("grad_input", gi, s_gi, tol)
    check("grad_om[offsets]", gom[:, :n_off], s_goff, tol)
    check("grad_om[logits]", gom[:, n_off:], s_gmask.float() * mf * (1 - mf), tol)
    check("grad_weight", gw, s_gw, tol)
    check("grad_bias", gb, s_gb, tol)


def test_dcn_module_fused_matches_unfused():
    torch.manual_seed(3)
    fused = DCN(24, 40, 3, stride=1, padding=1, deformable_groups=2).to(DEV)
    # a predictor that is not zero, so that offsets and mask vary per pixel
    with torch.no_grad():
        fused.conv_offset_mask.weight.normal_(0.0, 0.2)
        fused.conv_offset_mask.bias.normal_(0.0, 0.5)
    plain = DCN(24, 40, 3, stride=1, padding=1, deformable_groups=2,
                fused_offset_mask=False).to(DEV)
    plain.load_state_dict(fused.state_dict())
    x = torch.randn(2, 24, 14, 13, device=DEV)
    xs = [x.clone().requires_grad_(True) for _ in range(2)]
    ys = [m(xi) for m, xi in zip((fused, plain), xs)]
    g = torch.randn_like(ys[0])
    for y in ys:
        y.backward(g)
    tol = TOL[torch.float32]
    check("output", ys[0], ys[1], tol)
    check("grad_input", xs[0].grad, xs[1].grad, tol)
    for (n, a), (_, b) in zip(fused.named_parameters(), plain.named_parameters()):
        check(f"grad {n}", a.grad, b.grad, tol)
