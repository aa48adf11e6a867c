"""GPU parity of the HIP path (called through the C ABI via dcnv2_amd._C).

Checks: max|y - y_ref| / max|y_ref| <= 1e-2 for
fp16/bf16 and <= 1e-4 for fp32, for the output and all five gradients.

* golden fixtures (tests/golden, made by the independent grid_sample
  formulation): every dtype, forward and backward;
* the five BASELINE configurations at full size: forward of the first and last
  image against the CPU oracle, forward+backward of one image against the
  oracle in the config dtype and in an fp32 rerun, and the whole batch against
  the independent grid_sample formulation evaluated in fp32 on the GPU;
* edge cases: mask/bias None, Cout > 256 (two M tiles), grad_input across the
  gather's cell-tile boundaries, every sample outside the image, non-contiguous
  inputs, an empty batch.
"""
from __future__ import annotations

import functools
import glob
import os

import numpy as np
import pytest
import torch

from dcnv2_amd import _C
from dcnv2_amd.workloads import CONFIGS, make_inputs
from independent import forward_backward_gs, sample_positions
from oracle import oracle
from util import GRADS, TOL, check, load_fixture

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
IN5 = ("input", "weight", "mask", "offset", "bias")
FIXTURES = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def _args(geo):
    s, p, d, G = geo["stride"], geo["padding"], geo["dilation"], geo["deformable_groups"]
    return (s, s, p, p, d, d, G)


def gpu_forward(t, geo):
    return _C.dcn_v2_forward(*(None if t[k] is None else t[k].to(DEV) for k in IN5), *_args(geo))


def gpu_backward(t, geo):
    return _C.dcn_v2_backward(*(None if t[k] is None else t[k].to(DEV) for k in IN5),
                              t["grad_output"].to(DEV), *_args(geo))


def oracle_forward(t, geo):
    return oracle.dcn_forward(*(t[k] for k in IN5), pos_f32=True, **geo)


def oracle_backward(t, geo):
    return oracle.dcn_backward(*(t[k] for k in IN5), t["grad_output"], pos_f32=True, **geo)


@functools.lru_cache(maxsize=4)
def config_inputs(idx, dtype=None):
    w = CONFIGS[idx]
    return make_inputs(w, dtype=dtype, with_grad=True)


def slice_batch(t, b0, b1):
    return {k: (v[b0:b1] if k not in ("weight", "bias") and v is not None else v)
            for k, v in t.items()}


# --------------------------------------------------------------------------- fixtures
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("fx", FIXTURES, ids=lambda p: os.path.basename(p)[:-4])
def test_fixture(fx, dtype):
    a, geo = load_fixture(fx)
    t = {k: a[k].to(dtype) for k in IN5 + ("grad_output",)}
    out = gpu_forward(t, geo)
    grads = gpu_backward(t, geo)
    torch.cuda.synchronize()
    tol = TOL[dtype]
    if dtype == torch.float32:
        refs = [a["output"]] + [a[k] for k in GRADS]
    else:  # the fixture inputs rounded to dtype, evaluated exactly by the oracle
        refs = [oracle_forward(t, geo)] + list(oracle_backward(t, geo))
    check("output", out, refs[0], tol)
    for name, g, r in zip(GRADS, grads, refs[1:]):
        check(name, g, r, tol)


# --------------------------------------------------------------------------- configs
@pytest.mark.parametrize("idx", range(len(CONFIGS)), ids=[w.name for w in CONFIGS])
def test_config_forward_full_batch_vs_oracle(idx):
    w = CONFIGS[idx]
    t = config_inputs(idx)
    out = gpu_forward(t, w.geometry())
    torch.cuda.synchronize()
    for b in sorted({0, w.B - 1}):
        ref = oracle_forward(slice_batch(t, b, b + 1), w.geometry())
        check(f"output[b={b}]", out[b:b + 1], ref, TOL[w.dtype])


@pytest.mark.parametrize("fp32", [False, True], ids=["config_dtype", "fp32"])
@pytest.mark.parametrize("idx", range(len(CONFIGS)), ids=[w.name for w in CONFIGS])
def test_config_backward_one_image_vs_oracle(idx, fp32):
    w = CONFIGS[idx]
    dtype = torch.float32 if fp32 else w.dtype
    t = slice_batch(config_inputs(idx, dtype), 0, 1)
    out = gpu_forward(t, w.geometry())
    grads = gpu_backward(t, w.geometry())
    torch.cuda.synchronize()
    check("output", out, oracle_forward(t, w.geometry()), TOL[dtype])
    for name, g, r in zip(GRADS, grads, oracle_backward(t, w.geometry())):
        check(name, g, r, TOL[dtype])


@pytest.mark.parametrize("idx", range(len(CONFIGS)), ids=[w.name for w in CONFIGS])
def test_config_full_batch_vs_gridsample(idx):
    """Whole batch at full size against the independent formulation (fp32 on
    the GPU, from the same rounded inputs).  grad_offset is compared only at
    samples at least 1e-3 away from an integer coordinate: on an integer the
    one-sided derivative depends on how each side rounds the position, and
    those points are covered by the oracle tests above."""
    w = CONFIGS[idx]
    t = config_inputs(idx)
    out = gpu_forward(t, w.geometry())
    grads = gpu_backward(t, w.geometry())
    ref = forward_backward_gs(*(t[k].to(DEV) for k in ("input", "weight", "offset", "mask",
                                                         "bias")),
                              t["grad_output"].to(DEV), dtype=torch.float32, **w.geometry())
    torch.cuda.synchronize()
    r_out, r_gi, r_goff, r_gm, r_gw, r_gb = ref
    tol = TOL[w.dtype]
    check("output", out, r_out, tol)
    check("grad_input", grads[0], r_gi, tol)
    check("grad_mask", grads[2], r_gm, tol)
    check("grad_weight", grads[3], r_gw, tol)
    check("grad_bias", grads[4], r_gb, tol)
    y, x = sample_positions(t["offset"], w.k, w.k, w.Ho, w.Wo, **w.geometry())
    far = lambda v: (v - v.round()).abs() > 1e-3  # noqa: E731
    keep = (far(y) & far(x)).view(w.B, w.groups * w.k * w.k, 1, w.Ho, w.Wo)
    keep = keep.expand(-1, -1, 2, -1, -1).reshape(t["offset"].shape)
    got = grads[1].float().cpu()[keep]
    refv = r_goff.float().cpu()[keep]
    assert keep.float().mean() > 0.5
    check("grad_offset (non-integer samples)", got, refv, tol)


# --------------------------------------------------------------------------- edge cases
def _small(dtype, B=2, C=12, H=9, W=11, Cout=20, k=3, s=1, p=1, d=1, G=3, seed=7, osc=2.0):
    w = CONFIGS[0].with_(B=B, C=C, H=H, W=W, Cout=Cout, k=k, stride=s, pad=p, dil=d, groups=G,
                         seed=seed, offset_dist=f"normal:{osc}", backward=True)
    return w, make_inputs(w, dtype=dtype)


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_mask_and_bias_none(dtype):
    w, t = _small(dtype)
    t["mask"] = None
    t["bias"] = None
    out = gpu_forward(t, w.geometry())
    grads = gpu_backward(t, w.geometry())
    torch.cuda.synchronize()
    assert grads[2] is None and grads[4] is None
    check("output", out, oracle_forward(t, w.geometry()), TOL[dtype])
    rg = oracle_backward(t, w.geometry())
    for name, g, r in zip(GRADS, grads, rg):
        if g is not None:
            check(name, g, r, TOL[dtype])


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_cout_beyond_one_tile(dtype):
    w, t = _small(dtype, Cout=300, C=70, G=1, H=10, W=13)
    out = gpu_forward(t, w.geometry())
    grads = gpu_backward(t, w.geometry())
    torch.cuda.synchronize()
    check("output", out, oracle_forward(t, w.geometry()), TOL[dtype])
    for name, g, r in zip(GRADS, grads, oracle_backward(t, w.geometry())):
        check(name, g, r, TOL[dtype])


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_grad_input_tile_boundaries(dtype):
    """grad_input where the gather's 16x16 cell tiles meet: images of 37x45
    (not multiples of 16, so the last tiles are partial) and two deformable
    groups.  The pixels of rows and columns 15 and 31 are shared by two or four
    tiles' windows, whose partial sums are merged after the gather; offsets of
    +-3 pixels spread every tile's samples over its neighbours' cells."""
    w, t = _small(dtype, B=2, C=24, H=37, W=45, Cout=20, G=2, osc=3.0)
    grads = gpu_backward(t, w.geometry())
    torch.cuda.synchronize()
    for name, g, r in zip(GRADS, grads, oracle_backward(t, w.geometry())):
        check(name, g, r, TOL[dtype])


def test_all_samples_outside_give_bias():
    w, t = _small(torch.float32)
    t["offset"] = torch.full_like(t["offset"], 1e4)
    out = gpu_forward(t, w.geometry())
    grads = gpu_backward(t, w.geometry())
    torch.cuda.synchronize()
    expect = t["bias"].view(1, -1, 1, 1).expand_as(out.cpu())
    assert torch.equal(out.cpu(), expect)
    for g in (grads[0], grads[1], grads[2], grads[3]):
        assert torch.count_nonzero(g) == 0
    torch.testing.assert_close(grads[4].cpu(), t["grad_output"].sum((0, 2, 3)))


def test_non_contiguous_inputs():
    w, t = _small(torch.float16)
    ref = gpu_forward(t, w.geometry())
    nc = {k: (v.transpose(-1, -2).contiguous().transpose(-1, -2) if v is not None and v.dim() == 4
              else v) for k, v in t.items()}
    assert not nc["input"].is_contiguous()
    out = gpu_forward(nc, w.geometry())
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), ref.cpu())


def test_empty_batch():
    w, t = _small(torch.float32, B=0)
    out = gpu_forward(t, w.geometry())
    grads = gpu_backward(t, w.geometry())
    torch.cuda.synchronize()
    assert tuple(out.shape) == (0, w.Cout, w.Ho, w.Wo)
    assert torch.count_nonzero(grads[3]) == 0 and torch.count_nonzero(grads[4]) == 0


def test_forward_deterministic():
    w, t = _small(torch.bfloat16, G=1, C=64)
    a = gpu_forward(t, w.geometry())
    b = gpu_forward(t, w.geometry())
    torch.cuda.synchronize()
    assert torch.equal(a, b)


# --------------------------------------------------------------------------- weight groups
@pytest.mark.parametrize("case", [
    # C, Cout, deformable groups, weight groups, H, W
    (24, 36, 2, 3, 11, 13),
    (128, 128, 1, 2, 17, 15),    # 64 channels per weight group: one f16 chunk each
    (16, 32, 1, 16, 9, 10),      # one input channel per weight group
], ids=["wg3_dg2", "wg2_c128", "wg16_c16"])
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_weight_groups(dtype, case):
    """torchvision's weight groups (weight [Cout, C/WG, kh, kw]): forward and all
    five gradients against the oracle's grouped loops."""
    C, Cout, G, WG, H, W = case
    w, t = _small(dtype, B=2, C=C, H=H, W=W, Cout=Cout, G=G, osc=2.0)
    t["weight"] = t["weight"][:, : C // WG].contiguous()
    out = gpu_forward(t, w.geometry())
    grads = gpu_backward(t, w.geometry())
    torch.cuda.synchronize()
    assert tuple(grads[3].shape) == tuple(t["weight"].shape)
    check("output", out, oracle_forward(t, w.geometry()), TOL[dtype])
    for name, g, r in zip(GRADS, grads, oracle_backward(t, w.geometry())):
        check(name, g, r, TOL[dtype])


@pytest.mark.parametrize("case", [
    # C, Cout, deformable groups, weight groups: every channel chunk of the
    # packed K order lies in one weight group and each group has a multiple of
    # 128 output channels, so the forward runs one launch per group over its
    # own rows and chunks and grad_weight walks only the diagonal blocks
    (128, 256, 1, 2),    # 128 rows per group (128-row tiles)
    (256, 512, 2, 2),    # 256 rows per group, one weight group per deformable group
    (256, 512, 4, 4),    # four groups of 128 rows
    (256, 256, 4, 2),    # a weight group spans two deformable groups
], ids=["c128_wg2", "c256_dg2_wg2", "c256_dg4_wg4", "c256_dg4_wg2"])
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_weight_groups_split_per_group(dtype, case):
    """Grouped GEMMs that skip the zero blocks of the block-diagonal weight:
    forward and all five gradients against the oracle's grouped loops."""
    C, Cout, G, WG = case
    w, t = _small(dtype, B=2, C=C, H=11, W=13, Cout=Cout, G=G, osc=2.0, seed=13)
    t["weight"] = t["weight"][:, : C // WG].contiguous()
    out = gpu_forward(t, w.geometry())
    grads = gpu_backward(t, w.geometry())
    torch.cuda.synchronize()
    check("output", out, oracle_forward(t, w.geometry()), TOL[dtype])
    for name, g, r in zip(GRADS, grads, oracle_backward(t, w.geometry())):
        check(name, g, r, TOL[dtype])


@pytest.mark.parametrize("case", [
    # C, Cout, deformable groups, weight groups (per-group launches, as above)
    (128, 256, 1, 2),
    (256, 512, 4, 4),
], ids=["c128_wg2", "c256_dg4_wg4"])
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_weight_groups_split_per_group_channels_last(dtype, case):
    """The per-group launches with a channels_last input, output and
    grad_output (the input read in place, the output and grad_output
    channels-last): forward and all five gradients against the oracle."""
    C, Cout, G, WG = case
    w, t = _small(dtype, B=2, C=C, H=11, W=13, Cout=Cout, G=G, osc=2.0, seed=17)
    t["weight"] = t["weight"][:, : C // WG].contiguous()
    geo = w.geometry()
    cl = torch.channels_last
    args = [None if t[k] is None else t[k].to(DEV) for k in IN5]
    args[0] = args[0].to(memory_format=cl)
    out = _C.dcn_v2_forward(*args, *_args(geo))
    go = t["grad_output"].to(DEV).to(memory_format=cl)
    grads = _C.dcn_v2_backward(*args, go, *_args(geo))
    torch.cuda.synchronize()
    assert out.is_contiguous(memory_format=cl) and grads[0].is_contiguous(memory_format=cl)
    check("output", out, oracle_forward(t, geo), TOL[dtype])
    for name, g, r in zip(GRADS, grads, oracle_backward(t, geo)):
        check(name, g, r, TOL[dtype])


# --------------------------------------------------------------------------- NCHW vs channels_last
@pytest.mark.parametrize("case", [
    # B, C, H, W, Cout: fp16 3x3, <= 64 channels, 128 < Cout <= 256 (the
    # resident-weight forward)
    (8, 64, 16, 20, 256),    # 320 pixels per image: a partial last 64-pixel tile
    (16, 48, 12, 10, 200),   # 48 channels padded to 64
], ids=["b8_c64", "b16_c48"])
def test_forward_nchw_matches_channels_last(case):
    """The resident-weight forward on an NCHW input (transposed by the pack
    launch) is bitwise equal to the same call on a channels_last copy
    (repacked with padding channels, or read in place), twice in a row, and
    matches the oracle."""
    B, C, H, W, Cout = case
    w, t = _small(torch.float16, B=B, C=C, H=H, W=W, Cout=Cout, G=1, osc=2.0, seed=61)
    geo = w.geometry()
    args = [None if t[k] is None else t[k].to(DEV) for k in IN5]
    outs = [_C.dcn_v2_forward(*args, *_args(geo)) for _ in range(2)]
    x_cl = args[0].to(memory_format=torch.channels_last)
    ref = _C.dcn_v2_forward(x_cl, *args[1:], *_args(geo))
    torch.cuda.synchronize()
    for out in outs:
        assert torch.equal(out, ref)
    check("output (NCHW input)", outs[0], oracle_forward(t, geo), TOL[torch.float16])


# --------------------------------------------------------------------------- channels_last
@pytest.mark.parametrize("case", [
    # dtype, C, deformable groups, Cout: the input is read in place when C/G is a
    # multiple of the channel chunk; channels-last output rows are stored as
    # 16-byte pieces when Cout % 8 == 0, element by element otherwise
    (torch.float16, 64, 1, 40),      # read in place
    (torch.bfloat16, 128, 2, 40),    # read in place, two groups
    (torch.float32, 64, 2, 40),      # read in place (fp32 chunk is 32 channels)
    (torch.float16, 24, 2, 40),      # padded: repacked from channels-last
    (torch.bfloat16, 18, 2, 40),     # padded, 9 channels per group: element-wise grad_input stores
    (torch.float16, 64, 1, 36),      # Cout % 8 != 0: element-wise output / grad_output access
    (torch.bfloat16, 64, 1, 300),    # two M tiles, non-warp-specialised forward
], ids=["f16_c64", "bf16_c128_dg2", "f32_c64_dg2", "f16_c24_dg2_padded", "bf16_c18_dg2_padded",
        "f16_cout36", "bf16_cout300"])
def test_channels_last_input(case):
    """A channels_last input gives a channels_last output (read and written in
    place by the kernels) equal to the oracle and to the NCHW run, and a
    backward whose grad_input is channels_last; grad_output is read in place
    in either layout.  All five gradients against the oracle for both
    grad_output layouts."""
    dtype, C, G, Cout = case
    w, t = _small(dtype, B=2, C=C, H=13, W=11, Cout=Cout, G=G, osc=2.0)
    geo = w.geometry()
    cl = torch.channels_last
    x_cl = t["input"].to(DEV).to(memory_format=cl)
    assert not x_cl.is_contiguous()
    args = [None if t[k] is None else t[k].to(DEV) for k in IN5]
    out_nchw = _C.dcn_v2_forward(*args, *_args(geo))
    out_cl = _C.dcn_v2_forward(x_cl, *args[1:], *_args(geo))
    go = t["grad_output"].to(DEV)
    grads_go_cl = _C.dcn_v2_backward(x_cl, *args[1:], go.to(memory_format=cl), *_args(geo))
    grads_go_nchw = _C.dcn_v2_backward(x_cl, *args[1:], go, *_args(geo))
    torch.cuda.synchronize()
    assert out_cl.is_contiguous(memory_format=cl) and not out_cl.is_contiguous()
    assert out_nchw.is_contiguous()
    ref = oracle_forward(t, geo)
    check("output (channels_last)", out_cl, ref, TOL[dtype])
    check("output (channels_last vs NCHW run)", out_cl, out_nchw, TOL[dtype])
    rgrads = oracle_backward(t, geo)
    for grads, tag in ((grads_go_cl, "grad_output channels_last"),
                       (grads_go_nchw, "grad_output NCHW")):
        assert grads[0].is_contiguous(memory_format=cl)
        for name, g, r in zip(GRADS, grads, rgrads):
            check(f"{name} ({tag})", g, r, TOL[dtype])


@pytest.mark.parametrize("case", [
    # dtype, C, deformable groups, Cout, H, W: images with tile-boundary rows and
    # columns (every 16th pixel), so the boundary pixels come from the rings
    (torch.float16, 64, 1, 40, 37, 35),    # read in place, 16-byte stores of 8 channels
    (torch.bfloat16, 24, 2, 40, 33, 40),   # padded groups (12 channels): element-wise stores
    (torch.float32, 64, 2, 24, 34, 33),    # fp32 (32-channel chunks), two groups
    (torch.bfloat16, 18, 2, 24, 35, 34),   # 9 channels per group
], ids=["f16_c64", "bf16_c24_dg2", "f32_c64_dg2", "bf16_c18_dg2"])
def test_grad_input_channels_last_by_cells(case):
    """A channels_last grad_input written directly by the per-cell kernel and
    ring_final_kernel (option gi_push = 1), and by the per-pixel kernel with its
    finalisation (gi_push = 0): all five gradients against the oracle, for
    either grad_output layout."""
    dtype, C, G, Cout, H, W = case
    w, t = _small(dtype, B=2, C=C, H=H, W=W, Cout=Cout, G=G, osc=3.0, seed=29)
    geo = w.geometry()
    cl = torch.channels_last
    x_cl = t["input"].to(DEV).to(memory_format=cl)
    args = [None if t[k] is None else t[k].to(DEV) for k in IN5]
    go = t["grad_output"].to(DEV)
    rgrads = oracle_backward(t, geo)
    for push in (1, 0):
        for go_t, tag in ((go.to(memory_format=cl), "grad_output channels_last"), (go, "grad_output NCHW")):
            grads = _with_option("gi_push", push,
                                 lambda: _C.dcn_v2_backward(x_cl, *args[1:], go_t, *_args(geo)))
            torch.cuda.synchronize()
            assert grads[0].is_contiguous(memory_format=cl)
            for name, g, r in zip(GRADS, grads, rgrads):
                check(f"{name} (push={push}, {tag})", g, r, TOL[dtype])


def test_channels_last_predictor_output_path():
    """dcn_v2_forward_om / dcn_v2_backward_om with a channels_last input match
    the same calls on the NCHW copy."""
    w, t = _small(torch.float16, B=2, C=64, H=10, W=12, Cout=32, G=1, osc=1.5)
    geo = w.geometry()
    x = t["input"].to(DEV)
    om = torch.cat([t["offset"], torch.logit(t["mask"].float().clamp(1e-3, 1 - 1e-3)).to(
        t["offset"].dtype)], 1).to(DEV)
    wt, b, go = t["weight"].to(DEV), t["bias"].to(DEV), t["grad_output"].to(DEV)
    x_cl = x.to(memory_format=torch.channels_last)
    ref = _C.dcn_v2_forward_om(x, wt, om, b, *_args(geo))
    got = _C.dcn_v2_forward_om(x_cl, wt, om, b, *_args(geo))
    g_ref = _C.dcn_v2_backward_om(x, wt, om, b, go, *_args(geo))
    g_cl = _C.dcn_v2_backward_om(x_cl, wt, om, b, go, *_args(geo))
    torch.cuda.synchronize()
    assert got.is_contiguous(memory_format=torch.channels_last)
    check("output", got, ref, TOL[torch.float16])
    assert g_cl[0].is_contiguous(memory_format=torch.channels_last)
    for a, r in zip(g_cl, g_ref):
        check("grad", a, r, TOL[torch.float16])


# --------------------------------------------------------------------------- torchvision signature
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_torchvision_signature_nonsquare(dtype):
    """dcnv2_amd.deform_conv2d (torchvision's argument order) with stride (2, 1),
    padding (1, 2), dilation (1, 2), a 3x2 kernel, 2 deformable groups inferred
    from the offset and 2 weight groups inferred from the weight; forward and
    autograd gradients against the oracle."""
    import dcnv2_amd
    g = torch.Generator().manual_seed(11)
    B, C, H, W, Co, kh, kw, dg, wg = 2, 32, 15, 12, 24, 3, 2, 2, 2
    Ho, Wo = (H + 2 - (kh - 1) - 1) // 2 + 1, (W + 4 - 2 * (kw - 1) - 1) + 1
    t = {"input": torch.randn(B, C, H, W, generator=g),
         "weight": torch.randn(Co, C // wg, kh, kw, generator=g) * 0.2,
         "offset": torch.randn(B, 2 * dg * kh * kw, Ho, Wo, generator=g) * 1.5,
         "mask": torch.rand(B, dg * kh * kw, Ho, Wo, generator=g),
         "bias": torch.randn(Co, generator=g) * 0.1,
         "grad_output": torch.randn(B, Co, Ho, Wo, generator=g)}
    t = {k: v.to(dtype) for k, v in t.items()}
    dev = {k: t[k].to(DEV).requires_grad_(k != "grad_output") for k in t}
    y = dcnv2_amd.deform_conv2d(dev["input"], dev["offset"], dev["weight"], dev["bias"],
                                stride=(2, 1), padding=(1, 2), dilation=(1, 2), mask=dev["mask"])
    y.backward(dev["grad_output"])
    torch.cuda.synchronize()
    geo = dict(stride=(2, 1), padding=(1, 2), dilation=(1, 2), deformable_groups=dg)
    check("output", y.detach(), oracle_forward(t, geo), TOL[dtype])
    got = [dev[k].grad for k in ("input", "offset", "mask", "weight", "bias")]
    for name, a, r in zip(GRADS, got, oracle_backward(t, geo)):
        check(name, a, r, TOL[dtype])


# --------------------------------------------------------------------------- grad_input buckets
@pytest.mark.parametrize("k", [5, 7], ids=["5x5", "7x7"])
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_large_kernel_stride1(dtype, k):
    """5x5 and 7x7 kernels at stride 1: an interior 16x16 cell tile receives
    about 256*k*k samples (6400, 12544), more than one gather batch holds
    (4096), so every such bucket is gathered in several batches."""
    w, t = _small(dtype, B=2, C=64, H=48, W=48, Cout=32, k=k, p=k // 2, G=1, osc=2.0)
    out = gpu_forward(t, w.geometry())
    grads = gpu_backward(t, w.geometry())
    torch.cuda.synchronize()
    check("output", out, oracle_forward(t, w.geometry()), TOL[dtype])
    for name, g, r in zip(GRADS, grads, oracle_backward(t, w.geometry())):
        check(name, g, r, TOL[dtype])


def _clustered(dtype, B, C, H, W, Cout, G, target, spread, seed):
    """Offsets that move every sample of every tap to within +-spread pixels
    of `target` (the clustering that learned offsets converging on an object
    produce): all samples of an image land in one or a few cell tiles."""
    w, t = _small(dtype, B=B, C=C, H=H, W=W, Cout=Cout, G=G, seed=seed)
    gen = torch.Generator().manual_seed(seed + 100)
    kk = w.k * w.k
    oy = torch.arange(w.Ho).view(1, 1, -1, 1) * w.stride - w.pad
    ox = torch.arange(w.Wo).view(1, 1, 1, -1) * w.stride - w.pad
    ki = (torch.arange(kk) // w.k).view(1, -1, 1, 1) * w.dil
    kj = (torch.arange(kk) % w.k).view(1, -1, 1, 1) * w.dil
    shape = (B, G * kk, w.Ho, w.Wo)
    dy = (target[0] - (oy + ki.repeat(1, G, 1, 1))).expand(shape) + \
        (torch.rand(shape, generator=gen) * 2 - 1) * spread
    dx = (target[1] - (ox + kj.repeat(1, G, 1, 1))).expand(shape) + \
        (torch.rand(shape, generator=gen) * 2 - 1) * spread
    off = torch.stack([dy, dx], 2).reshape(B, 2 * G * kk, w.Ho, w.Wo)
    t["offset"] = off.to(dtype)
    return w, t


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_clustered_offsets_one_bucket(dtype):
    """Every sample of an image pulled into a 7x7-pixel patch around (20.3,
    17.6): about 9*1600*2 = 28800 samples share one or two buckets (several
    gather batches each) while the other buckets are empty.  All five
    gradients against the oracle."""
    w, t = _clustered(dtype, B=1, C=64, H=40, W=40, Cout=32, G=2, target=(20.3, 17.6),
                      spread=3.0, seed=21)
    out = gpu_forward(t, w.geometry())
    grads = gpu_backward(t, w.geometry())
    torch.cuda.synchronize()
    check("output", out, oracle_forward(t, w.geometry()), TOL[dtype])
    for name, g, r in zip(GRADS, grads, oracle_backward(t, w.geometry())):
        check(name, g, r, TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["float32", "float16"])
def test_bucket_table_beyond_lds(dtype):
    """An image of 2063 x 2063 pixels has 129 x 129 = 16641 cell tiles, more
    than the bucket pre-pass's LDS tables hold (8192), so the count and place
    passes take their global-atomic variant.  1x1 kernel, 4 channels, offsets
    N(0, 2): all five gradients against the oracle."""
    w, t = _small(dtype, B=1, C=4, H=2063, W=2063, Cout=4, k=1, p=0, G=1, osc=2.0, seed=5)
    out = gpu_forward(t, w.geometry())
    grads = gpu_backward(t, w.geometry())
    torch.cuda.synchronize()
    check("output", out, oracle_forward(t, w.geometry()), TOL[dtype])
    for name, g, r in zip(GRADS, grads, oracle_backward(t, w.geometry())):
        check(name, g, r, TOL[dtype])
    del out, grads
    torch.cuda.empty_cache()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["float32", "bfloat16"])
def test_bucket_scan_launch(dtype):
    """8 images x 2 groups of 256 x 256 pixels: 17 x 17 cell tiles each, 4624
    buckets in all, more than the place pass scans by itself (4096), so the
    separate scan launch runs between the LDS-table count and place passes.
    1x1 kernel, offsets N(0, 2): all five gradients against the oracle."""
    w, t = _small(dtype, B=8, C=4, H=256, W=256, Cout=4, k=1, p=0, G=2, osc=2.0, seed=6)
    out = gpu_forward(t, w.geometry())
    grads = gpu_backward(t, w.geometry())
    torch.cuda.synchronize()
    check("output", out, oracle_forward(t, w.geometry()), TOL[dtype])
    for name, g, r in zip(GRADS, grads, oracle_backward(t, w.geometry())):
        check(name, g, r, TOL[dtype])


# --------------------------------------------------------------------------- fused backward
def _backward_path(t, geo, go, fused):
    """Backward with the fused kernel allowed or not (option bwd_fused), and
    whether the separate grad_weight stage ran (it does not when fused)."""
    with _C.option("bwd_fused", -1 if fused else 0):
        try:
            _C.profile_enable(True)
            for s in _C.STAGES:
                _C.profile_read(s)
            args = [None if t[k] is None else t[k].to(DEV) for k in IN5]
            grads = _C.dcn_v2_backward(*args, go, *_args(geo))
            torch.cuda.synchronize()
            gradw_launches = _C.profile_read("bwd_gradw")[1]
        finally:
            _C.profile_enable(False)
    return grads, gradw_launches


@pytest.mark.parametrize("case", [
    # C, deformable groups, Cout, H, W, kernel, mask and bias, grad_output channels_last
    (64, 1, 200, 12, 14, 3, True, False),   # Cout not a multiple of 32; last pixel tile partial
    (128, 2, 256, 9, 16, 3, False, False),  # two deformable groups; no mask, no bias
    (48, 1, 160, 12, 12, 3, True, False),   # 48 channels padded to the 64-channel chunk
    (64, 1, 136, 13, 11, 3, True, True),    # channels-last grad_output, N % 8 != 0
    (64, 1, 256, 10, 16, 1, True, False),   # 1x1 kernel
], ids=["cout200", "dg2_nomask", "c48_padded", "go_channels_last", "k1"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["float16", "bfloat16"])
def test_fused_backward(dtype, case):
    """The fused backward kernel (2-byte types, 129..256 output channels, one
    channel chunk per deformable group, 16-byte grad_output rows) takes the
    place of the column-gradient and grad_weight kernels: all five gradients
    against the oracle, and the two-kernel path on the same inputs likewise."""
    C, G, Cout, H, W, k, mb, go_cl = case
    w, t = _small(dtype, B=2, C=C, H=H, W=W, Cout=Cout, k=k, p=k // 2, G=G, osc=2.0, seed=21)
    if not mb:
        t["mask"] = None
        t["bias"] = None
    geo = w.geometry()
    go = t["grad_output"].to(DEV)
    if go_cl:
        go = go.to(memory_format=torch.channels_last)
    rg = oracle_backward(t, geo)
    for fused in (True, False):
        grads, gradw_launches = _backward_path(t, geo, go, fused)
        assert (gradw_launches == 0) == fused, "fused kernel selection"
        if not mb:
            assert grads[2] is None and grads[4] is None
        for name, g, r in zip(GRADS, grads, rg):
            if g is not None:
                check(f"{name} ({'fused' if fused else 'two kernels'})", g, r, TOL[dtype])


@pytest.mark.parametrize("case", [
    # C, deformable groups, Cout, H, W, stride, pad, dilation, mask and bias, grad_output channels_last
    (128, 1, 128, 23, 32, 2, 2, 2, True, False),   # the c4 shape class: two chunks, stride 2, dilation 2
    (256, 1, 100, 14, 12, 1, 1, 1, True, False),   # four chunks per group, Cout not a multiple of 32
    (96, 1, 64, 15, 16, 1, 1, 1, False, False),    # 96 channels padded to two chunks; no mask, no bias
    (256, 2, 256, 11, 16, 1, 1, 1, True, False),   # 256 padded rows, two groups of two chunks
    (128, 1, 120, 13, 11, 2, 1, 1, True, True),    # channels-last grad_output, N % 8 != 0
    (64, 1, 128, 12, 14, 1, 1, 1, True, False),    # 128 rows, one chunk per group
], ids=["c4_class", "chunks4_cout100", "c96_nomask", "mp256_dg2_chunks2", "go_channels_last",
        "mp128_one_chunk"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32],
                         ids=["float16", "bfloat16", "float32"])
def test_fused_backward_several_chunks(dtype, case):
    """The fused backward kernel on up to 128 output channels (one 128-row M
    chunk) and on deformable groups of several 64-channel chunks, whose corner
    sums each chunk adds to a per-sample buffer that a second launch turns
    into grad_offset / grad_mask.  f16 and bf16 run the fused and the
    two-kernel path, fp32 (which the fused kernel does not serve) the
    two-kernel path whatever the option says; all five gradients against the
    oracle.  (NCHW grad_output needs Ho*Wo % 8 == 0 for the fused kernel's
    16-byte row loads.)"""
    C, G, Cout, H, W, s, p, d, mb, go_cl = case
    w = CONFIGS[0].with_(B=2, C=C, H=H, W=W, Cout=Cout, k=3, stride=s, pad=p, dil=d, groups=G,
                         seed=29, offset_dist="uniform:6", mask_dist="uniform", backward=True)
    t = make_inputs(w, dtype=dtype)
    if not mb:
        t["mask"] = None
        t["bias"] = None
    geo = w.geometry()
    go = t["grad_output"].to(DEV)
    if go_cl:
        go = go.to(memory_format=torch.channels_last)
    rg = oracle_backward(t, geo)
    for fused in (True, False):
        print(f"{dtype} {case} fused={fused}", flush=True)
        grads, gradw_launches = _backward_path(t, geo, go, fused)
        assert (gradw_launches == 0) == (fused and dtype != torch.float32), "fused kernel selection"
        if not mb:
            assert grads[2] is None and grads[4] is None
        for name, g, r in zip(GRADS, grads, rg):
            if g is not None:
                check(f"{name} ({'fused' if fused else 'two kernels'})", g, r, TOL[dtype])


@pytest.mark.parametrize("scale_exp", [100, -100, 0], ids=["x2^100", "x2^-100", "x1"])
@pytest.mark.parametrize("path", [(-1, 1), (0, 1), (-1, 0)], ids=["fused_by_cells", "two_kernels_by_cells",
                                                                 "fused_per_pixel"])
def test_bf16_handoff_rows_keep_range(scale_exp, path):
    """bf16 hands the column gradient to grad_input as fp16 rows with a
    power-of-two scale per 32 channels: a grad_output scaled far outside fp16's
    range (2^100, 2^-100; bf16 holds both) gives the same relative errors as
    an unscaled one, on either column-gradient kernel and either grad_input
    kernel; one row block of all zeros (a zero grad_output image) reads back
    as zeros.  Against the fp64 oracle on the same scaled values."""
    fused, push = path
    w, t = _small(torch.bfloat16, B=2, C=64, H=19, W=17, Cout=256, G=1, osc=2.5, seed=53)
    go = t["grad_output"].double() * 2.0 ** scale_exp
    go[1] = 0.0
    t["grad_output"] = go.bfloat16()
    geo = w.geometry()
    rg = oracle_backward(t, geo)
    with _C.option("bwd_fused", fused), _C.option("gi_push", push):
        grads = gpu_backward(t, geo)
        torch.cuda.synchronize()
    assert torch.isfinite(grads[0].float()).all()
    assert (grads[0][1] == 0).all()
    for name, g, r in zip(GRADS, grads, rg):
        check(f"{name} (grad_output x 2^{scale_exp})", g, r, TOL[torch.bfloat16])


# --------------------------------------------------------------------------- grad_input kernels
def _with_option(name, value, fn):
    with _C.option(name, value):
        return fn()


@pytest.mark.parametrize("case", [
    # C, deformable groups, Cout, H, W, kernel, stride, offset scale, clustered
    (24, 2, 20, 37, 45, 3, 1, 3.0, False),    # partial edge tiles, two groups, padded channels
    (128, 1, 32, 33, 20, 3, 2, 4.0, False),   # two channel chunks per group, stride 2
    (64, 2, 32, 40, 40, 3, 1, 0.0, True),     # one crowded bucket: several record batches
    (16, 1, 8, 70, 70, 1, 1, 1.0, False),     # many buckets, 1x1 kernel, nearly empty cells
], ids=["edges_dg2", "two_chunks_s2", "clustered", "sparse_1x1"])
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_grad_input_by_cells_and_by_pixels(dtype, case):
    """grad_input from the per-cell kernel (rows read once, window summed in
    LDS) and from the per-pixel kernel (option gi_push = 1 / 0; the host picks by
    samples per bucket): all five gradients against the oracle for both."""
    C, G, Cout, H, W, k, st, osc, clustered = case
    if clustered:
        w, t = _clustered(dtype, B=1, C=C, H=H, W=W, Cout=Cout, G=G, target=(20.3, 17.6),
                          spread=3.0, seed=23)
    else:
        w, t = _small(dtype, B=2, C=C, H=H, W=W, Cout=Cout, k=k, p=k // 2, s=st, G=G, osc=osc, seed=23)
    geo = w.geometry()
    rg = oracle_backward(t, geo)
    for push in (1, 0):
        grads = _with_option("gi_push", push, lambda: gpu_backward(t, geo))
        torch.cuda.synchronize()
        for name, g, r in zip(GRADS, grads, rg):
            check(f"{name} (push={push})", g, r, TOL[dtype])
