"""The backward run in slices of whole images (option ``bwd_slice_bytes``).

The library bounds the backward's workspace by running the batch in slices
whose workspace fits a budget (default 192 MiB; the reference holds one
image's columns, ``com.cu:766``).  Here the budget is set to the workspace of
two images, so a batch of five runs as slices of 2 + 2 + 1 (a batch that is
not a multiple of the slice): all five gradients against the fp64 oracle, on
the fused and the two-kernel column-gradient paths, with grad_input by cells
and per pixel, with a channels_last input read in place, and through the
predictor-output entry point (``dcn2_backward_om``, whose offsets and mask
share one tensor).  The number of slices is read off the per-stage launch
count of the pack stage (one pack launch per slice).
"""
from __future__ import annotations

import ctypes

import pytest
import torch

from dcnv2_amd import _C
from dcnv2_amd.workloads import CONFIGS, make_inputs
from oracle import oracle
from util import GRADS, TOL, check

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
IN5 = ("input", "weight", "mask", "offset", "bias")


def _args(geo):
    s, p, d, G = geo["stride"], geo["padding"], geo["dilation"], geo["deformable_groups"]
    return (s, s, p, p, d, d, G)


def _case(dtype, B, C, H, W, Cout, G, seed):
    w = CONFIGS[0].with_(B=B, C=C, H=H, W=W, Cout=Cout, k=3, stride=1, pad=1, dil=1, groups=G,
                         seed=seed, offset_dist="normal:2.5", backward=True)
    return w, make_inputs(w, dtype=dtype)


def _budget(x, weight, geo, go_layout=0, in_layout=0, images=2):
    """Backward workspace of `images` images under the current options."""
    d = _C.make_desc(x[:images], weight, *_args(geo), in_layout, go_layout)
    n = _C.lib().dcn2_backward_workspace_bytes(ctypes.byref(d))
    assert n > 0
    return n


def _sliced(fn, gradw=False):
    """Runs fn() with the pack stage's launches counted; returns (result,
    slices), and with gradw also the launches of the separate grad_weight
    stage (none when the fused kernel ran)."""
    _C.profile_enable(True)
    try:
        _C.profile_read("bwd_pack")
        _C.profile_read("bwd_gradw")
        out = fn()
        torch.cuda.synchronize()
        slices = _C.profile_read("bwd_pack")[1]
        return (out, slices, _C.profile_read("bwd_gradw")[1]) if gradw else (out, slices)
    finally:
        _C.profile_enable(False)


@pytest.mark.parametrize("case", [
    # dtype, C, deformable groups, Cout, H, W, option bwd_fused
    # (Ho*Wo % 8 == 0 where the fused kernel is to run: 16-byte grad_output rows)
    (torch.float16, 64, 1, 256, 17, 16, -1),   # fused column gradient + grad_weight
    (torch.float16, 64, 1, 256, 17, 18, 0),    # two kernels
    (torch.bfloat16, 64, 1, 200, 18, 16, -1),  # fused, Cout not a multiple of 32
    (torch.float32, 24, 2, 40, 17, 19, -1),    # fp32, two padded groups (two kernels)
    (torch.float16, 128, 1, 128, 17, 16, -1),  # fused, two chunks per group: corner sums per slice
], ids=["f16_fused", "f16_two_kernels", "bf16_fused", "f32_dg2", "f16_fused_two_chunks"])
@pytest.mark.parametrize("push", [1, 0], ids=["by_cells", "per_pixel"])
def test_backward_in_slices_vs_oracle(case, push):
    dtype, C, G, Cout, H, W, fused = case
    print(f"case {case} push={push}", flush=True)
    w, t = _case(dtype, 5, C, H, W, Cout, G, seed=41)
    geo = w.geometry()
    rg = oracle.dcn_backward(*(t[k] for k in IN5), t["grad_output"], pos_f32=True, **geo)
    dev = [t[k].to(DEV) for k in IN5]
    go = t["grad_output"].to(DEV)
    with _C.option("gi_push", push), _C.option("bwd_fused", fused):
        with _C.option("bwd_slice_bytes", _budget(dev[0], dev[1], geo)):
            grads, slices, gradw = _sliced(lambda: _C.dcn_v2_backward(*dev, go, *_args(geo)), True)
    assert slices == 3, "5 images in slices of 2 + 2 + 1"
    assert (gradw == 0) == (fused != 0 and dtype != torch.float32), "fused kernel selection"
    for name, g, r in zip(GRADS, grads, rg):
        check(f"{name} (sliced)", g, r, TOL[dtype])


def test_backward_in_slices_channels_last_input():
    """A channels_last fp16 input with 64 channels is read in place: each
    slice's input pointer is the slice's first image in the caller's tensor."""
    w, t = _case(torch.float16, 5, 64, 17, 16, 256, 1, seed=43)
    geo = w.geometry()
    rg = oracle.dcn_backward(*(t[k] for k in IN5), t["grad_output"], pos_f32=True, **geo)
    dev = [t[k].to(DEV) for k in IN5]
    x_cl = dev[0].to(memory_format=torch.channels_last)
    go = t["grad_output"].to(DEV)
    with _C.option("bwd_slice_bytes", _budget(x_cl, dev[1], geo, in_layout=1)):
        grads, slices = _sliced(lambda: _C.dcn_v2_backward(x_cl, *dev[1:], go, *_args(geo)))
    assert slices == 3
    assert grads[0].is_contiguous(memory_format=torch.channels_last)
    for name, g, r in zip(GRADS, grads, rg):
        check(f"{name} (sliced, channels_last)", g, r, TOL[torch.float16])


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=["float16", "float32"])
def test_backward_om_in_slices(dtype):
    """dcn2_backward_om in slices: offsets, mask logits and their gradients
    live in one [B, 3*G*kh*kw, Ho, Wo] tensor per image."""
    g = torch.Generator().manual_seed(47)
    B, C, H, W, Cout, G = 5, 32, 15, 14, 48, 2
    kk = G * 9
    om = torch.cat([torch.randn(B, 2 * kk, H, W, generator=g) * 2.0,
                    torch.randn(B, kk, H, W, generator=g) * 1.5], dim=1)
    t = dict(input=torch.randn(B, C, H, W, generator=g),
             weight=torch.randn(Cout, C, 3, 3, generator=g) * (2.0 / (C * 9)) ** 0.5,
             bias=torch.randn(Cout, generator=g) * 0.1, om=om,
             grad_output=torch.randn(B, Cout, H, W, generator=g))
    t = {k: v.to(dtype) for k, v in t.items()}
    geo = dict(stride=1, padding=1, dilation=1, deformable_groups=G)
    dev = {k: v.to(DEV) for k, v in t.items()}
    with _C.option("bwd_slice_bytes", _budget(dev["input"], dev["weight"], geo)):
        (gi, gom, gw, gb), slices = _sliced(lambda: _C.dcn_v2_backward_om(
            dev["input"], dev["weight"], dev["om"], dev["bias"], dev["grad_output"], *_args(geo)))
    assert slices == 3
    o = t["om"].double()
    offset, mask = o[:, :2 * kk], torch.sigmoid(o[:, 2 * kk:])
    x64 = {k: t[k].double() for k in ("input", "weight", "bias", "grad_output")}
    r_gi, r_goff, r_gmask, r_gw, r_gb = oracle.dcn_backward(
        x64["input"], x64["weight"], mask, offset, x64["bias"], x64["grad_output"],
        pos_f32=True, **geo)
    m = mask.numpy()
    tol = TOL[dtype]
    check("grad_input (om, sliced)", gi, r_gi, tol)
    check("grad_om[offsets] (sliced)", gom[:, :2 * kk], r_goff, tol)
    check("grad_om[logits] (sliced)", gom[:, 2 * kk:], r_gmask * m * (1.0 - m), tol)
    check("grad_weight (om, sliced)", gw, r_gw, tol)
    check("grad_bias (om, sliced)", gb, r_gb, tol)
