"""Seeded sweep over random layer geometries: the forward and all five
gradients against the fp64 oracle, in the three dtypes.

Each case draws the batch, channels, deformable groups, weight groups, output
channels, image size, kernel size, stride, padding and dilation, whether mask
and bias are given, the offset spread (the widest pulls many samples outside
the image), channels_last input and / or grad_output, and the backward path
(options bwd_fused and gi_push: the fused kernel or two kernels, grad_input by
cells or per pixel, or the library's own choice).  The shapes are capped so
that the oracle takes well under a second per case.  The list is fixed by the
seed, so a failure names a reproducible case (its id spells the geometry).
"""
from __future__ import annotations

import random

import pytest
import torch

from dcnv2_amd import _C
from dcnv2_amd.workloads import CONFIGS, make_inputs
from oracle import oracle
from util import GRADS, TOL, check

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
IN5 = ("input", "weight", "mask", "offset", "bias")
DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
MAX_MACS = 4e8  # oracle work per case (forward), multiply-adds


def _out(n, k, s, p, d):
    return (n + 2 * p - (d * (k - 1) + 1)) // s + 1


def _draw(rng):
    dt = rng.choice(list(DT))
    G = rng.choice([1, 1, 2, 4])
    Cg = rng.choice([4, 8, 12, 16, 24, 32, 48, 64, 80, 128])
    C = G * Cg
    Cout = rng.choice([8, 20, 32, 64, 96, 128, 160, 200, 256, 264])
    WG = rng.choice([1, 1, 1, 2, 4])
    if C % WG or Cout % WG:
        WG = 1
    k = rng.choice([1, 3, 3, 3, 5])
    s = rng.choice([1, 1, 2])
    d = rng.choice([1, 1, 2])
    p = rng.choice([0, k // 2, d * (k // 2)])
    B = rng.randint(1, 3)
    H, W = rng.randint(5, 40), rng.randint(5, 40)
    # shrink the image until the oracle's work fits
    while True:
        Ho, Wo = _out(H, k, s, p, d), _out(W, k, s, p, d)
        if Ho >= 1 and Wo >= 1 and B * Cout * Ho * Wo * (C // WG) * k * k <= MAX_MACS:
            break
        if H <= 5 and W <= 5:
            B, Cout = 1, max(8, Cout // 2)
            if Ho < 1 or Wo < 1:  # the dilated kernel overhangs the smallest image
                p += 1
        H, W = max(5, H * 3 // 4), max(5, W * 3 // 4)
    return dict(dt=dt, B=B, C=C, G=G, WG=WG, Cout=Cout, H=H, W=W, k=k, s=s, p=p, d=d,
                osc=rng.choice([0.5, 2.0, 5.0]), mask=rng.random() < 0.8, bias=rng.random() < 0.8,
                in_cl=rng.random() < 0.25, go_cl=rng.random() < 0.25,
                fused=rng.choice([-1, -1, 0]), push=rng.choice([-1, 0, 1]))


def _cases(n=120, seed=20261202):
    rng = random.Random(seed)
    return [_draw(rng) for _ in range(n)]


def _id(c):
    return (f"{c['dt']}_b{c['B']}c{c['C']}g{c['G']}w{c['WG']}o{c['Cout']}_{c['H']}x{c['W']}"
            f"k{c['k']}s{c['s']}p{c['p']}d{c['d']}_o{c['osc']}"
            f"{'' if c['mask'] else '_nomask'}{'' if c['bias'] else '_nobias'}"
            f"{'_incl' if c['in_cl'] else ''}{'_gocl' if c['go_cl'] else ''}"
            f"_f{c['fused']}_p{c['push']}")


CASES = _cases()


@pytest.mark.parametrize("c", CASES, ids=[_id(c) for c in CASES])
def test_random_geometry_vs_oracle(c):
    print(_id(c), flush=True)
    dtype = DT[c["dt"]]
    w = CONFIGS[0].with_(B=c["B"], C=c["C"], H=c["H"], W=c["W"], Cout=c["Cout"], k=c["k"],
                         stride=c["s"], pad=c["p"], dil=c["d"], groups=c["G"], seed=97,
                         offset_dist=f"normal:{c['osc']}", backward=True)
    t = make_inputs(w, dtype=dtype)
    if c["WG"] > 1:
        t["weight"] = t["weight"][:, : c["C"] // c["WG"]].contiguous()
    if not c["mask"]:
        t["mask"] = None
    if not c["bias"]:
        t["bias"] = None
    geo = w.geometry()
    args = (c["s"], c["s"], c["p"], c["p"], c["d"], c["d"], c["G"])
    dev = [None if t[k] is None else t[k].to(DEV) for k in IN5]
    if c["in_cl"]:
        dev[0] = dev[0].to(memory_format=torch.channels_last)
    go = t["grad_output"].to(DEV)
    if c["go_cl"]:
        go = go.to(memory_format=torch.channels_last)
    with _C.option("bwd_fused", c["fused"]), _C.option("gi_push", c["push"]):
        out = _C.dcn_v2_forward(*dev, *args)
        grads = _C.dcn_v2_backward(*dev, go, *args)
        torch.cuda.synchronize()
    tol = TOL[dtype]
    check("output", out, oracle.dcn_forward(*(t[k] for k in IN5), pos_f32=True, **geo), tol)
    ref = oracle.dcn_backward(*(t[k] for k in IN5), t["grad_output"], pos_f32=True, **geo)
    for name, g, r in zip(GRADS, grads, ref):
        if g is None:
            assert r is None or name in ("grad_mask", "grad_bias")
            continue
        check(name, g, r, tol)


@pytest.mark.parametrize("c", CASES[:48], ids=[_id(c) for c in CASES[:48]])
def test_random_geometry_om_vs_oracle(c):
    """The offset/mask entry points (the predictor's [B, 3*G*kh*kw, Ho, Wo]
    output read directly, mask logits through the sigmoid) on the same random
    geometries: output, grad_input, both parts of grad_om, grad_weight and
    grad_bias against the oracle."""
    print(_id(c), flush=True)
    dtype = DT[c["dt"]]
    w = CONFIGS[0].with_(B=c["B"], C=c["C"], H=c["H"], W=c["W"], Cout=c["Cout"], k=c["k"],
                         stride=c["s"], pad=c["p"], dil=c["d"], groups=c["G"], seed=101,
                         offset_dist=f"normal:{c['osc']}", backward=True)
    t = make_inputs(w, dtype=dtype)
    if c["WG"] > 1:
        t["weight"] = t["weight"][:, : c["C"] // c["WG"]].contiguous()
    if not c["bias"]:
        t["bias"] = None
    n_off = t["offset"].shape[1]
    g = torch.Generator().manual_seed(103)
    logits = (torch.randn(t["mask"].shape, generator=g) * 1.5).to(dtype)
    om = torch.cat([t["offset"], logits], dim=1)
    geo = w.geometry()
    args = (c["s"], c["s"], c["p"], c["p"], c["d"], c["d"], c["G"])
    x = t["input"].to(DEV)
    if c["in_cl"]:
        x = x.to(memory_format=torch.channels_last)
    wt, omd = t["weight"].to(DEV), om.to(DEV)
    b = None if t["bias"] is None else t["bias"].to(DEV)
    go = t["grad_output"].to(DEV)
    if c["go_cl"]:
        go = go.to(memory_format=torch.channels_last)
    with _C.option("bwd_fused", c["fused"]), _C.option("gi_push", c["push"]):
        y = _C.dcn_v2_forward_om(x, wt, omd, b, *args)
        gi, gom, gw, gb = _C.dcn_v2_backward_om(x, wt, omd, b, go, *args)
        torch.cuda.synchronize()
    tol = TOL[dtype]
    o64 = om.double()
    offset, mask = o64[:, :n_off], torch.sigmoid(o64[:, n_off:])
    x64 = {k: None if t[k] is None else t[k].double() for k in ("input", "weight", "bias", "grad_output")}
    check("output", y, oracle.dcn_forward(x64["input"], x64["weight"], mask, offset, x64["bias"],
                                          pos_f32=True, **geo), tol)
    r_gi, r_goff, r_gmask, r_gw, r_gb = oracle.dcn_backward(
        x64["input"], x64["weight"], mask, offset, x64["bias"], x64["grad_output"], pos_f32=True, **geo)
    m = mask.numpy()
    check("grad_input", gi, r_gi, tol)
    check("grad_om[offsets]", gom[:, :n_off], r_goff, tol)
    check("grad_om[logits]", gom[:, n_off:], r_gmask * m * (1.0 - m), tol)
    check("grad_weight", gw, r_gw, tol)
    if gb is not None:
        check("grad_bias", gb, r_gb, tol)
