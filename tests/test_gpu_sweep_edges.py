"""Seeded sweep over extreme layer geometries: the forward and all five
gradients against the fp64 oracle, in the three dtypes.

Where `test_gpu_sweep.py` draws ordinary layers, this one draws the corners of
the geometry space: images of 1 to 33 pixels a side, kernels of 1 to 7 taps a
side (square or not, larger than the image included), stride, padding and
dilation of 1 to 3 chosen separately per axis, one to a few channels per
group, odd channel counts, 1 to 257 output channels, and offset fields that are
all zero, whole integers (every sample exactly on a pixel, the measure-zero
tie points of the bilinear weights), half-integers, ordinary, or hundreds of
pixels out (every sample outside the image).  The list is fixed by the seed.
"""
from __future__ import annotations

import random

import pytest
import torch

from dcnv2_amd import _C
from oracle import oracle
from util import GRADS, TOL, check

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
OFFSETS = ("zero", "int", "half", "normal", "far")


def _out(n, k, s, p, d):
    return (n + 2 * p - (d * (k - 1) + 1)) // s + 1


def _draw(rng):
    G = rng.choice([1, 1, 2, 3])
    Cg = rng.choice([1, 2, 3, 5, 8, 17, 64, 65])
    C = G * Cg
    Cout = rng.choice([1, 2, 3, 7, 33, 129, 257])
    WG = rng.choice([d for d in (1, 1, 2, 3) if C % d == 0 and Cout % d == 0])
    kh, kw = rng.choice([1, 2, 3, 5, 7]), rng.choice([1, 2, 3, 5, 7])
    sh, sw = rng.choice([1, 1, 2, 3]), rng.choice([1, 1, 2, 3])
    dh, dw = rng.choice([1, 1, 2, 3]), rng.choice([1, 1, 2, 3])
    ph, pw = rng.choice([0, 1, 2, 3]), rng.choice([0, 1, 2, 3])
    H, W = rng.choice([1, 2, 3, 4, 7, 16, 17, 33]), rng.choice([1, 2, 3, 4, 7, 16, 17, 33])
    # the smallest padding that leaves one output pixel, when the drawn one does not
    while _out(H, kh, sh, ph, dh) < 1:
        ph += 1
    while _out(W, kw, sw, pw, dw) < 1:
        pw += 1
    return dict(dt=rng.choice(list(DT)), B=rng.choice([1, 2]), C=C, G=G, WG=WG, Cout=Cout, H=H, W=W,
                kh=kh, kw=kw, sh=sh, sw=sw, ph=ph, pw=pw, dh=dh, dw=dw, off=rng.choice(OFFSETS),
                mask=rng.random() < 0.8, bias=rng.random() < 0.8, seed=rng.randrange(1 << 30))


def _id(c):
    return (f"{c['dt']}_b{c['B']}c{c['C']}g{c['G']}w{c['WG']}o{c['Cout']}_{c['H']}x{c['W']}"
            f"_k{c['kh']}x{c['kw']}s{c['sh']}{c['sw']}p{c['ph']}{c['pw']}d{c['dh']}{c['dw']}_{c['off']}"
            f"{'' if c['mask'] else '_nomask'}{'' if c['bias'] else '_nobias'}")


def _inputs(c):
    g = torch.Generator().manual_seed(c["seed"])
    B, C, H, W, Cout, G = c["B"], c["C"], c["H"], c["W"], c["Cout"], c["G"]
    kh, kw = c["kh"], c["kw"]
    Ho, Wo = _out(H, kh, c["sh"], c["ph"], c["dh"]), _out(W, kw, c["sw"], c["pw"], c["dw"])
    shape = (B, 2 * G * kh * kw, Ho, Wo)
    kind = c["off"]
    if kind == "zero":
        off = torch.zeros(shape)
    elif kind == "int":
        off = torch.randint(-3, 4, shape, generator=g).float()
    elif kind == "half":
        off = torch.randint(-3, 3, shape, generator=g).float() + 0.5
    elif kind == "normal":
        off = torch.randn(shape, generator=g) * 2.0
    else:  # far outside the image, either side
        off = torch.where(torch.rand(shape, generator=g) < 0.5, -1.0, 1.0) * (300.0 + 50 * torch.rand(shape, generator=g))
    t = dict(input=torch.randn(B, C, H, W, generator=g),
             weight=torch.randn(Cout, C // c["WG"], kh, kw, generator=g) * (2.0 / (C * kh * kw)) ** 0.5,
             mask=torch.rand(B, G * kh * kw, Ho, Wo, generator=g) if c["mask"] else None,
             offset=off,
             bias=torch.randn(Cout, generator=g) * 0.1 if c["bias"] else None,
             grad_output=torch.randn(B, Cout, Ho, Wo, generator=g))
    dtype = DT[c["dt"]]
    return {k: None if v is None else v.to(dtype) for k, v in t.items()}


CASES = [_draw(r) for r in [random.Random(7)] for _ in range(90)]


@pytest.mark.parametrize("c", CASES, ids=[_id(c) for c in CASES])
def test_edge_geometry_vs_oracle(c):
    print(_id(c), flush=True)
    t = _inputs(c)
    keys = ("input", "weight", "mask", "offset", "bias")
    args = (c["sh"], c["sw"], c["ph"], c["pw"], c["dh"], c["dw"], c["G"])
    geo = dict(stride=(c["sh"], c["sw"]), padding=(c["ph"], c["pw"]), dilation=(c["dh"], c["dw"]),
               deformable_groups=c["G"])
    dev = [None if t[k] is None else t[k].to(DEV) for k in keys]
    out = _C.dcn_v2_forward(*dev, *args)
    grads = _C.dcn_v2_backward(*dev, t["grad_output"].to(DEV), *args)
    torch.cuda.synchronize()
    tol = TOL[DT[c["dt"]]]
    check("output", out, oracle.dcn_forward(*(t[k] for k in keys), pos_f32=True, **geo), tol)
    ref = oracle.dcn_backward(*(t[k] for k in keys), t["grad_output"], pos_f32=True, **geo)
    for name, gv, r in zip(GRADS, grads, ref):
        if gv is None:
            continue
        check(name, gv, r, tol)
