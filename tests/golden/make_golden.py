"""Writes the golden fixtures ``tests/golden/*.npz``.

The reference ships no golden vectors (its only numeric check, ``test.py``,
compares against the un-vendored lbin/DCNv2), and torchvision, the semantic
comparator named for this path, is not installed here.  The expected values are
therefore produced by ``tests/independent.py``: ``F.grid_sample`` sampling,
matmul contraction and torch autograd in float64 -- a formulation that shares no
code with the C oracle, so the fixtures pin the oracle as well as the HIP path.

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
from independent import forward_backward_gs  # noqa: E402

# name: (B, C, H, W, Cout, kh, kw, stride, pad, dilation, groups, offset_scale)
CASES = {
    "g0_basic": (1, 4, 8, 8, 4, 3, 3, 1, 1, 1, 1, 2.0),
    "g1_dil2_dg2": (1, 4, 8, 8, 4, 3, 3, 1, 2, 2, 2, 2.0),
    "g2_s2_dg3": (2, 6, 7, 9, 3, 3, 3, 2, 1, 1, 3, 1.5),
    "g3_1x1": (2, 5, 6, 6, 3, 1, 1, 1, 0, 1, 1, 1.0),
    "g4_5x3_far": (1, 3, 6, 7, 2, 5, 3, 1, 2, 1, 1, 6.0),
}


def make(name, spec, seed):
    B, C, H, W, Co, kh, kw, s, p, d, G, osc = spec
    g = torch.Generator().manual_seed(seed)
    Ho = (H + 2 * p - (d * (kh - 1) + 1)) // s + 1
    Wo = (W + 2 * p - (d * (kw - 1) + 1)) // s + 1
    f64 = torch.float64
    x = torch.randn(B, C, H, W, generator=g, dtype=f64)
    w = torch.randn(Co, C, kh, kw, generator=g, dtype=f64) * 0.5
    off = torch.randn(B, 2 * G * kh * kw, Ho, Wo, generator=g, dtype=f64) * osc
    m = torch.rand(B, G * kh * kw, Ho, Wo, generator=g, dtype=f64)
    b = torch.randn(Co, generator=g, dtype=f64) * 0.1
    go = torch.randn(B, Co, Ho, Wo, generator=g, dtype=f64)
    out, gi, goff, gm, gw, gb = forward_backward_gs(
        x, w, off, m, b, go, stride=s, padding=p, dilation=d, deformable_groups=G)
    arrays = dict(input=x, weight=w, offset=off, mask=m, bias=b, grad_output=go, output=out,
                  grad_input=gi, grad_offset=goff, grad_mask=gm, grad_weight=gw, grad_bias=gb)
    np.savez_compressed(
        os.path.join(HERE, name + ".npz"),
        geometry=np.array([s, p, d, G], dtype=np.int64),
        **{k: v.numpy() for k, v in arrays.items()})


def main():
    for i, (name, spec) in enumerate(CASES.items()):
        make(name, spec, seed=1000 + i)
        print("wrote", name)


if __name__ == "__main__":
    main()
