"""The benchmark workloads of this path: the five configurations of
BASELINE.json, with seeded synthetic inputs.

Inputs are drawn on the CPU from ``torch.Generator(seed)`` in float32, in the
fixed order input, offset, mask, weight, bias, grad_output, and only then cast
to the workload dtype, so the GPU run and the CPU oracle see identical values.
Distributions follow the configuration text; where it is silent the input is
N(0,1), the weight Kaiming-normal (fan_in), the bias N(0, 0.1) and grad_output
N(0,1).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, replace

import torch


@dataclass(frozen=True)
class Workload:
    name: str
    B: int
    C: int
    H: int
    W: int
    Cout: int
    k: int
    stride: int
    pad: int
    dil: int
    groups: int
    dtype: torch.dtype
    offset_dist: str      # "normal:<std>" or "uniform:<half-width>"
    mask_dist: str        # "sigmoid_normal" or "uniform"
    weight_dist: str      # "normal:<std>" or "kaiming"
    backward: bool
    seed: int

    @property
    def Ho(self):
        return (self.H + 2 * self.pad - (self.dil * (self.k - 1) + 1)) // self.stride + 1

    @property
    def Wo(self):
        return (self.W + 2 * self.pad - (self.dil * (self.k - 1) + 1)) // self.stride + 1

    def gemm_flops(self) -> float:
        """Real forward GEMM FLOPs: 2*B*Cout*Ho*Wo*C*kh*kw."""
        return 2.0 * self.B * self.Cout * self.Ho * self.Wo * self.C * self.k * self.k

    def readme_flops(self) -> float:
        """The reference README formula (README.md:17-19):
        B*Hout*Wout*Cout*(10*kh*kw*C + 2*kh*kw)."""
        kk = self.k * self.k
        return float(self.B * self.Ho * self.Wo * self.Cout * (10 * kk * self.C + 2 * kk))

    def with_(self, **kw) -> "Workload":
        return replace(self, **kw)

    def geometry(self):
        return dict(stride=self.stride, padding=self.pad, dilation=self.dil,
                    deformable_groups=self.groups)


# BASELINE.json "configs", in order.
CONFIGS = [
    Workload("c0_cpu_plumbing", 1, 16, 32, 32, 32, 3, 1, 1, 1, 1, torch.float32,
             "normal:1", "sigmoid_normal", "normal:0.1", False, 0),
    Workload("c1_readme_fwd", 8, 64, 128, 128, 256, 3, 1, 1, 1, 1, torch.float16,
             "normal:2", "sigmoid_normal", "kaiming", False, 1),
    Workload("c2_readme_fwd_bwd", 8, 64, 128, 128, 256, 3, 1, 1, 1, 1, torch.float16,
             "normal:2", "sigmoid_normal", "kaiming", True, 2),
    Workload("c3_neck_bf16_dg4", 16, 256, 64, 64, 256, 3, 1, 1, 1, 4, torch.bfloat16,
             "normal:1.5", "sigmoid_normal", "kaiming", True, 3),
    Workload("c4_stress_s2_d2", 2, 128, 256, 256, 128, 3, 2, 2, 2, 1, torch.float16,
             "uniform:16", "uniform", "kaiming", True, 4),
]
BY_NAME = {w.name: w for w in CONFIGS}


def _draw(dist: str, shape, gen, fan_in=None):
    kind, _, arg = dist.partition(":")
    if kind == "normal":
        return torch.randn(shape, generator=gen) * float(arg)
    if kind == "uniform":
        return (torch.rand(shape, generator=gen) * 2 - 1) * float(arg)
    if kind == "kaiming":
        return torch.randn(shape, generator=gen) * math.sqrt(2.0 / fan_in)
    if kind == "sigmoid_normal":
        return torch.sigmoid(torch.randn(shape, generator=gen))
    if kind == "unit_uniform":
        return torch.rand(shape, generator=gen)
    raise ValueError(dist)


def make_inputs(w: Workload, device="cpu", dtype=None, with_grad=None):
    """Returns dict(input, offset, mask, weight, bias[, grad_output]) in
    ``dtype`` (default: the workload dtype) on ``device``."""
    g = torch.Generator().manual_seed(w.seed)
    kk = w.k * w.k
    t = {}
    t["input"] = torch.randn(w.B, w.C, w.H, w.W, generator=g)
    t["offset"] = _draw(w.offset_dist, (w.B, 2 * w.groups * kk, w.Ho, w.Wo), g)
    t["mask"] = _draw("unit_uniform" if w.mask_dist == "uniform" else w.mask_dist,
                      (w.B, w.groups * kk, w.Ho, w.Wo), g)
    t["weight"] = _draw(w.weight_dist, (w.Cout, w.C, w.k, w.k), g, fan_in=w.C * kk)
    t["bias"] = torch.randn(w.Cout, generator=g) * 0.1
    if w.backward if with_grad is None else with_grad:
        t["grad_output"] = torch.randn(w.B, w.Cout, w.Ho, w.Wo, generator=g)
    dt = dtype or w.dtype
    return {k: v.to(dtype=dt).to(device) for k, v in t.items()}
