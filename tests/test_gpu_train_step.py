"""GPU regressions for the reference's own callers of the operator.

* ``test.py``'s scenario (``DCN(64, 256, 7x7, stride 2, pad 3)`` on an all-ones
  batch with all-ones weights, zero-initialised predictor): every output equals
  0.5 (the mask sigmoid(0)) x 64 channels x the number of kernel taps inside the
  image, 1568 in the interior -- an exact known answer in fp32;
* the 1x1 deformable convolutions ``train.py``'s network is built from (up to
  Cout 2048, which runs the forward kernel past the warp-specialised tile and
  the backward with several M chunks) against the CPU oracle;
* one whole training step (forward, backward, Adam) of ``train.py``'s network,
  reduced in depth and image size, against the same network whose deformable
  convolutions are the independent grid_sample formulation (fp64 reference,
  with the grid_sample network's own fp32 error as the yardstick).
"""
from __future__ import annotations

import copy

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.optim as optim

from dcnv2_amd import _C
from dcnv2_amd.dcn_v2_mm import DCN
from independent import deform_conv2d_gs
from oracle import oracle
from train import build_net, synthetic_batch, train_step
from util import TOL, check

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.mark.parametrize("fused", [True, False], ids=["fused_om", "separate"])
def test_reference_test_py_known_answer(fused):
    torch.manual_seed(0)
    dcn = DCN(64, 256, kernel_size=(7, 7), stride=2, padding=3, deformable_groups=1,
              fused_offset_mask=fused).to(DEV)
    nn.init.constant_(dcn.weight, 1.0)
    x = torch.ones((8, 64, 128, 128), dtype=torch.float32, device=DEV)
    with torch.no_grad():
        y = dcn(x)
    # taps inside the image along one axis: positions o*2 - 3 + i, i = 0..6
    o = np.arange(64)[:, None] * 2 - 3 + np.arange(7)[None, :]
    inside = ((o >= 0) & (o < 128)).sum(1)
    want = 0.5 * 64 * inside[:, None] * inside[None, :]
    assert want[10, 10] == 1568.0
    got = y.cpu().numpy()
    assert np.array_equal(got, np.broadcast_to(want, got.shape)), \
        f"max |diff| {np.abs(got - want).max()}"


POINTWISE = {
    "c256_to_512_14x14": (2, 256, 14, 14, 512),
    "c128_to_2048_7x7": (2, 128, 7, 7, 2048),
    "c64_to_64_28x28": (1, 64, 28, 28, 64),
}


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["float32", "float16"])
@pytest.mark.parametrize("case", list(POINTWISE), ids=list(POINTWISE))
def test_pointwise_dcn_vs_oracle(case, dtype):
    B, C, H, W, Cout = POINTWISE[case]
    g = torch.Generator().manual_seed(7)
    t = dict(input=torch.randn(B, C, H, W, generator=g),
             weight=torch.randn(Cout, C, 1, 1, generator=g) * (2.0 / C) ** 0.5,
             mask=torch.sigmoid(torch.randn(B, 1, H, W, generator=g)),
             offset=torch.randn(B, 2, H, W, generator=g) * 1.5,
             bias=torch.randn(Cout, generator=g) * 0.1,
             grad_output=torch.randn(B, Cout, H, W, generator=g))
    t = {k: v.to(dtype) for k, v in t.items()}
    names = ("input", "weight", "mask", "offset", "bias")
    dev = [t[k].to(DEV) for k in names]
    geo = dict(stride=1, padding=0, dilation=1, deformable_groups=1)
    y = _C.dcn_v2_forward(*dev, 1, 1, 0, 0)
    grads = _C.dcn_v2_backward(*dev, t["grad_output"].to(DEV), 1, 1, 0, 0)
    torch.cuda.synchronize()
    ref64 = [t[k].double() for k in names]
    check("output", y, oracle.dcn_forward(*ref64, pos_f32=True, **geo), TOL[dtype])
    rg = oracle.dcn_backward(*ref64, t["grad_output"].double(), pos_f32=True, **geo)
    for n, a, r in zip(("grad_input", "grad_offset", "grad_mask", "grad_weight", "grad_bias"),
                       grads, rg):
        check(n, a, r, TOL[dtype])


class GridSampleDCN(DCN):
    """The reference's DCN module with the independent grid_sample formulation
    as the operator (chunk / cat / sigmoid as in dcn_v2_mm.py:133-137)."""

    def forward(self, input):
        out = self.conv_offset_mask(input)
        o1, o2, m = torch.chunk(out, 3, dim=1)
        return deform_conv2d_gs(input, self.weight, torch.cat((o1, o2), 1), torch.sigmoid(m),
                                self.bias, self.stride, self.padding, self.dilation,
                                self.deformable_groups)


def test_train_step_matches_gridsample_network():
    """One Adam step of train.py's network (depths (1, 1, 1, 1), 96x96 images,
    batch 8) with non-zero offset/mask predictors.  Reference: the same network
    with the grid_sample operator in fp64.  Per parameter, the max-abs error of
    our fp32 gradient must be at most 3x that of the grid_sample network's own
    fp32 run plus 1e-3 of the network's largest gradient.  A plumbing mistake
    (a swapped gradient, a missing sigmoid derivative) is an O(1) error and
    fails by orders of magnitude; fp32 rounding stays below the bound (the
    worst parameter measured sits at 0.66 of it, in every run).  Errors are absolute
    with a network-wide scale because some gradients are ~0 by construction
    (conv biases feeding BatchNorm) or near-cancelling sums, where a
    per-parameter relative error measures nothing; and the yardstick is the
    independent fp32 run because a dozen layers of backward and small-batch
    BatchNorm amplify fp32 rounding past the per-op 1e-4.

    The networks' ordinary convolutions (the stem, the 3x3 convs and the
    offset/mask predictors) run on torch's native kernels, not MIOpen: MIOpen
    picks its convolution algorithm per run, and in about one run in four it
    picked one whose rounding alone moved an offset predictor's gradient from
    0.6x to 1.1x of the bound (measured with this library unchanged)."""
    prev = torch.backends.cudnn.enabled
    torch.backends.cudnn.enabled = False
    try:
        _train_step_vs_gridsample()
    finally:
        torch.backends.cudnn.enabled = prev


def _train_step_vs_gridsample():
    torch.manual_seed(0)
    net = build_net((1, 1, 1, 1)).to(DEV)
    for m in net.modules():
        if isinstance(m, DCN):
            with torch.no_grad():
                m.conv_offset_mask.weight.normal_(0.0, 0.02)
                m.conv_offset_mask.bias.normal_(0.0, 0.5)
    gs32 = build_net((1, 1, 1, 1), dcn=GridSampleDCN).to(DEV)
    gs32.load_state_dict(copy.deepcopy(net.state_dict()))
    gs64 = copy.deepcopy(gs32).double()
    x, y = synthetic_batch(8, 96, device=DEV)
    crit = nn.CrossEntropyLoss()
    losses = []
    for n, xx in ((net, x), (gs32, x), (gs64, x.double())):
        opt = optim.Adam(n.parameters(), betas=(0.9, 0.999), eps=1e-8, lr=1e-4)
        losses.append(float(train_step(n, opt, crit, xx, y)))
    print(f"  loss: ours {losses[0]:.8f}, grid_sample fp32 {losses[1]:.8f}, fp64 {losses[2]:.8f}")
    assert abs(losses[0] - losses[2]) <= 3 * abs(losses[1] - losses[2]) + 1e-6 * abs(losses[2])

    params = list(zip(net.named_parameters(), gs32.named_parameters(), gs64.named_parameters()))
    scale = max(float(c.grad.abs().max()) for _, _, (_, c) in params)
    n_pred = 0
    for (name, a), (_, b), (_, c) in params:
        ref = c.grad.double()
        e_ours = float((a.grad.double() - ref).abs().max())
        e_gs = float((b.grad.double() - ref).abs().max())
        bound = 3.0 * e_gs + 1e-3 * scale
        print(f"  grad {name}: ours {e_ours:.2e}, grid_sample fp32 {e_gs:.2e} "
              f"(bound {bound:.1e}, scale {scale:.1e})")
        assert e_ours <= bound, f"grad {name}: {e_ours:.3e} > {bound:.3e}"
        n_pred += name.endswith("conv_offset_mask.weight")
    assert n_pred == sum(isinstance(m, DCN) for m in net.modules()) > 0
