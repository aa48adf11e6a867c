"""Python operator surface, drop-in for the reference's ``dcn_v2_mm.py``.

Same names, positional order and return order as the reference:

* ``_DCNv2`` autograd Function, ``forward(ctx, input, weight, mask, offset,
  bias, stride, padding)`` and a ``once_differentiable`` backward returning
  ``(grad_input, grad_weight, grad_mask, grad_offset, grad_bias, None, ...)``
  (reference ``dcn_v2_mm.py:15-53``);
* ``dcn_v2_conv = _DCNv2.apply`` (``:56``);
* ``DCNv2(in_channels, out_channels, kernel_size, stride, padding, dilation=1,
  deformable_groups=1)`` with ``forward(input, offset, mask)`` (``:59-102``);
* ``DCN(...)``, which predicts offset and mask with a zero-initialised conv and
  splits its output as ``o1, o2, mask = chunk(3)``, ``offset = cat(o1, o2)``,
  ``mask = sigmoid(mask)`` (``:105-146``).

Differences from the reference, by design:

* ``dilation`` and ``deformable_groups`` are forwarded to the operator (the
  reference accepts and drops them, ``:94-102``), appended as two optional
  trailing arguments of ``dcn_v2_conv``;
* ``DCN.forward`` hands the predictor's raw output to the operator
  (``dcn_v2_conv_om``): the kernels read the offsets from its first
  ``2*G*kh*kw`` channels and apply ``sigmoid`` to the rest while loading, and
  the backward returns the gradient of that tensor, so the ``chunk`` / ``cat`` /
  ``sigmoid`` passes (``:133-137``) and their backward are not materialised.
  ``DCN(..., fused_offset_mask=False)`` keeps the reference's separate steps;
* a trailing ``groups=1`` on ``DCNv2`` / ``DCN`` gives torchvision's weight
  groups (weight ``[Cout, C/groups, kh, kw]``); the operator infers them from
  the weight's shape, as ``torchvision.ops.deform_conv2d`` does.
"""
from __future__ import annotations

import math

import torch
from torch import nn
from torch.autograd import Function
from torch.autograd.function import once_differentiable
from torch.nn.modules.utils import _pair

from . import _C


class _DCNv2(Function):
    @staticmethod
    def forward(ctx, input, weight, mask, offset, bias, stride, padding, dilation=1,
                deformable_groups=1):
        ctx.stride = _pair(stride)
        ctx.padding = _pair(padding)
        ctx.dilation = _pair(dilation)
        ctx.deformable_groups = int(deformable_groups)
        output = _C.dcn_v2_forward(
            input, weight, mask, offset, bias,
            ctx.stride[0], ctx.stride[1], ctx.padding[0], ctx.padding[1],
            ctx.dilation[0], ctx.dilation[1], ctx.deformable_groups)
        ctx.save_for_backward(input, weight, mask, offset, bias)
        return output

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_output):
        input, weight, mask, offset, bias = ctx.saved_tensors
        grad_input, grad_offset, grad_mask, grad_weight, grad_bias = _C.dcn_v2_backward(
            input, weight, mask, offset, bias, grad_output,
            ctx.stride[0], ctx.stride[1], ctx.padding[0], ctx.padding[1],
            ctx.dilation[0], ctx.dilation[1], ctx.deformable_groups)
        return (grad_input, grad_weight, grad_mask, grad_offset, grad_bias,
                None, None, None, None)


dcn_v2_conv = _DCNv2.apply


def deform_conv2d(input, offset, weight, bias=None, stride=(1, 1), padding=(0, 0),
                  dilation=(1, 1), mask=None):
    """``torchvision.ops.deform_conv2d``'s signature on these kernels, the
    comparator the reference names: deformable groups follow from
    ``offset.shape[1] // (2*kh*kw)`` and weight groups from ``weight.shape[1]``,
    as torchvision infers them; ``mask=None`` is DCNv1.  Differentiable in
    input, offset, weight, bias and mask (through :func:`dcn_v2_conv`)."""
    kh, kw = int(weight.shape[-2]), int(weight.shape[-1])
    if offset.dim() != 4 or offset.shape[1] % (2 * kh * kw) or offset.shape[1] == 0:
        raise RuntimeError(f"deform_conv2d: offset channels {tuple(offset.shape)[1:2]} are not a "
                           f"positive multiple of 2*kh*kw = {2 * kh * kw}")
    dg = offset.shape[1] // (2 * kh * kw)
    if mask is not None and (mask.dim() != 4 or mask.shape[1] != dg * kh * kw):
        raise RuntimeError(f"deform_conv2d: mask has {mask.shape[1]} channels, "
                           f"offset implies {dg * kh * kw}")
    return dcn_v2_conv(input, weight, mask, offset, bias, stride, padding, dilation, dg)


class _DCNv2OM(Function):
    """``dcn_v2_conv`` on the offset-and-mask predictor's raw output ``om``
    ``[B, 3*G*kh*kw, Ho, Wo]``: equal to ``dcn_v2_conv(input, weight,
    sigmoid(m), cat(o1, o2), bias, ...)`` with ``o1, o2, m = om.chunk(3, 1)``."""

    @staticmethod
    def forward(ctx, input, weight, om, bias, stride, padding, dilation=1, deformable_groups=1):
        ctx.stride = _pair(stride)
        ctx.padding = _pair(padding)
        ctx.dilation = _pair(dilation)
        ctx.deformable_groups = int(deformable_groups)
        output = _C.dcn_v2_forward_om(
            input, weight, om, bias,
            ctx.stride[0], ctx.stride[1], ctx.padding[0], ctx.padding[1],
            ctx.dilation[0], ctx.dilation[1], ctx.deformable_groups)
        ctx.save_for_backward(input, weight, om, bias)
        return output

    @staticmethod
    @once_differentiable
    def backward(ctx, grad_output):
        input, weight, om, bias = ctx.saved_tensors
        grad_input, grad_om, grad_weight, grad_bias = _C.dcn_v2_backward_om(
            input, weight, om, bias, grad_output,
            ctx.stride[0], ctx.stride[1], ctx.padding[0], ctx.padding[1],
            ctx.dilation[0], ctx.dilation[1], ctx.deformable_groups)
        return grad_input, grad_weight, grad_om, grad_bias, None, None, None, None


dcn_v2_conv_om = _DCNv2OM.apply


class DCNv2(nn.Module):
    def __init__(self, in_channels, out_channels, kernel_size, stride, padding, dilation=1,
                 deformable_groups=1, groups=1):
        super().__init__()
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.kernel_size = _pair(kernel_size)
        self.stride = _pair(stride)
        self.padding = _pair(padding)
        self.dilation = _pair(dilation)
        self.deformable_groups = deformable_groups
        # groups: torchvision's weight groups (DeformConv2d(groups=...)); the
        # reference's module has none, and groups=1 is its behaviour
        self.groups = groups
        if in_channels % deformable_groups != 0:
            raise ValueError("in_channels must be divisible by deformable_groups")
        if in_channels % groups != 0 or out_channels % groups != 0:
            raise ValueError("in_channels and out_channels must be divisible by groups")
        self.weight = nn.Parameter(torch.Tensor(out_channels, in_channels // groups,
                                                *self.kernel_size))
        self.bias = nn.Parameter(torch.Tensor(out_channels))
        self.reset_parameters()

    def reset_parameters(self):
        # reference dcn_v2_mm.py:83-89: U(+-1/sqrt(fan_in)), zero bias
        n = self.in_channels // self.groups
        for k in self.kernel_size:
            n *= k
        stdv = 1.0 / math.sqrt(n)
        self.weight.data.uniform_(-stdv, stdv)
        self.bias.data.zero_()

    def forward(self, input, offset, mask):
        kk = self.kernel_size[0] * self.kernel_size[1]
        assert 2 * self.deformable_groups * kk == offset.shape[1]
        assert self.deformable_groups * kk == mask.shape[1]
        return dcn_v2_conv(input, self.weight, mask, offset, self.bias, self.stride,
                           self.padding, self.dilation, self.deformable_groups)


class DCN(DCNv2):
    def __init__(self, in_channels, out_channels, kernel_size, stride=1, padding=0,
                 dilation=1, deformable_groups=1, fused_offset_mask=True, groups=1):
        super().__init__(in_channels, out_channels, kernel_size, stride, padding, dilation,
                         deformable_groups, groups)
        self.fused_offset_mask = fused_offset_mask
        channels_ = self.deformable_groups * 3 * self.kernel_size[0] * self.kernel_size[1]
        # The offset/mask predictor sees the same sampling grid as the DCN
        # (stride, padding and dilation), so its output matches Ho x Wo.
        self.conv_offset_mask = nn.Conv2d(
            self.in_channels, channels_, kernel_size=self.kernel_size, stride=self.stride,
            padding=self.padding, dilation=self.dilation, bias=True)
        self.init_offset()

    def init_offset(self):
        self.conv_offset_mask.weight.data.zero_()
        self.conv_offset_mask.bias.data.zero_()

    def forward(self, input):
        out = self.conv_offset_mask(input)
        if self.fused_offset_mask:
            return dcn_v2_conv_om(input, self.weight, out, self.bias, self.stride, self.padding,
                                  self.dilation, self.deformable_groups)
        o1, o2, mask = torch.chunk(out, 3, dim=1)
        offset = torch.cat((o1, o2), dim=1)
        mask = torch.sigmoid(mask)
        return dcn_v2_conv(input, self.weight, mask, offset, self.bias, self.stride,
                           self.padding, self.dilation, self.deformable_groups)
