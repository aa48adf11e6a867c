"""A second, independently formulated DCNv2 used to pin the C oracle.

It shares no code or loop structure with ``oracle/dcn_oracle.c``: sampling is
``torch.nn.functional.grid_sample(mode="bilinear", padding_mode="zeros",
align_corners=True)`` (a library routine whose zero-padded bilinear rule is the
same as the reference's ``dcn_bilinear_cuda``, ``com.cu:119-148``), the
contraction is a matmul, and every gradient comes from torch autograd.  At
samples exactly on an integer coordinate the one-sided floor derivative of
grid_sample equals torchvision's ``get_coordinate_weight``; the normalisation
round trip can move such points by one ulp, so comparisons against this module
use continuous random offsets, except on images whose H - 1 and W - 1 are
powers of two, where the round trip is exact.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def _pair(v):
    return (int(v[0]), int(v[1])) if isinstance(v, (tuple, list)) else (int(v), int(v))


def deform_conv2d_gs(input, weight, offset, mask, bias, stride=1, padding=0, dilation=1,
                     deformable_groups=1):
    """Modulated deformable conv by grid_sample, differentiable in all inputs.
    A weight of shape [Cout, C/WG, kh, kw] gives WG weight groups, contracted
    group by group (torchvision's deform_conv2d semantics)."""
    B, C, H, W = input.shape
    Cout, Cw, kh, kw = weight.shape
    WG = C // Cw
    sh, sw = _pair(stride)
    ph, pw = _pair(padding)
    dh, dw = _pair(dilation)
    G = deformable_groups
    Cg = C // G
    KK = kh * kw
    Ho = (H + 2 * ph - (dh * (kh - 1) + 1)) // sh + 1
    Wo = (W + 2 * pw - (dw * (kw - 1) + 1)) // sw + 1
    dt, dev = input.dtype, input.device
    oy = torch.arange(Ho, dtype=dt, device=dev) * sh - ph
    ox = torch.arange(Wo, dtype=dt, device=dev) * sw - pw
    ki = torch.arange(kh, dtype=dt, device=dev).repeat_interleave(kw) * dh  # [KK]
    kj = torch.arange(kw, dtype=dt, device=dev).repeat(kh) * dw
    base_y = ki[:, None, None] + oy[None, :, None]  # [KK, Ho, 1]
    base_x = kj[:, None, None] + ox[None, None, :]  # [KK, 1, Wo]
    off = offset.view(B, G, KK, 2, Ho, Wo)
    y = base_y + off[:, :, :, 0]  # [B, G, KK, Ho, Wo]
    x = base_x + off[:, :, :, 1]
    gy = 2 * y / (H - 1) - 1
    gx = 2 * x / (W - 1) - 1
    cols = []
    for g in range(G):
        grid = torch.stack((gx[:, g], gy[:, g]), dim=-1).reshape(B, KK * Ho, Wo, 2)
        s = F.grid_sample(input[:, g * Cg:(g + 1) * Cg], grid, mode="bilinear",
                          padding_mode="zeros", align_corners=True)  # [B, Cg, KK*Ho, Wo]
        s = s.view(B, Cg, KK, Ho, Wo)
        if mask is not None:
            s = s * mask.view(B, G, KK, Ho, Wo)[:, g].unsqueeze(1)
        cols.append(s)
    cols = torch.cat(cols, dim=1).reshape(B, WG, Cw * KK, Ho * Wo)
    out = torch.matmul(weight.reshape(WG, Cout // WG, Cw * KK), cols).view(B, Cout, Ho, Wo)
    if bias is not None:
        out = out + bias.view(1, Cout, 1, 1)
    return out


def forward_backward_gs(input, weight, offset, mask, bias, grad_out, dtype=torch.float64,
                        **geo):
    """Returns out, grad_input, grad_offset, grad_mask, grad_weight, grad_bias
    computed in ``dtype`` on the device of ``input``."""
    ts = [t.detach().to(dtype).clone().requires_grad_(True) for t in
          (input, weight, offset, mask, bias)]
    out = deform_conv2d_gs(ts[0], ts[1], ts[2], ts[3], ts[4], **geo)
    out.backward(grad_out.to(dtype))
    gi, gw, goff, gm, gb = (t.grad for t in ts)
    return out.detach(), gi, goff, gm, gw, gb


def sample_positions(offset, kh, kw, Ho, Wo, stride=1, padding=0, dilation=1,
                     deformable_groups=1):
    """Exact sample coordinates y, x of every (b, g, tap, oy, ox), float64."""
    sh, sw = _pair(stride)
    ph, pw = _pair(padding)
    dh, dw = _pair(dilation)
    B = offset.shape[0]
    off = offset.detach().double().cpu().view(B, deformable_groups, kh * kw, 2, Ho, Wo)
    oy = torch.arange(Ho, dtype=torch.float64) * sh - ph
    ox = torch.arange(Wo, dtype=torch.float64) * sw - pw
    ki = torch.arange(kh, dtype=torch.float64).repeat_interleave(kw) * dh
    kj = torch.arange(kw, dtype=torch.float64).repeat(kh) * dw
    y = ki[:, None, None] + oy[None, :, None] + off[:, :, :, 0]
    x = kj[:, None, None] + ox[None, None, :] + off[:, :, :, 1]
    return y, x
