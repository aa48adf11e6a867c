"""Pins the CPU oracle (oracle/dcn_oracle.c) before it is trusted as the
checker of the HIP path.  CPU only.

The reference ships no golden vectors or unit tests (its one numeric check,
``test.py``, compares against the un-vendored lbin/DCNv2), so every check here
is either a vector of the independent grid_sample formulation
(tests/golden/*.npz, tests/independent.py) or a property the mathematics of
modulated deformable convolution fixes:

* zero offset, mask 1: exactly ``F.conv2d`` -- forward and the grad_input,
  grad_weight, grad_bias of conv2d autograd (catches transposed weights, wrong
  tap order, dilation or padding mistakes);
* integer offsets: conv2d of the shifted, zero-filled input;
* half-pixel offsets: the mean of two pixels; one-sided at the border;
* the reference ``test.py`` known answer (ones, 7x7 s2 p3, weight 1, mask 0.5:
  interior 1568);
* mask 0 and far-away samples: output = bias, zero gradients;
* linearity in the mask; groups with copied offsets equal one group;
* grad_offset and grad_mask against central finite differences of the
  oracle's own forward (catches sign and corner mistakes in the coordinate
  weight);
* the torchvision vs reference rule at a sample exactly on y == -1.
"""
from __future__ import annotations

import glob
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle
from util import GRADS, load_fixture, rel_err

FIXTURES = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))
IN5 = ("input", "weight", "mask", "offset", "bias")
f64 = torch.float64


def rand_case(B, C, H, W, Co, kh, kw, s=1, p=0, d=1, G=1, seed=0, osc=1.0):
    g = torch.Generator().manual_seed(seed)
    Ho = (H + 2 * p - (d * (kh - 1) + 1)) // s + 1
    Wo = (W + 2 * p - (d * (kw - 1) + 1)) // s + 1
    t = dict(
        input=torch.randn(B, C, H, W, generator=g, dtype=f64),
        weight=torch.randn(Co, C, kh, kw, generator=g, dtype=f64) * 0.5,
        offset=torch.randn(B, 2 * G * kh * kw, Ho, Wo, generator=g, dtype=f64) * osc,
        mask=torch.rand(B, G * kh * kw, Ho, Wo, generator=g, dtype=f64),
        bias=torch.randn(Co, generator=g, dtype=f64) * 0.1,
        grad_output=torch.randn(B, Co, Ho, Wo, generator=g, dtype=f64))
    geo = dict(stride=s, padding=p, dilation=d, deformable_groups=G)
    return t, geo


def fwd(t, geo, **kw):
    return oracle.dcn_forward(*(t[k] for k in IN5), **geo, **kw)


def bwd(t, geo, **kw):
    return oracle.dcn_backward(*(t[k] for k in IN5), t["grad_output"], **geo, **kw)


GEOMS = [
    # B, C, H, W, Co, kh, kw, s, p, d, G
    (1, 3, 7, 7, 2, 3, 3, 1, 1, 1, 1),
    (2, 4, 9, 8, 3, 3, 3, 2, 1, 1, 2),
    (1, 4, 10, 9, 2, 3, 3, 1, 2, 2, 4),
    (1, 2, 6, 7, 3, 5, 3, 1, 2, 1, 1),
    (2, 5, 5, 5, 4, 1, 1, 1, 0, 1, 1),
    (1, 2, 11, 12, 2, 3, 2, 3, 0, 2, 1),
]


# -- golden vectors of the independent formulation --------------------------------
@pytest.mark.parametrize("path", FIXTURES, ids=lambda p: os.path.basename(p)[:-4])
def test_golden_f64(path):
    t, geo = load_fixture(path)
    assert rel_err(fwd(t, geo), t["output"]) < 1e-12
    for name, got in zip(GRADS, bwd(t, geo)):
        assert rel_err(got, t[name]) < 1e-12, name


@pytest.mark.parametrize("path", FIXTURES, ids=lambda p: os.path.basename(p)[:-4])
def test_golden_f32_and_pos_f32(path):
    """The float32 build (the CPU baseline) and the float32 sample-position
    option stay within float32 rounding of the float64 answer."""
    t, geo = load_fixture(path)
    assert rel_err(fwd(t, geo, precision="f32"), t["output"]) < 1e-5
    assert rel_err(fwd(t, geo, pos_f32=True), t["output"]) < 1e-5
    for name, got in zip(GRADS, bwd(t, geo, precision="f32")):
        assert rel_err(got, t[name]) < 1e-4, name


# -- zero offset, mask 1 == conv2d ------------------------------------------------
@pytest.mark.parametrize("geom", GEOMS)
def test_zero_offset_is_conv2d(geom):
    B, C, H, W, Co, kh, kw, s, p, d, G = geom
    t, geo = rand_case(*geom, seed=1)
    t["offset"].zero_()
    t["mask"].fill_(1.0)
    x = t["input"].clone().requires_grad_(True)
    w = t["weight"].clone().requires_grad_(True)
    b = t["bias"].clone().requires_grad_(True)
    ref = F.conv2d(x, w, b, stride=s, padding=p, dilation=d)
    ref.backward(t["grad_output"])
    assert rel_err(fwd(t, geo), ref) < 1e-13
    gi, goff, gm, gw, gb = bwd(t, geo)
    assert rel_err(gi, x.grad) < 1e-13
    assert rel_err(gw, w.grad) < 1e-13
    assert rel_err(gb, b.grad) < 1e-13
    # with mask 1 the output is linear in the mask with coefficient = column
    # value, so grad_mask is the column-weighted grad_output; its sum over
    # everything equals <grad_output, output - bias>.
    out_nb = ref.detach() - b.detach().view(1, -1, 1, 1)
    assert abs(gm.sum() - float((t["grad_output"] * out_nb).sum())) < 1e-9 * (
        1 + float(np.abs(gm).sum()))


def shifted_conv(x, w, b, dy, dx, s, p, d):
    """conv2d whose every tap reads x[y + dy, x + dx] (zero outside the
    image): pad x by a margin, start the window dy, dx further, no padding."""
    P = p + 8
    Ho = (x.shape[-2] + 2 * p - (d * (w.shape[-2] - 1) + 1)) // s + 1
    Wo = (x.shape[-1] + 2 * p - (d * (w.shape[-1] - 1) + 1)) // s + 1
    xp = F.pad(x, (P, P, P, P))[..., P - p + dy:, P - p + dx:]
    return F.conv2d(xp, w, b, stride=s, dilation=d)[..., :Ho, :Wo]


@pytest.mark.parametrize("dy,dx", [(1, 0), (0, -2), (-1, 3), (2, 2), (-7, 0)])
@pytest.mark.parametrize("geom", [GEOMS[0], GEOMS[5]])
def test_integer_offset_is_shifted_conv(geom, dy, dx):
    B, C, H, W, Co, kh, kw, s, p, d, G = geom
    t, geo = rand_case(*geom, seed=2)
    t["offset"][:, 0::2] = float(dy)
    t["offset"][:, 1::2] = float(dx)
    t["mask"].fill_(1.0)
    ref = shifted_conv(t["input"], t["weight"], t["bias"], dy, dx, s, p, d)
    assert rel_err(fwd(t, geo), ref) < 1e-13


def test_half_pixel_is_mean_of_two_pixels():
    """1x1 kernel, identity weight, offset (+0.5, 0): the mean of rows y and
    y+1; on the last row only the in-image corner counts (half the pixel);
    offset (-0.5, 0) on row 0 likewise gives half of row 0."""
    C, H, W = 3, 5, 5
    x = torch.randn(1, C, H, W, generator=torch.Generator().manual_seed(3), dtype=f64)
    w = torch.eye(C, dtype=f64).view(C, C, 1, 1)
    for dy in (0.5, -0.5):
        off = torch.zeros(1, 2, H, W, dtype=f64)
        off[:, 0] = dy
        out = torch.from_numpy(oracle.dcn_forward(x, w, None, off, None))
        if dy > 0:
            want = torch.cat([(x[..., :-1, :] + x[..., 1:, :]) / 2, x[..., -1:, :] / 2], -2)
        else:
            want = torch.cat([x[..., :1, :] / 2, (x[..., :-1, :] + x[..., 1:, :]) / 2], -2)
        assert rel_err(out, want) < 1e-15


def test_reference_known_answer_1568():
    """Reference test.py: ones input, DCN(64, 256, 7x7, stride 2, pad 3) with
    weight 1 and the zero-initialised offset/mask conv (offset 0, mask
    sigmoid(0) = 0.5, bias 0): interior 0.5*64*49 = 1568, border 0.5*64 x the
    number of in-image taps.  Cout reduced to 4, H=W=24."""
    B, C, H, W, Co, k, s, p = 1, 64, 24, 24, 4, 7, 2, 3
    Ho = (H + 2 * p - k) // s + 1
    x = torch.ones(B, C, H, W, dtype=f64)
    w = torch.ones(Co, C, k, k, dtype=f64)
    off = torch.zeros(B, 2 * k * k, Ho, Ho, dtype=f64)
    m = torch.full((B, k * k, Ho, Ho), 0.5, dtype=f64)
    out = oracle.dcn_forward(x, w, m, off, torch.zeros(Co, dtype=f64), s, p)
    assert out[0, 0, 3, 3] == 1568.0
    taps_in = lambda o: sum(0 <= o * s - p + i < H for i in range(k))  # noqa: E731
    want = np.array([[0.5 * C * taps_in(oy) * taps_in(ox) for ox in range(Ho)]
                     for oy in range(Ho)])
    assert np.array_equal(out[0, 2], want)


# -- mask 0, far samples, linearity, groups ------------------------------------
def test_mask_zero_gives_bias_and_zero_grads():
    t, geo = rand_case(2, 4, 7, 7, 3, 3, 3, 1, 1, 1, 2, seed=4)
    t["mask"].zero_()
    out = fwd(t, geo)
    assert np.array_equal(out, np.broadcast_to(t["bias"].numpy().reshape(1, -1, 1, 1), out.shape))
    gi, goff, gm, gw, gb = bwd(t, geo)
    assert not gi.any() and not goff.any() and not gw.any()
    assert rel_err(gb, t["grad_output"].sum((0, 2, 3))) < 1e-14
    assert np.abs(gm).max() > 0  # the mask gradient is the sampled value, not 0


def test_far_samples_give_bias():
    t, geo = rand_case(1, 3, 6, 6, 2, 3, 3, 1, 1, 1, 1, seed=5)
    t["offset"][:, 0::2] = 1e4
    t["offset"][:, 1::2] = -3e7
    out = fwd(t, geo)
    assert np.array_equal(out, np.broadcast_to(t["bias"].numpy().reshape(1, -1, 1, 1), out.shape))
    gi, goff, gm, gw, gb = bwd(t, geo)
    assert not gi.any() and not goff.any() and not gm.any() and not gw.any()


def test_linear_in_mask():
    t, geo = rand_case(1, 4, 8, 8, 3, 3, 3, 2, 1, 1, 2, seed=6, osc=2.0)
    b = t["bias"].numpy().reshape(1, -1, 1, 1)
    m1, m2 = t["mask"].clone(), torch.rand(t["mask"].shape, dtype=f64,
                                           generator=torch.Generator().manual_seed(7))
    y1 = fwd(dict(t, mask=m1), geo) - b
    y2 = fwd(dict(t, mask=m2), geo) - b
    y12 = fwd(dict(t, mask=2.0 * m1 - 3.0 * m2), geo) - b
    assert rel_err(y12, 2.0 * y1 - 3.0 * y2) < 1e-13


def test_groups_with_copied_offsets_equal_one_group():
    G = 3
    t1, geo1 = rand_case(2, 6, 7, 8, 4, 3, 3, 1, 1, 1, 1, seed=8, osc=1.5)
    tG = dict(t1, offset=t1["offset"].repeat(1, G, 1, 1), mask=t1["mask"].repeat(1, G, 1, 1))
    geoG = dict(geo1, deformable_groups=G)
    assert rel_err(fwd(tG, geoG), fwd(t1, geo1)) < 1e-13
    g1, gG = bwd(t1, geo1), bwd(tG, geoG)
    assert rel_err(gG[0], g1[0]) < 1e-13  # grad_input
    assert rel_err(gG[3], g1[3]) < 1e-13  # grad_weight
    # per-group offset/mask gradients sum to the one-group gradient
    KK = 9
    goff = gG[1].reshape(2, G, 2 * KK, *gG[1].shape[2:]).sum(1)
    gm = gG[2].reshape(2, G, KK, *gG[2].shape[2:]).sum(1)
    assert rel_err(goff, g1[1]) < 1e-13
    assert rel_err(gm, g1[2]) < 1e-13


# -- finite differences ----------------------------------------------------------
@pytest.mark.parametrize("geom", [GEOMS[0], GEOMS[1], GEOMS[2], GEOMS[5]])
def test_gradients_match_finite_differences(geom):
    """Central differences of L = <grad_output, forward(...)> in float64 at 40
    random coordinates of every input; offsets are kept 0.05 away from integer
    sample coordinates so the bilinear function is smooth there."""
    t, geo = rand_case(*geom, seed=9, osc=1.3)
    off = t["offset"]
    frac = off - off.floor()
    off += torch.where(frac < 0.05, 0.05, 0.0) - torch.where(frac > 0.95, 0.05, 0.0)
    go = t["grad_output"].numpy()
    grads = dict(zip(GRADS, bwd(t, geo)))
    rng = np.random.default_rng(10)
    h = 1e-6
    for key, gname in (("input", "grad_input"), ("offset", "grad_offset"),
                       ("mask", "grad_mask"), ("weight", "grad_weight"),
                       ("bias", "grad_bias")):
        base = t[key]
        flat = base.view(-1)
        idx = rng.choice(flat.numel(), size=min(40, flat.numel()), replace=False)
        num = np.empty(len(idx))
        for j, i in enumerate(idx):
            keep = float(flat[i])
            flat[i] = keep + h
            lp = float((fwd(t, geo) * go).sum())
            flat[i] = keep - h
            lm = float((fwd(t, geo) * go).sum())
            flat[i] = keep
            num[j] = (lp - lm) / (2 * h)
        ana = grads[gname].reshape(-1)[idx]
        scale = max(1.0, float(np.abs(grads[gname]).max()))
        assert np.abs(ana - num).max() < 1e-6 * scale, gname


# -- the boundary rule at y == -1 ------------------------------------------------
def test_coordinate_weight_at_minus_one():
    """A sample exactly on y = -1: its value is 0 either way, but moving up by
    dy picks up row 0 with weight dy, so torchvision's rule (the default) gives
    the one-sided derivative = the row-0 value, while the reference's early
    exit (com.cu:392-396, ref_boundary=True) gives 0.  Likewise at x = -1."""
    C, H, W = 2, 4, 5
    x = torch.randn(1, C, H, W, generator=torch.Generator().manual_seed(11), dtype=f64)
    w = torch.eye(C, dtype=f64).view(C, C, 1, 1)
    go = torch.zeros(1, C, H, W, dtype=f64)
    go[0, :, 0, 2] = torch.tensor([1.0, -2.0], dtype=f64)
    for d in (0, 1):  # 0: y component, 1: x component
        off = torch.zeros(1, 2, H, W, dtype=f64)
        if d == 0:
            off[0, 0, 0, 2] = -1.0  # pixel (0, 2) samples (-1, 2)
            want = float((go[0, :, 0, 2] * x[0, :, 0, 2]).sum())
        else:
            off[0, 1, 0, 2] = -3.0  # pixel (0, 2) samples (0, -1)
            want = float((go[0, :, 0, 2] * x[0, :, 0, 0]).sum())
        _, goff_tv, _, _, _ = oracle.dcn_backward(x, w, None, off, None, go)
        _, goff_ref, _, _, _ = oracle.dcn_backward(x, w, None, off, None, go,
                                                   ref_boundary=True)
        assert abs(goff_tv[0, d, 0, 2] - want) < 1e-14
        assert goff_ref[0, d, 0, 2] == 0.0
        # elsewhere the two rules agree
        diff = goff_tv - goff_ref
        diff[0, d, 0, 2] = 0.0
        assert not diff.any()


def test_backward_rejects_bad_shapes():
    t, geo = rand_case(1, 2, 5, 5, 2, 3, 3, 1, 1, 1, 1, seed=12)
    with pytest.raises(ValueError):
        oracle.dcn_forward(t["input"], t["weight"], t["mask"], t["offset"][:, :4], t["bias"],
                           **geo)
    with pytest.raises(ValueError):
        oracle.dcn_backward(*(t[k] for k in IN5), t["grad_output"][:, :1], **geo)


# -- torchvision weight groups -------------------------------------------------------
WG_GEOMS = [
    # B, C, H, W, Co, kh, kw, s, p, d, G, WG
    (1, 4, 7, 7, 6, 3, 3, 1, 1, 1, 1, 2),
    (2, 6, 8, 9, 9, 3, 3, 2, 1, 1, 2, 3),
    (1, 4, 9, 8, 8, 3, 3, 1, 2, 2, 4, 4),   # depthwise-like: one input channel per group
    (1, 6, 6, 7, 4, 3, 2, 1, 1, 1, 3, 2),   # deformable groups cut across weight groups
]


def _grouped_case(geom, seed, osc=1.0):
    *g11, WG = geom
    t, geo = rand_case(*g11, seed=seed, osc=osc)
    C = g11[1]
    t["weight"] = t["weight"][:, : C // WG].contiguous()
    return t, geo, WG


@pytest.mark.parametrize("geom", WG_GEOMS)
def test_weight_groups_zero_offset_is_grouped_conv2d(geom):
    """Zero offset, mask 1: exactly F.conv2d(groups=WG), forward and the
    grad_input / grad_weight / grad_bias of its autograd."""
    t, geo, WG = _grouped_case(geom, seed=3)
    t["offset"].zero_()
    t["mask"].fill_(1.0)
    x = t["input"].clone().requires_grad_(True)
    w = t["weight"].clone().requires_grad_(True)
    b = t["bias"].clone().requires_grad_(True)
    ref = F.conv2d(x, w, b, stride=geo["stride"], padding=geo["padding"],
                   dilation=geo["dilation"], groups=WG)
    ref.backward(t["grad_output"])
    assert rel_err(fwd(t, geo), ref) < 1e-13
    gi, goff, gm, gw, gb = bwd(t, geo)
    assert gw.shape == tuple(w.shape)
    assert rel_err(gi, x.grad) < 1e-13
    assert rel_err(gw, w.grad) < 1e-13
    assert rel_err(gb, b.grad) < 1e-13


@pytest.mark.parametrize("geom", WG_GEOMS)
def test_weight_groups_match_independent_formulation(geom):
    """Random fractional offsets: the oracle's grouped loops against the
    grid_sample formulation, which contracts each weight group with its own
    matmul and takes every gradient from autograd."""
    from independent import forward_backward_gs
    t, geo, WG = _grouped_case(geom, seed=4, osc=1.3)
    out, *grads = forward_backward_gs(t["input"], t["weight"], t["offset"], t["mask"],
                                      t["bias"], t["grad_output"], **geo)
    assert rel_err(fwd(t, geo), out) < 1e-12
    for name, a, r in zip(GRADS, bwd(t, geo), grads):
        assert rel_err(a, r) < 1e-10, name


@pytest.mark.parametrize("geom", [
    # B, C, H, W, Co, kh, kw, s, p, d, G: H - 1 and W - 1 powers of two
    (2, 6, 17, 17, 5, 3, 3, 1, 1, 1, 2),
    (1, 4, 9, 17, 3, 3, 2, 2, 1, 2, 1),
    (1, 3, 5, 9, 2, 5, 5, 1, 2, 1, 1),
])
def test_integer_coordinates_match_grid_sample(geom):
    """Samples exactly on integer coordinates, the tie points of the bilinear
    weights where the coordinate gradient is one-sided: the oracle against the
    grid_sample formulation on images whose H - 1 and W - 1 are powers of two,
    so that grid_sample's align_corners normalisation maps every integer
    position to itself exactly.  grid_sample takes the floor-side difference
    there, as torchvision's get_coordinate_weight does, at y = -1 and x = -1
    too; there the reference's early exit (com.cu:392-396, ref_boundary=True)
    gives 0 instead, which this comparison tells apart.  A left-side rule (the
    positions nudged below the integers) misses by O(1)."""
    from independent import forward_backward_gs, sample_positions
    B, C, H, W, Co, kh, kw, s, p, d, G = geom
    t, geo = rand_case(*geom, seed=11)
    g = torch.Generator().manual_seed(12)
    t["offset"] = torch.randint(-4, 5, t["offset"].shape, generator=g).to(f64)
    out, *ref = forward_backward_gs(t["input"], t["weight"], t["offset"], t["mask"], t["bias"],
                                    t["grad_output"], **geo)
    Ho, Wo = out.shape[-2:]
    y, x = sample_positions(t["offset"], kh, kw, Ho, Wo, s, p, d, G)
    assert bool(((y == y.round()) & (x == x.round())).all())
    assert bool(((y == -1) | (x == -1)).any())  # boundary ties occur
    assert rel_err(fwd(t, geo), out) < 1e-13
    for name, a, r in zip(GRADS, bwd(t, geo), ref):
        assert rel_err(a, r) < 1e-12, name
    goff_ref_rule = bwd(t, geo, ref_boundary=True)[1]
    assert rel_err(goff_ref_rule, ref[1]) > 1e-3
    left = forward_backward_gs(t["input"], t["weight"], t["offset"] - 1e-9, t["mask"], t["bias"],
                               t["grad_output"], **geo)[2]
    assert rel_err(bwd(t, geo)[1], left) > 1e-2


def test_weight_groups_are_block_diagonal():
    """A grouped weight equals the full weight that is zero outside each output
    channel's group (forward and grad_input), and its grad_weight is that full
    weight's grad_weight restricted to the group blocks."""
    t, geo, WG = _grouped_case(WG_GEOMS[1], seed=5, osc=2.0)
    Co, Cw = t["weight"].shape[:2]
    full = torch.zeros(Co, Cw * WG, *t["weight"].shape[2:], dtype=f64)
    mpg = Co // WG
    for gw in range(WG):
        full[gw * mpg:(gw + 1) * mpg, gw * Cw:(gw + 1) * Cw] = t["weight"][gw * mpg:(gw + 1) * mpg]
    tf = dict(t, weight=full)
    assert rel_err(fwd(t, geo), fwd(tf, geo)) < 1e-13
    g_grp, g_full = bwd(t, geo), bwd(tf, geo)
    for i in (0, 1, 2, 4):
        assert rel_err(g_grp[i], g_full[i]) < 1e-12
    blocks = np.concatenate([g_full[3][gw * mpg:(gw + 1) * mpg, gw * Cw:(gw + 1) * Cw]
                             for gw in range(WG)])
    assert rel_err(g_grp[3], blocks) < 1e-13


def test_weight_groups_reject_bad_split():
    t, geo, _ = _grouped_case(WG_GEOMS[0], seed=6)
    t["weight"] = t["weight"][:5]   # Cout 5 does not split over 2 groups
    with pytest.raises(ValueError):
        fwd(t, geo)
