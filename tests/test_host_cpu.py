"""Host-side checks that need no GPU.

* the C-ABI library loads and exports every entry point ``include/dcnv2_amd.h``
  declares;
* its host-only entry points: output shape, workspace sizes, argument
  validation and error codes/messages (no kernel is launched by any of them);
* the Python operator surface: the reference's argument checks raise
  ``RuntimeError`` (``com.cu:209-213, 760-761``), and there is no CPU
  fallback;
* autograd plumbing of ``_DCNv2``/``DCN`` (reference ``dcn_v2_mm.py:15-56,
  133-137``): with ``_C`` replaced by the CPU oracle, the module's gradients
  equal the independent grid_sample formulation's, which pins the argument
  order, the ``(gI, gOff, gMask, gW, gB)`` -> ``(gI, gW, gMask, gOff, gB)``
  remapping and the chunk/cat/sigmoid split;
* the workload table and FLOP formulas used by bench.py.
"""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest
import torch

import dcnv2_amd
from dcnv2_amd import _C, dcn_v2_mm
from dcnv2_amd.workloads import CONFIGS, make_inputs
from independent import deform_conv2d_gs
from oracle import oracle
from util import rel_err

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dcnv2_amd.h")


@pytest.fixture(scope="module")
def L():
    if not os.path.exists(_C.library_path()):
        from dcnv2_amd import build
        build.build()
    return _C.lib()


def header_functions():
    text = open(HEADER).read()
    return re.findall(r"DCN2_API\s+[\w\s\*]+?\b(dcn2_\w+)\s*\(", text)


def desc(B=2, C=8, H=9, W=10, Co=5, kh=3, kw=3, sh=1, sw=1, ph=1, pw=1, dh=1, dw=1, G=1,
         dtype=0, WG=0, layout=0, out_layout=0):
    return _C.Desc(B, C, H, W, Co, kh, kw, sh, sw, ph, pw, dh, dw, G, dtype, WG, layout,
                   out_layout)


def out_hw(L, d):
    ho, wo = ctypes.c_int32(-1), ctypes.c_int32(-1)
    rc = L.dcn2_output_shape(ctypes.byref(d), ctypes.byref(ho), ctypes.byref(wo))
    return rc, ho.value, wo.value


# -- the C ABI -----------------------------------------------------------------
def test_exports_every_declared_symbol(L):
    names = header_functions()
    assert set(names) >= {"dcn2_forward", "dcn2_backward", "dcn2_output_shape",
                          "dcn2_forward_workspace_bytes", "dcn2_backward_workspace_bytes",
                          "dcn2_last_error", "dcn2_version"}
    raw = ctypes.CDLL(_C.library_path())
    for n in names:
        assert hasattr(raw, n), n


def test_version(L):
    """The version string carries the header's ABI version, and the Python
    descriptor has the header's field count."""
    abi = re.search(r"#define DCN2_ABI_VERSION (\d+)", open(HEADER).read()).group(1)
    assert L.dcn2_version().decode() == f"dcnv2_amd {abi} gfx950"
    struct = re.search(r"typedef struct dcn2_desc \{(.*?)\} dcn2_desc;", open(HEADER).read(), re.S)
    fields = re.findall(r"\b(\w+)\s*[,;]", re.sub(r"/\*.*?\*/", "", struct.group(1)))
    assert [f for f, _ in _C.Desc._fields_] == fields


@pytest.mark.parametrize("geo", [
    dict(H=9, W=10, kh=3, kw=3, sh=1, sw=1, ph=1, pw=1, dh=1, dw=1),
    dict(H=128, W=128, kh=3, kw=3, sh=2, sw=2, ph=2, pw=2, dh=2, dw=2),
    dict(H=7, W=5, kh=5, kw=3, sh=1, sw=2, ph=2, pw=0, dh=1, dw=1),
    dict(H=6, W=6, kh=1, kw=1, sh=1, sw=1, ph=0, pw=0, dh=1, dw=1),
])
def test_output_shape_matches_formula(L, geo):
    d = desc(**geo)
    rc, ho, wo = out_hw(L, d)
    assert rc == 0
    assert ho == oracle.out_size(geo["H"], geo["kh"], geo["sh"], geo["ph"], geo["dh"])
    assert wo == oracle.out_size(geo["W"], geo["kw"], geo["sw"], geo["pw"], geo["dw"])


@pytest.mark.parametrize("bad,code,msg", [
    (dict(G=3), 1, "divisible"),
    (dict(WG=3), 1, "weight_groups"),
    (dict(C=8, Co=6, WG=4), 1, "weight_groups"),
    (dict(WG=-1), 1, "weight_groups"),
    (dict(layout=2), 1, "input_layout"),
    (dict(out_layout=-1), 1, "output_layout"),
    (dict(dtype=7), 1, "dtype"),
    (dict(C=0), 1, "shape"),
    (dict(sh=0), 1, "stride"),
    (dict(H=2, W=2, ph=0, pw=0), 1, "empty output"),
    (dict(H=40000, W=4), 4, "32-bit"),
    (dict(B=70000), 4, "32-bit"),
])
def test_invalid_descriptors(L, bad, code, msg):
    d = desc(**bad)
    rc, _, _ = out_hw(L, d)
    assert rc == code
    assert msg in L.dcn2_last_error().decode()
    assert L.dcn2_forward_workspace_bytes(ctypes.byref(d)) == 0
    assert L.dcn2_backward_workspace_bytes(ctypes.byref(d)) == 0


def test_workspace_sizes(L):
    for dtype, esz in ((0, 4), (1, 2), (2, 2)):
        small, big = desc(dtype=dtype), desc(B=4, dtype=dtype)
        fs, fb = (L.dcn2_forward_workspace_bytes(ctypes.byref(x)) for x in (small, big))
        bs, bb = (L.dcn2_backward_workspace_bytes(ctypes.byref(x)) for x in (small, big))
        assert 0 < fs < fb and 0 < bs < bb
        assert fs % 256 == 0 and bs % 256 == 0
        # at least the channels-last input copy (channels padded to the chunk)
        Cgp = 32 if dtype == 0 else 64
        assert fs >= 2 * 9 * 10 * Cgp * esz
    # empty batch still has a valid workspace (weight packing)
    assert L.dcn2_forward_workspace_bytes(ctypes.byref(desc(B=0))) > 0


def test_backward_workspace_is_exact_size(L):
    """The grad_input buckets hold one row per sample (B*G*kh*kw*Ho*Wo rows of
    Cg rounded to 64 channels), however the samples cluster, so the c2 shape
    (B8 C64 128x128 Cout256 fp16) needs about 188 MB: channels-last input
    copy 16.8 MB (whose bytes the 10.6 MB of border rings reuse once the
    column-gradient kernel is done with it), rows 151 MB, 12-byte records
    14.2 MB, sample rows 4.7 MB, packed weights and grad_weight accumulator
    0.9 MB.  Its
    buckets are full enough for the by-cells grad_input.  Both grad_input
    kernels write the caller's grad_input directly; the per-pixel form
    (option gi_push = 0) adds an fp32 accumulator of one slot of 15 x 15
    interior pixels per bucket of more than 4096 samples, of which there are
    at most rows / 4097: 287 slots of 57.6 KB, 16.5 MB (an accumulator for
    every pixel would be 33.6 MB).  (Unsliced: the slice budget is raised for
    the comparison.)"""
    with _C.option("bwd_slice_bytes", 1 << 40):
        d = desc(B=8, C=64, H=128, W=128, Co=256, dtype=1)
        nbytes = L.dcn2_backward_workspace_bytes(ctypes.byref(d))
        rows = 8 * 9 * 128 * 128
        assert rows * (64 * 2 + 12) < nbytes < 200e6
        # bf16 hands fp16 rows with one scale byte per 32 channels to the gather
        d16 = desc(B=8, C=64, H=128, W=128, Co=256, dtype=2)
        assert L.dcn2_backward_workspace_bytes(ctypes.byref(d16)) - nbytes == rows * 2
        with _C.option("gi_push", 0):
            acc = rows // 4097 * 15 * 15 * 64 * 4
            pad = -acc % 256
            assert L.dcn2_backward_workspace_bytes(ctypes.byref(d)) - nbytes == acc + pad


def _ws(L, **kw):
    return L.dcn2_backward_workspace_bytes(ctypes.byref(desc(**kw)))


def test_backward_workspace_slices_the_batch(L):
    """The backward runs the batch in slices of whole images whose workspace
    fits the slice budget (default 192 MiB): c2 (188 MB) and c4 (128 MB) fit in
    one slice; c3 (B16 C256 64x64 dg4 bf16, 23.6 MB per image, 382 MB in one
    piece) runs as two slices of eight images, within 200 MB.  A smaller budget gives equal
    slices (B = 7 with room for 3 images: 3 + 2 + 2, workspace of 3), and a
    budget below one image still runs one image per slice."""
    assert _C.get_option("bwd_slice_bytes") == 192 << 20
    c2 = dict(B=8, C=64, H=128, W=128, Co=256, dtype=1)
    c3 = dict(B=16, C=256, H=64, W=64, Co=256, G=4, dtype=2)
    c4 = dict(B=2, C=128, H=256, W=256, Co=128, sh=2, sw=2, ph=2, pw=2, dh=2, dw=2, dtype=1)
    with _C.option("bwd_slice_bytes", 1 << 40):
        full = {k: _ws(L, **v) for k, v in (("c2", c2), ("c3", c3), ("c4", c4))}
        c3_one, c3_eight = _ws(L, **dict(c3, B=1)), _ws(L, **dict(c3, B=8))
        # eight images fit the budget, nine do not: 16 = 8 + 8
        assert c3_eight <= 192 << 20 < _ws(L, **dict(c3, B=9))
    assert _ws(L, **c2) == full["c2"] < 190e6
    assert _ws(L, **c4) == full["c4"] < 130e6
    assert full["c3"] > 380e6
    assert _ws(L, **c3) == c3_eight < 200e6
    one, two, three = (_ws(L, **dict(c2, B=b)) for b in (1, 2, 3))
    with _C.option("bwd_slice_bytes", three):
        assert _ws(L, **dict(c2, B=7)) == three
        assert _ws(L, **dict(c2, B=6)) == three
        assert _ws(L, **dict(c2, B=4)) == two
    with _C.option("bwd_slice_bytes", one - 1):
        assert _ws(L, **dict(c2, B=5)) == one
    assert c3_one < c3_eight


def test_options_reject_bad_values(L):
    for name, bad in (("bwd_slice_bytes", 0), ("bwd_fused", 1), ("gi_push", 2), ("gi_push", -2)):
        prev = _C.get_option(name)
        with pytest.raises(RuntimeError, match="dcn2_set_option"):
            _C.set_option(name, bad)
        assert _C.get_option(name) == prev
    assert L.dcn2_set_option(7, 0) == 1 and "unknown option" in L.dcn2_last_error().decode()
    assert L.dcn2_get_option(7) == -2


def test_per_image_byte_range(L):
    """A channels-last input copy of 4 GiB or more per image is rejected with
    DCN2_ERANGE before anything runs (fp32, C 256, 2048 x 2048: 4 GiB), while
    one just below fits (2047 x 2048)."""
    d = desc(B=1, C=256, H=2048, W=2048, Co=32, dtype=0)
    rc, _, _ = out_hw(L, d)
    assert rc == 4 and "byte range" in L.dcn2_last_error().decode()
    assert L.dcn2_forward_workspace_bytes(ctypes.byref(d)) == 0
    assert L.dcn2_backward_workspace_bytes(ctypes.byref(d)) == 0
    rc, _, _ = out_hw(L, desc(B=1, C=256, H=2047, W=2048, Co=32, dtype=0))
    assert rc == 0


def test_entry_points_reject_before_any_launch(L):
    """Error paths that return before touching the device."""
    d = desc()
    vp = ctypes.c_void_p
    fake = vp(0x1000)
    # invalid descriptor
    rc = L.dcn2_forward(ctypes.byref(desc(G=3)), fake, fake, None, fake, None, fake,
                        fake, 1 << 20, None)
    assert rc == 1
    # null input pointer
    rc = L.dcn2_forward(ctypes.byref(d), None, fake, None, fake, None, fake, fake, 1 << 20,
                        None)
    assert rc == 1 and "null" in L.dcn2_last_error().decode()
    # workspace too small / misaligned
    need = L.dcn2_forward_workspace_bytes(ctypes.byref(d))
    rc = L.dcn2_forward(ctypes.byref(d), fake, fake, None, fake, None, fake, vp(0x10000),
                        need - 1, None)
    assert rc == 2 and str(need) in L.dcn2_last_error().decode()
    rc = L.dcn2_forward(ctypes.byref(d), fake, fake, None, fake, None, fake, vp(0x10010),
                        need, None)
    assert rc == 2
    # backward: grad_mask must be given exactly when mask is
    rc = L.dcn2_backward(ctypes.byref(d), fake, fake, fake, fake, fake, fake, fake, None,
                         fake, None, fake, 1 << 30, None)
    assert rc == 1 and "grad_mask" in L.dcn2_last_error().decode()
    need = L.dcn2_backward_workspace_bytes(ctypes.byref(d))
    rc = L.dcn2_backward(ctypes.byref(d), fake, fake, None, fake, fake, fake, fake, None,
                         fake, None, vp(0x10000), need - 256, None)
    assert rc == 2
    # the fused offset/mask entry points: null om, invalid descriptor, small workspace
    rc = L.dcn2_forward_om(ctypes.byref(d), fake, fake, None, None, fake, fake, 1 << 20, None)
    assert rc == 1 and "om" in L.dcn2_last_error().decode()
    rc = L.dcn2_forward_om(ctypes.byref(desc(G=3)), fake, fake, fake, None, fake, fake,
                           1 << 20, None)
    assert rc == 1
    rc = L.dcn2_backward_om(ctypes.byref(d), fake, fake, fake, fake, fake, None, fake, None,
                            fake, 1 << 30, None)
    assert rc == 1 and "grad_om" in L.dcn2_last_error().decode()
    rc = L.dcn2_backward_om(ctypes.byref(d), fake, fake, fake, fake, fake, fake, fake, None,
                            vp(0x10000), need - 256, None)
    assert rc == 2


# -- the Python operator surface -------------------------------------------------
def _cpu_case(dtype=torch.float32):
    return make_inputs(CONFIGS[0], dtype=dtype, with_grad=True)


def test_cpu_tensors_raise_runtime_error():
    t = _cpu_case()
    with pytest.raises(RuntimeError, match="GPU"):
        _C.dcn_v2_forward(t["input"], t["weight"], t["mask"], t["offset"], t["bias"],
                          1, 1, 1, 1)
    with pytest.raises(RuntimeError, match="GPU"):
        _C.dcn_v2_backward(t["input"], t["weight"], t["mask"], t["offset"], t["bias"],
                           t["grad_output"], 1, 1, 1, 1)
    om = torch.cat([t["offset"], t["mask"]], 1)
    with pytest.raises(RuntimeError, match="GPU"):
        _C.dcn_v2_forward_om(t["input"], t["weight"], om, t["bias"], 1, 1, 1, 1)
    with pytest.raises(RuntimeError, match="GPU"):
        _C.dcn_v2_backward_om(t["input"], t["weight"], om, t["bias"], t["grad_output"],
                              1, 1, 1, 1)


def test_module_without_gpu_raises_not_falls_back():
    m = dcnv2_amd.DCN(4, 4, 3, 1, 1)
    with pytest.raises(RuntimeError):
        m(torch.randn(1, 4, 6, 6))


# -- autograd plumbing with _C replaced by the CPU oracle -------------------------
def _oracle_forward(input, weight, mask, offset, bias, sh, sw, ph, pw, dh=1, dw=1, G=1):
    out = oracle.dcn_forward(input, weight, mask, offset, bias, (sh, sw), (ph, pw), (dh, dw), G)
    return torch.from_numpy(out)


def _oracle_backward(input, weight, mask, offset, bias, grad_output, sh, sw, ph, pw, dh=1,
                     dw=1, G=1):
    gi, goff, gm, gw, gb = oracle.dcn_backward(input, weight, mask, offset, bias, grad_output,
                                               (sh, sw), (ph, pw), (dh, dw), G)
    gb = torch.from_numpy(gb) if bias is not None else None
    gm = torch.from_numpy(gm) if mask is not None else None
    return [torch.from_numpy(gi), torch.from_numpy(goff), gm, torch.from_numpy(gw), gb]


def _oracle_forward_om(input, weight, om, bias, sh, sw, ph, pw, dh=1, dw=1, G=1):
    n = om.shape[1] // 3 * 2
    return _oracle_forward(input, weight, torch.sigmoid(om[:, n:]), om[:, :n], bias, sh, sw,
                           ph, pw, dh, dw, G)


def _oracle_backward_om(input, weight, om, bias, grad_output, sh, sw, ph, pw, dh=1, dw=1, G=1):
    n = om.shape[1] // 3 * 2
    s = torch.sigmoid(om[:, n:])
    gi, goff, gm, gw, gb = _oracle_backward(input, weight, s, om[:, :n], bias, grad_output,
                                            sh, sw, ph, pw, dh, dw, G)
    return [gi, torch.cat([goff, gm * s * (1 - s)], 1), gw, gb]


@pytest.fixture
def oracle_C(monkeypatch):
    monkeypatch.setattr(dcn_v2_mm._C, "dcn_v2_forward", _oracle_forward)
    monkeypatch.setattr(dcn_v2_mm._C, "dcn_v2_backward", _oracle_backward)
    monkeypatch.setattr(dcn_v2_mm._C, "dcn_v2_forward_om", _oracle_forward_om)
    monkeypatch.setattr(dcn_v2_mm._C, "dcn_v2_backward_om", _oracle_backward_om)


def test_dcn_v2_conv_gradients_in_reference_order(oracle_C):
    g = torch.Generator().manual_seed(0)
    f64 = torch.float64
    x = torch.randn(2, 4, 7, 8, generator=g, dtype=f64)
    w = torch.randn(3, 4, 3, 3, generator=g, dtype=f64)
    off = torch.randn(2, 2 * 2 * 9, 4, 4, generator=g, dtype=f64) * 1.5
    m = torch.rand(2, 2 * 9, 4, 4, generator=g, dtype=f64)
    b = torch.randn(3, generator=g, dtype=f64)
    go = torch.randn(2, 3, 4, 4, generator=g, dtype=f64)
    ours = [t.clone().requires_grad_(True) for t in (x, w, m, off, b)]
    y = dcnv2_amd.dcn_v2_conv(*ours, 2, 1, 1, 2)
    y.backward(go)
    ref = [t.clone().requires_grad_(True) for t in (x, w, off, m, b)]
    y_ref = deform_conv2d_gs(*ref, stride=2, padding=1, dilation=1, deformable_groups=2)
    y_ref.backward(go)
    assert rel_err(y, y_ref) < 1e-12
    ref_by_name = dict(zip(("input", "weight", "offset", "mask", "bias"), ref))
    for name, t in zip(("input", "weight", "mask", "offset", "bias"), ours):
        assert rel_err(t.grad, ref_by_name[name].grad) < 1e-12, name


@pytest.mark.parametrize("fused", [True, False], ids=["fused_om", "separate"])
def test_dcn_module_split_and_sigmoid(oracle_C, fused):
    """DCN: offset = cat(o1, o2), mask = sigmoid(third chunk) of the predictor
    output; with a non-zero predictor the whole module (predictor included)
    matches the independent formulation, values and parameter gradients.  The
    fused path hands the raw predictor output to the operator, whose backward
    returns the gradient of the logits (grad_mask * s * (1 - s))."""
    torch.manual_seed(1)
    mod = dcnv2_amd.DCN(4, 3, 3, stride=1, padding=1, dilation=1, deformable_groups=2,
                        fused_offset_mask=fused).double()
    assert not mod.conv_offset_mask.weight.any()  # zero-initialised, reference :129-131
    with torch.no_grad():
        mod.conv_offset_mask.weight.normal_(0, 0.3)
        mod.conv_offset_mask.bias.normal_(0, 0.3)
    x = torch.randn(2, 4, 6, 6, dtype=torch.float64, requires_grad=True)
    y = mod(x)
    go = torch.randn_like(y)
    y.backward(go)
    grads = {n: p.grad.clone() for n, p in mod.named_parameters()}
    gx = x.grad.clone()

    x2 = x.detach().clone().requires_grad_(True)
    params = {n: p.detach().clone().requires_grad_(True) for n, p in mod.named_parameters()}
    om = torch.nn.functional.conv2d(x2, params["conv_offset_mask.weight"],
                                    params["conv_offset_mask.bias"], padding=1)
    o1, o2, mk = torch.chunk(om, 3, dim=1)
    y2 = deform_conv2d_gs(x2, params["weight"], torch.cat((o1, o2), 1), torch.sigmoid(mk),
                          params["bias"], stride=1, padding=1, dilation=1, deformable_groups=2)
    y2.backward(go)
    assert rel_err(y, y2) < 1e-12
    assert rel_err(gx, x2.grad) < 1e-10
    for n, p in params.items():
        assert rel_err(grads[n], p.grad) < 1e-10, n


def test_reference_import_shims():
    import Conv2d
    import dcn_v2_mm as shim
    assert Conv2d._C is _C
    assert shim.DCN is dcnv2_amd.DCN and shim.dcn_v2_conv is dcnv2_amd.dcn_v2_conv


# -- workloads ---------------------------------------------------------------
def test_workload_flops_and_determinism():
    c1 = CONFIGS[1]
    assert c1.gemm_flops() == pytest.approx(3.8655e10, rel=1e-4)
    assert c1.readme_flops() == pytest.approx(1.93878e11, rel=1e-5)
    assert CONFIGS[3].gemm_flops() == pytest.approx(7.7309e10, rel=1e-4)
    assert CONFIGS[4].gemm_flops() == pytest.approx(9.6637e9, rel=1e-4)
    a = make_inputs(CONFIGS[0])
    b = make_inputs(CONFIGS[0])
    for k in a:
        if a[k] is not None:
            assert torch.equal(a[k], b[k]), k
    assert np.isfinite(a["offset"].numpy()).all()


def test_dcnv2_module_weight_groups(oracle_C):
    """DCNv2(groups=2): weight [Cout, C/2, kh, kw], fan-in init over C/2*kh*kw,
    and the autograd plumbing carries the grouped weight through unchanged
    (values and gradients against the grid_sample formulation)."""
    torch.manual_seed(2)
    mod = dcnv2_amd.DCNv2(6, 4, 3, stride=1, padding=1, deformable_groups=3, groups=2).double()
    assert tuple(mod.weight.shape) == (4, 3, 3, 3)
    assert float(mod.weight.detach().abs().max()) <= 1.0 / (3 * 9) ** 0.5
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 6, 7, 6, generator=g, dtype=torch.float64)
    off = torch.randn(2, 2 * 3 * 9, 7, 6, generator=g, dtype=torch.float64) * 1.2
    m = torch.rand(2, 3 * 9, 7, 6, generator=g, dtype=torch.float64)
    go = torch.randn(2, 4, 7, 6, generator=g, dtype=torch.float64)
    with torch.no_grad():
        mod.bias.normal_()
    y = mod(x, off, m)
    y.backward(go)
    w = mod.weight.detach().clone().requires_grad_(True)
    y_ref = deform_conv2d_gs(x, w, off, m, mod.bias.detach(), stride=1, padding=1,
                             dilation=1, deformable_groups=3)
    y_ref.backward(go)
    assert rel_err(y, y_ref) < 1e-12
    assert rel_err(mod.weight.grad, w.grad) < 1e-12
    with pytest.raises(ValueError):
        dcnv2_amd.DCNv2(6, 5, 3, 1, 1, groups=2)


def test_channels_last_workspace(L):
    """A channels-last input whose channels need no padding is read in place:
    the workspace drops exactly the repacked copy; with padding it keeps it.
    (The backward's border rings, 64 pixels x Cgp fp32 per cell-tile bucket,
    reuse the copy's bytes when they fit there, so without a copy they take
    their own.)"""
    al = lambda n: (n + 255) // 256 * 256
    for dtype, esz, C in ((1, 2, 64), (2, 2, 128), (0, 4, 32)):
        nchw, nhwc = desc(C=C, dtype=dtype), desc(C=C, dtype=dtype, layout=1)
        copy = al(2 * 9 * 10 * C * esz)
        rings = al(2 * 64 * C * 4)  # B = 2 images of one bucket each; Cgp == C here
        a, b = (L.dcn2_forward_workspace_bytes(ctypes.byref(x)) for x in (nchw, nhwc))
        assert 0 < b < a and a - b == copy
        a, b = (L.dcn2_backward_workspace_bytes(ctypes.byref(x)) for x in (nchw, nhwc))
        assert 0 < b < a and a - b == copy - (rings if rings <= copy else 0)
    padded_cl, padded = desc(C=24, dtype=1, layout=1), desc(C=24, dtype=1)
    assert L.dcn2_forward_workspace_bytes(ctypes.byref(padded_cl)) == \
        L.dcn2_forward_workspace_bytes(ctypes.byref(padded))


def test_torchvision_signature(oracle_C):
    """deform_conv2d(input, offset, weight, bias, stride, padding, dilation,
    mask): deformable groups from the offset's channels, weight groups from the
    weight's shape, non-square geometry passed through, all five gradients."""
    g = torch.Generator().manual_seed(4)
    f64 = torch.float64
    x = torch.randn(2, 6, 9, 8, generator=g, dtype=f64)
    w = torch.randn(4, 3, 3, 2, generator=g, dtype=f64)        # 2 weight groups, 3x2 kernel
    Ho, Wo = (9 + 2 * 1 - (1 * 2 + 1)) // 2 + 1, (8 + 2 * 2 - (2 * 1 + 1)) // 1 + 1
    off = torch.randn(2, 2 * 3 * 6, Ho, Wo, generator=g, dtype=f64) * 1.3   # 3 deformable groups
    m = torch.rand(2, 3 * 6, Ho, Wo, generator=g, dtype=f64)
    b = torch.randn(4, generator=g, dtype=f64)
    go = torch.randn(2, 4, Ho, Wo, generator=g, dtype=f64)
    ours = [t.clone().requires_grad_(True) for t in (x, off, w, b, m)]
    y = dcnv2_amd.deform_conv2d(ours[0], ours[1], ours[2], ours[3], stride=(2, 1),
                                padding=(1, 2), dilation=(1, 2), mask=ours[4])
    y.backward(go)
    ref = [t.clone().requires_grad_(True) for t in (x, off, w, b, m)]
    y_ref = deform_conv2d_gs(ref[0], ref[2], ref[1], ref[4], ref[3], stride=(2, 1),
                             padding=(1, 2), dilation=(1, 2), deformable_groups=3)
    y_ref.backward(go)
    assert y.shape == (2, 4, Ho, Wo)
    assert rel_err(y, y_ref) < 1e-12
    for a, r in zip(ours, ref):
        assert rel_err(a.grad, r.grad) < 1e-11
    with pytest.raises(RuntimeError):
        dcnv2_amd.deform_conv2d(x, off[:, :5], w)
    with pytest.raises(RuntimeError):
        dcnv2_amd.deform_conv2d(x, off, w, mask=m[:, :4])
