"""dcn2_forward_noalloc (include/dcnv2_amd.h): the forward with its workspace
in the library's static device scratch array instead of a caller-provided
buffer.  Called through the C ABI and compared with dcn2_forward on the same
inputs: the two run the same kernels on the same data, so the outputs must be
bitwise equal (stricter than the 1e-2 / 1e-4 parity tolerance).  Two calls in
a row, the second on a smaller problem (and a third in another dtype), so
leftovers of an earlier call in the shared array would show."""
from __future__ import annotations

import ctypes

import pytest
import torch

from dcnv2_amd import _C
from dcnv2_amd.workloads import CONFIGS, make_inputs

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
IN5 = ("input", "weight", "mask", "offset", "bias")


def _noalloc(t, w, out, in_layout=0, out_layout=0):
    desc = _C.make_desc(t["input"], t["weight"], w.stride, w.stride, w.pad, w.pad, w.dil, w.dil,
                        w.groups, in_layout, out_layout)
    stream = torch.cuda.current_stream(DEV).cuda_stream
    ptr = lambda v: ctypes.c_void_p(v.data_ptr())  # noqa: E731
    rc = _C.lib().dcn2_forward_noalloc(ctypes.byref(desc), *(ptr(t[k]) for k in IN5), ptr(out),
                                       ctypes.c_void_p(stream))
    return rc


@pytest.mark.parametrize("cases", [[
    # first call: the c1 headline shape (17 MB of workspace); second: a
    # smaller problem with channel padding and two deformable groups; third:
    # fp32
    CONFIGS[1],
    CONFIGS[0].with_(B=2, C=24, H=17, W=13, Cout=40, groups=2, dtype=torch.float16, seed=9),
    CONFIGS[0].with_(B=1, C=16, H=20, W=18, Cout=24, seed=10),
]], ids=["c1_then_smaller_then_fp32"])
def test_noalloc_matches_forward(cases):
    for w in cases:
        t = {k: v.to(DEV) for k, v in make_inputs(w).items()}
        ref = _C.dcn_v2_forward(*(t[k] for k in IN5), w.stride, w.stride, w.pad, w.pad, w.dil,
                                w.dil, w.groups)
        out = torch.full_like(ref, float("nan"))
        rc = _noalloc(t, w, out)
        assert rc == 0, _C.lib().dcn2_last_error().decode()
        torch.cuda.synchronize()
        print(f"  {w.name} B{w.B} C{w.C} {w.H}x{w.W} Cout{w.Cout} {w.dtype}: "
              f"max|diff| = {(out.float() - ref.float()).abs().max().item():.3e}")
        assert torch.equal(out, ref)


def test_noalloc_rejects_oversized_problem():
    """A problem whose workspace exceeds the scratch array is refused before
    anything is launched."""
    w = CONFIGS[1].with_(B=64)  # 134 MB of channels-last input copy
    t = {k: v.to(DEV) for k, v in make_inputs(w.with_(B=1)).items()}
    desc = _C.make_desc(t["input"].expand(64, -1, -1, -1), t["weight"], 1, 1, 1, 1, 1, 1, 1)
    assert _C.lib().dcn2_forward_workspace_bytes(ctypes.byref(desc)) > 64 << 20
    rc = _C.lib().dcn2_forward_noalloc(ctypes.byref(desc), *([None] * 7))
    assert rc == 2  # DCN2_EWORKSPACE
    assert "static scratch" in _C.lib().dcn2_last_error().decode()


def test_noalloc_channels_last():
    """A channels_last fp16 input of 64 channels (read in place) and a
    channels_last output (input_layout = output_layout = 1): bitwise equal to
    dcn_v2_forward on the same channels_last tensors."""
    w = CONFIGS[0].with_(B=2, C=64, H=15, W=14, Cout=200, dtype=torch.float16, seed=12)
    t = {k: v.to(DEV) for k, v in make_inputs(w).items()}
    cl = torch.channels_last
    t["input"] = t["input"].to(memory_format=cl)
    ref = _C.dcn_v2_forward(*(t[k] for k in IN5), w.stride, w.stride, w.pad, w.pad, w.dil,
                            w.dil, w.groups)
    assert ref.is_contiguous(memory_format=cl)
    out = torch.full_like(ref, float("nan"))  # keeps the channels_last layout
    rc = _noalloc(t, w, out, 1, 1)
    assert rc == 0, _C.lib().dcn2_last_error().decode()
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def test_noalloc_under_graph_capture():
    """The first call on a device looks the scratch array up (outside any
    capture); after that dcn2_forward_noalloc can be captured into a HIP graph
    (it allocates nothing and issues no memset).  Every replay, with eager
    work and synchronisation in between and new input values copied in, is
    bitwise equal to dcn_v2_forward on the same inputs."""
    w = CONFIGS[0].with_(B=2, C=32, H=16, W=15, Cout=160, dtype=torch.float16, seed=14)
    t = {k: v.to(DEV) for k, v in make_inputs(w).items()}
    out = torch.empty(w.B, w.Cout, w.H, w.W, dtype=torch.float16, device=DEV)
    assert _noalloc(t, w, out) == 0  # warm-up: the per-device lookup happens here
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            rc = _noalloc(t, w, out)
    assert rc == 0, _C.lib().dcn2_last_error().decode()
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(3):
        g = torch.Generator(device="cpu").manual_seed(100 + rep)
        t["input"].copy_(torch.randn(t["input"].shape, generator=g).to(torch.float16))
        t["offset"].copy_((torch.randn(t["offset"].shape, generator=g) * 2.0).to(torch.float16))
        junk = torch.randn(1 << 16, device=DEV).sum()  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ref = _C.dcn_v2_forward(*(t[k] for k in IN5), w.stride, w.stride, w.pad, w.pad, w.dil,
                                w.dil, w.groups)
        torch.cuda.synchronize()
        assert torch.isfinite(junk)
        assert torch.equal(out, ref), f"replay {rep}"
