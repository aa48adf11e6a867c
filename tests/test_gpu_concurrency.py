"""Calls from two host threads on two streams at once.

The library keeps no per-call state outside the caller's workspace (the Python
layer allocates one per call on the call's stream), its options are atomics
and its error text and stage timers are per thread, so forward and backward
calls that overlap on different streams must give what the same calls give one
at a time: the forward bitwise (it is deterministic), the backward within the
tolerance (its fp32 atomics and bucket order are not).
"""
from __future__ import annotations

import threading

import pytest
import torch

from dcnv2_amd import _C
from dcnv2_amd.workloads import CONFIGS, make_inputs
from util import GRADS, TOL, check

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
IN5 = ("input", "weight", "mask", "offset", "bias")


def _geo(w):
    return (w.stride, w.stride, w.pad, w.pad, w.dil, w.dil, w.groups)


def test_two_threads_two_streams():
    ws = [CONFIGS[0].with_(B=2, C=64, H=24, W=20, Cout=256, dtype=torch.float16, seed=61, backward=True),
          CONFIGS[0].with_(B=3, C=48, H=17, W=16, Cout=96, dtype=torch.bfloat16, seed=62, groups=2,
                           backward=True)]
    ts = [{k: v.to(DEV) for k, v in make_inputs(w).items()} for w in ws]

    def run(w, t):
        y = _C.dcn_v2_forward(*(t[k] for k in IN5), *_geo(w))
        g = _C.dcn_v2_backward(*(t[k] for k in IN5), t["grad_output"], *_geo(w))
        return y, g

    ref = []
    for w, t in zip(ws, ts):
        ref.append(run(w, t))
        torch.cuda.synchronize()
    results = [[], []]
    errors = []

    def worker(i):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                for _ in range(5):
                    results[i].append(run(ws[i], ts[i]))
            s.synchronize()
        except Exception as e:  # reported by the main thread
            errors.append(e)

    th = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for x in th:
        x.start()
    for x in th:
        x.join(timeout=120)
    assert not any(x.is_alive() for x in th), "a worker did not finish"
    assert not errors, errors
    torch.cuda.synchronize()
    for i, w in enumerate(ws):
        y0, g0 = ref[i]
        for y, g in results[i]:
            assert torch.equal(y, y0), f"forward of thread {i}"
            for name, a, b in zip(GRADS, g, g0):
                check(f"{name} (thread {i})", a, b, TOL[w.dtype])
