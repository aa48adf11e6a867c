"""Sustained dense fp16 MFMA rate of the GPU (libdcn2_probe.so).

The MI355X lowers its shader clock under dense MFMA work on toggling data, so
the rate it sustains depends on the operands.  mfma_ceiling() measures it in
the issue pattern of the forward kernel for zero and N(0,1) operands; bench.py
reports the result beside the published peak.  A measurement tool only: the
operator path never calls it.
"""
from __future__ import annotations

import ctypes
import os

_LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libdcn2_probe.so")


def mfma_ceiling(steps: int = 1440) -> dict:
    """{"zero": {"tflops", "mhz"}, "normal": {...}} for 32x32x16 f16 MFMAs."""
    lib = ctypes.CDLL(_LIB)
    fn = lib.dcn2_probe_mfma
    fn.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_double),
                   ctypes.POINTER(ctypes.c_double)]
    fn.restype = ctypes.c_int
    out = {}
    for kind, name in ((0, "zero"), (1, "normal")):
        tf, mhz = ctypes.c_double(), ctypes.c_double()
        rc = fn(kind, steps, ctypes.byref(tf), ctypes.byref(mhz))
        if rc != 0:
            raise RuntimeError(f"dcn2_probe_mfma failed (HIP error {rc})")
        out[name] = {"tflops": round(tf.value, 1), "mhz": round(mhz.value)}
    return out
