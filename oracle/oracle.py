"""Python front end of the CPU oracle (``dcn_oracle.c``).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of bench.py, as the checker or as the timed CPU
baseline.  The product path (``dcnv2_amd``) never imports it.

The semantics are those of ``torchvision.ops.deform_conv2d(input, offset,
weight, bias, stride, padding, dilation, mask)``, which the reference uses as
its comparator; the restated kernels cite the reference file:line they follow
in ``dcn_oracle.c``.  Argument order of :func:`dcn_forward` /
:func:`dcn_backward` mirrors ``_C.dcn_v2_forward`` / ``_C.dcn_v2_backward``
(reference ``dcn_v2_mm.py:20-30, 38-49``) with the dilation/group extension
appended.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile (gcc + OpenMP)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-B" if force else "all"], cwd=_HERE, check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        for suffix, ct in (("_f64", ctypes.c_double), ("_f32", ctypes.c_float)):
            p = ctypes.POINTER(ct)
            i = ctypes.c_int
            fwd = getattr(lib, "oracle_dcn_forward" + suffix)
            fwd.argtypes = [p] * 5 + [i] * 15 + [p, i, i]
            fwd.restype = i
            bwd = getattr(lib, "oracle_dcn_backward" + suffix)
            bwd.argtypes = [p] * 5 + [i] * 15 + [p] * 5 + [i, i, i]
            bwd.restype = i
        _lib = lib
    return _lib


def _pair(v):
    if isinstance(v, (tuple, list)):
        return int(v[0]), int(v[1])
    return int(v), int(v)


def _arr(x, dtype):
    if x is None:
        return None
    if hasattr(x, "detach"):  # torch tensor
        x = x.detach().cpu().double().numpy()
    return np.ascontiguousarray(np.asarray(x, dtype=np.float64), dtype=dtype)


def _ptr(a, ct):
    if a is None:
        return ctypes.POINTER(ct)()
    return a.ctypes.data_as(ctypes.POINTER(ct))


def out_size(n, k, s, p, d):
    return (n + 2 * p - (d * (k - 1) + 1)) // s + 1


def _geometry(input, weight, offset, mask, stride, padding, dilation, deformable_groups):
    B, C, H, W = input.shape
    Cout, Cw, kh, kw = weight.shape
    # torchvision's weight groups: C / weight.shape[1] of them
    if Cw <= 0 or C % Cw or Cout % (C // Cw):
        raise ValueError(f"weight has {Cw} input channels per group, input has {C}, "
                         f"output {Cout}")
    sh, sw = _pair(stride)
    ph, pw = _pair(padding)
    dh, dw = _pair(dilation)
    G = int(deformable_groups)
    Ho, Wo = out_size(H, kh, sh, ph, dh), out_size(W, kw, sw, pw, dw)
    if offset.shape != (B, 2 * G * kh * kw, Ho, Wo):
        raise ValueError(f"offset shape {offset.shape} != {(B, 2 * G * kh * kw, Ho, Wo)}")
    if mask is not None and mask.shape != (B, G * kh * kw, Ho, Wo):
        raise ValueError(f"mask shape {mask.shape} != {(B, G * kh * kw, Ho, Wo)}")
    return (B, C, H, W, Cout, kh, kw, sh, sw, ph, pw, dh, dw, G, C // Cw), (Ho, Wo)


def dcn_forward(input, weight, mask, offset, bias, stride=1, padding=0, dilation=1,
                deformable_groups=1, precision="f64", pos_f32=False, nthreads=0):
    """Oracle forward.  Returns a numpy array [B, Cout, Hout, Wout] in the
    requested precision ("f64" for parity, "f32" for the CPU baseline).
    ``pos_f32`` rounds each sample position to float32 first, as a float32
    implementation computes it (see dcn_oracle.c)."""
    dt, ct, sfx = ((np.float64, ctypes.c_double, "_f64") if precision == "f64"
                   else (np.float32, ctypes.c_float, "_f32"))
    x, w, o, m, b = (_arr(t, dt) for t in (input, weight, offset, mask, bias))
    geo, (Ho, Wo) = _geometry(x, w, o, m, stride, padding, dilation, deformable_groups)
    out = np.empty((geo[0], geo[4], Ho, Wo), dtype=dt)
    rc = getattr(_load(), "oracle_dcn_forward" + sfx)(
        _ptr(x, ct), _ptr(w, ct), _ptr(o, ct), _ptr(m, ct), _ptr(b, ct), *geo,
        _ptr(out, ct), int(bool(pos_f32)), int(nthreads))
    if rc != 0:
        raise ValueError(f"oracle forward rejected the arguments (rc={rc})")
    return out


def dcn_backward(input, weight, mask, offset, bias, grad_output, stride=1, padding=0,
                 dilation=1, deformable_groups=1, ref_boundary=False, precision="f64",
                 pos_f32=False, nthreads=0):
    """Oracle backward.  Returns (grad_input, grad_offset, grad_mask,
    grad_weight, grad_bias) -- the order of ``_C.dcn_v2_backward``
    (reference ``com.cu:845-847``).  ``ref_boundary`` selects the reference's
    early exit in the coordinate weight (``com.cu:392-396``) instead of
    torchvision's rule; they differ only for samples exactly on y == -1 or
    x == -1."""
    dt, ct, sfx = ((np.float64, ctypes.c_double, "_f64") if precision == "f64"
                   else (np.float32, ctypes.c_float, "_f32"))
    x, w, o, m, go = (_arr(t, dt) for t in (input, weight, offset, mask, grad_output))
    geo, (Ho, Wo) = _geometry(x, w, o, m, stride, padding, dilation, deformable_groups)
    B, C, H, W, Cout, kh, kw = geo[:7]
    G = geo[13]
    if go.shape != (B, Cout, Ho, Wo):
        raise ValueError(f"grad_output shape {go.shape} != {(B, Cout, Ho, Wo)}")
    gi = np.empty_like(x)
    gw = np.empty_like(w)
    gb = np.empty((Cout,), dtype=dt)
    goff = np.empty_like(o)
    gm = np.empty((B, G * kh * kw, Ho, Wo), dtype=dt) if m is not None else None
    rc = getattr(_load(), "oracle_dcn_backward" + sfx)(
        _ptr(x, ct), _ptr(w, ct), _ptr(o, ct), _ptr(m, ct), _ptr(go, ct), *geo,
        _ptr(gi, ct), _ptr(gw, ct), _ptr(gb, ct), _ptr(goff, ct), _ptr(gm, ct),
        int(bool(ref_boundary)), int(bool(pos_f32)), int(nthreads))
    if rc != 0:
        raise ValueError(f"oracle backward failed (rc={rc})")
    return gi, goff, gm, gw, gb
