"""Shared helpers of the test suite."""
from __future__ import annotations

import os

import numpy as np
import torch

# Tolerance on max|y - y_ref| / max|y_ref| per compute dtype.
TOL = {torch.float32: 1e-4, torch.float16: 1e-2, torch.bfloat16: 1e-2}
GRADS = ("grad_input", "grad_offset", "grad_mask", "grad_weight", "grad_bias")


def rel_err(a, ref) -> float:
    if isinstance(a, torch.Tensor):
        a = a.detach().cpu().double().numpy()
    if isinstance(ref, torch.Tensor):
        ref = ref.detach().cpu().double().numpy()
    a = np.asarray(a, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert a.shape == ref.shape, (a.shape, ref.shape)
    den = float(np.abs(ref).max()) if ref.size else 0.0
    if ref.size == 0:
        return 0.0
    return float(np.abs(a - ref).max()) / (den if den > 0 else 1.0)


def load_fixture(path):
    d = np.load(path, allow_pickle=False)
    s, p, dl, G = (int(v) for v in d["geometry"])
    arrays = {k: torch.from_numpy(d[k]) for k in d.files if k != "geometry"}
    return arrays, dict(stride=s, padding=p, dilation=dl, deformable_groups=G)


# Every GPU parity comparison (test id, tensor, max relative error, tolerance),
# written to $DCN2_PARITY_LOG as JSON at the end of the session when that is
# set (tests/conftest.py), so the margins of a run can be tabulated.
PARITY_LOG: list = []


def record(name: str, err: float, tol: float) -> None:
    test = os.environ.get("PYTEST_CURRENT_TEST", "?").split(" ")[0]
    PARITY_LOG.append({"test": test, "tensor": name, "rel_err": err, "tol": tol})


def check(name, got, ref, tol):
    """Asserts max|got - ref| / max|ref| <= tol, printing and recording it."""
    e = rel_err(got, ref)
    record(name, e, tol)
    print(f"  {name}: rel_err={e:.3e} (tol {tol:.0e})")
    assert e <= tol, f"{name}: {e:.3e} > {tol:.0e}"
