"""Shared checks for the parity tests."""
from __future__ import annotations

import sys

import numpy as np

# Tolerance of every f32 GEMM / GEMV output against the float64 oracle:
# normwise  max_i |y_i - ref_i| / max_i |ref_i| <= 1e-3.
NORMWISE_TOL = 1e-3


def normwise_err(got, ref) -> float:
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    denom = np.abs(ref).max() if ref.size else 1.0
    if denom == 0.0:
        return float(np.abs(got).max()) if got.size else 0.0
    return float(np.abs(got - ref).max() / denom)


def assert_close(got, ref, tol: float = NORMWISE_TOL, what: str = "") -> float:
    got = np.asarray(got, dtype=np.float64)
    assert np.isfinite(got).all(), f"{what}: non-finite output (unwritten or overflow)"
    err = normwise_err(got, ref)
    assert err <= tol, f"{what}: normwise error {err:.3e} > {tol:.1e}"
    return err


def note(msg: str) -> None:
    """Name the case on stdout before a GPU step (flushed)."""
    print(msg, flush=True)
    sys.stdout.flush()
