"""Shared helpers for the parity tests (GPU result vs the CPU oracle)."""
from __future__ import annotations

import numpy as np


def tol(K: int, amax: float, bmax: float) -> float:
    """max |err| <= 1e-5·√K·max|A|·max|B| (the parity bound for fp32 GEMM)."""
    return 1e-5 * (max(K, 1) ** 0.5) * float(amax) * float(bmax)


def assert_close(got: np.ndarray, want: np.ndarray, K: int, amax: float, bmax: float,
                 what: str = "", extra: float = 0.0) -> float:
    """Assert the GEMM parity bound; `extra` adds room for a fused bias/beta term."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = float(np.max(np.abs(got - want))) if got.size else 0.0
    bound = tol(K, amax, bmax) + extra
    print(f"[parity] {what}: max|err|={err:.3e} bound={bound:.3e}", flush=True)
    assert err <= bound, f"{what}: max|err| {err:.3e} > {bound:.3e}"
    return err


def amax(*arrays) -> float:
    return max(float(np.max(np.abs(a))) if a.size else 0.0 for a in arrays)
