"""The reference's error metrics and NaN-aware gates (test infrastructure).

* FP8 convention (``examples/fp8-gemm/v002_dense_tp8_validated_065.cu:345-360``,
  ``examples/fp8-group-gemm/v007_dsv3_decode_verified_105.cu:545-551``):
  ``err = |g - r| / max(|r|, 1e-3 * max|r|)``; any NaN/Inf fails
  (``tasks/kimi-moe-w13-int4-grouped-gemm.yaml:171-184``).
* decode-linear convention (``v019_swapab_cg2_l2hints.cu:654-660``):
  ``|g - r| / max(|r|, |g|, 1)``.
* Kimi absolute gate ``max|g - r| < 0.012``
  (``tasks/kimi-moe-w13-int4-grouped-gemm.yaml:161``).
"""
from __future__ import annotations

import numpy as np


def fp8_rel_err(got: np.ndarray, ref: np.ndarray) -> tuple[float, int]:
    """Return (max relative error, count of non-finite values in got or ref)."""
    g = np.asarray(got, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    bad = ~(np.isfinite(g) & np.isfinite(r))
    nbad = int(bad.sum())
    if g.size == 0:
        return 0.0, nbad
    rf = np.where(bad, 0.0, r)
    max_abs = float(np.abs(rf).max()) if rf.size else 0.0
    denom = np.maximum(np.abs(rf), 1e-3 * max_abs)
    denom = np.where(denom == 0, 1.0, denom)
    e = np.where(bad, 0.0, np.abs(np.where(bad, 0.0, g) - rf) / denom)
    return float(e.max()), nbad


def linear_rel_err(got: np.ndarray, ref: np.ndarray) -> tuple[float, int]:
    g = np.asarray(got, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    bad = ~(np.isfinite(g) & np.isfinite(r))
    g0 = np.where(bad, 0.0, g)
    r0 = np.where(bad, 0.0, r)
    e = np.abs(g0 - r0) / np.maximum(np.maximum(np.abs(r0), np.abs(g0)), 1.0)
    return (float(e.max()) if e.size else 0.0), int(bad.sum())


def max_abs_err(got: np.ndarray, ref: np.ndarray) -> tuple[float, int]:
    g = np.asarray(got, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    bad = ~(np.isfinite(g) & np.isfinite(r))
    d = np.where(bad, 0.0, np.abs(g - r))
    return (float(d.max()) if d.size else 0.0), int(bad.sum())


def gate_fp8(got, ref, tol: float = 1e-2) -> bool:
    e, nbad = fp8_rel_err(got, ref)
    return nbad == 0 and e < tol
