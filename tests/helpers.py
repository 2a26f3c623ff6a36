"""Shared checks for the parity tests."""
from __future__ import annotations

import numpy as np

from xllms_amd import workloads as W

# Tolerances stated by the task for this path.
FP32_REL = 1e-5          # per (seq, head): max|g - r| <= 1e-5 * max|r|
HALF_ATOL = 2e-3         # fp16 / bf16: |g - r| <= atol + rtol*|r|, elementwise
HALF_RTOL = 1e-2


def assert_close(got: np.ndarray, ref: np.ndarray, kv_dtype: int, what: str = "") -> dict:
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err = np.abs(got - ref)
    stats = {"max_abs": float(err.max(initial=0.0))}
    if kv_dtype == W.FP32:
        scale = np.abs(ref).max(axis=-1, keepdims=True)
        rel = err.max(axis=-1, keepdims=True) / np.maximum(scale, 1e-30)
        rel = np.where(scale > 0, rel, err.max(axis=-1, keepdims=True))
        stats["max_rel_row"] = float(rel.max(initial=0.0))
        assert stats["max_rel_row"] <= FP32_REL, f"{what}: fp32 rel error {stats}"
    else:
        bound = HALF_ATOL + HALF_RTOL * np.abs(ref)
        bad = err > bound
        stats["violations"] = int(bad.sum())
        stats["max_excess"] = float((err / bound).max(initial=0.0))
        assert not bad.any(), f"{what}: {stats['violations']} elements out of tolerance {stats}"
    return stats
