"""The parity bars, written once and used by every GPU test.

- fp32 GEMM: |got - want| <= 1e-4 * max(1, |want|) elementwise (the
  reference conformance rule, scripts/tools/vx_xpu_conformance.cpp:433-436,
  with the north star's 1e-4).
- bf16 GEMM and attention: max |got - want| <= 2e-2 after f32 accumulation.
- int8 GEMV: |got - want| <= 1e-4 * max(1, |want|) against the f64 value.
- Sum invariant for a GEMM too large to check entry by entry:
  sum(C) = sum_k colsum(A)_k * rowsum(B)_k (reference
  scripts/tools/vx_xpu_conformance.cpp:995-1017).
"""

from __future__ import annotations

import numpy as np

FP32_REL = 1e-4
BF16_ABS = 2e-2
GEMV_REL = 1e-4


def assert_rel(got: np.ndarray, want: np.ndarray, tol: float, what: str = "") -> None:
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    bad = np.abs(got - want) > tol * np.maximum(1.0, np.abs(want))
    bad |= ~np.isfinite(got)
    if bad.any():
        idx = np.argwhere(bad)[0]
        raise AssertionError(f"{what}: {int(bad.sum())} entries off; first at {tuple(idx)}: "
                             f"got {got[tuple(idx)]!r} want {want[tuple(idx)]!r}")


def assert_max_abs(got: np.ndarray, want: np.ndarray, tol: float, what: str = "") -> float:
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    err = np.abs(got - want)
    worst = float(np.nanmax(err)) if err.size else 0.0
    if not np.isfinite(got).all() or worst > tol:
        raise AssertionError(f"{what}: max abs error {worst} > {tol}")
    return worst


def sum_invariant(a: np.ndarray, b: np.ndarray) -> float:
    """sum(A B) from A's column sums and B's row sums, in f64."""
    return float(a.astype(np.float64).sum(axis=0) @ b.astype(np.float64).sum(axis=1))
