"""Support sparsification of a restricted-OT primal: ``sparsify_transport_support``.

Same signature, validation and result as the reference's routine (``restricted_ot/support_sparsification.py:13-145``,
engine ``"cpp_lct"``), run by ``hm_sparsify_support`` in the native library: cycle cancelling on the host over a
parent-pointer spanning forest with eager flow updates (the reference uses a link-cut tree on its CPU; the
GPU-resident reference solver exports the support to host memory for this step, ``gpu_resident/support.py:124-137``).
The solver calls it only when an LP leaves more positive edges than the support cap allows.
"""
from __future__ import annotations

import ctypes
import time
from dataclasses import dataclass

import numpy as np

from .. import _lib
from ..config import POSITIVE_SUPPORT_TOLERANCE


@dataclass(frozen=True)
class SupportSparsificationResult:
    values: np.ndarray
    input_nnz: int
    output_nnz: int
    target_nnz: int
    cycle_updates: int
    tree_operations: int
    wall_time: float

    @property
    def positive_mask(self) -> np.ndarray:
        return self.values > 0.0


def sparsify_transport_support(rows, cols, values, costs, *, n_source: int, n_target: int, target_nnz: int,
                               zero_tolerance: float = POSITIVE_SUPPORT_TOLERANCE) -> SupportSparsificationResult:
    """Cancel support cycles in non-increasing-cost directions until the positive support reaches the target."""
    n_source, n_target, target_nnz = int(n_source), int(n_target), int(target_nnz)
    zero_tolerance = float(zero_tolerance)
    if n_source <= 0 or n_target <= 0:
        raise ValueError("n_source and n_target must be positive")
    if target_nnz < n_source + n_target - 1:
        raise ValueError("target_nnz must be at least n_source + n_target - 1")
    if not np.isfinite(zero_tolerance) or zero_tolerance < 0.0:
        raise ValueError("zero_tolerance must be finite and nonnegative")
    rows = np.ascontiguousarray(rows, dtype=np.int64).reshape(-1)
    cols = np.ascontiguousarray(cols, dtype=np.int64).reshape(-1)
    out = np.array(values, dtype=np.float64).reshape(-1)
    costs = np.ascontiguousarray(costs, dtype=np.float64).reshape(-1)
    e = rows.size
    if cols.size != e or out.size != e or costs.size != e:
        raise ValueError("rows, cols, values, and costs must have equal lengths")
    if np.any(rows < 0) or np.any(rows >= n_source):
        raise ValueError("rows contain an out-of-range source index")
    if np.any(cols < 0) or np.any(cols >= n_target):
        raise ValueError("cols contain an out-of-range target index")
    if not np.all(np.isfinite(out)) or np.any(out < -zero_tolerance):
        raise ValueError("values must be finite and nonnegative up to zero_tolerance")
    if not np.all(np.isfinite(costs)):
        raise ValueError("costs must be finite")
    input_nnz = int(np.count_nonzero(out > zero_tolerance))
    stats = np.zeros(3, dtype=np.int64)
    started = time.perf_counter()
    p = lambda a: ctypes.c_void_p(a.ctypes.data)  # noqa: E731
    rc = _lib.load().hm_sparsify_support(n_source, n_target, e, p(rows), p(cols), p(out), p(costs), target_nnz,
                                         zero_tolerance, p(stats))
    _lib.check(rc, "hm_sparsify_support")
    return SupportSparsificationResult(out, input_nnz, int(stats[0]), target_nnz, int(stats[1]), int(stats[2]),
                                       float(time.perf_counter() - started))


__all__ = ["SupportSparsificationResult", "sparsify_transport_support"]
