"""Exact solve of the coarsest hierarchy level (the role of POT's ``emd`` in ``gpu_resident/solver.py:168-191``).

The level has at most ``coarsest_size_threshold`` points per side, so its dense cost matrix is small: it is
evaluated on the device by the same pair-cost kernels the refinement uses, copied to the host, and solved exactly by
``hm_transport_simplex`` (primal network simplex, host code of the native library). The plan's entries above 1e-12
become the level's support and the simplex duals (u, v) seed the next level, as the reference keeps
``plan > 1e-12`` and ``log["u"], log["v"]``.
"""
from __future__ import annotations

import ctypes
import time

import numpy as np
import torch

from .. import _lib
from ..types import CoarsestSolveStats, LevelResult
from .support import ActiveSet

PLAN_THRESHOLD = 1e-12
MAX_PIVOTS = 10_000_000


def transport_simplex(costs: np.ndarray, a: np.ndarray, b: np.ndarray, max_pivots: int = MAX_PIVOTS):
    """Exact optimal basic plan and duals of a dense balanced transport problem (host arrays).

    Returns (rows, cols, flows, u, v, pivots): the basic transport arcs (degenerate zero flows included) and duals
    with u_i + v_j = c_ij on them and u_i + v_j <= c_ij (to 1e-12 of the cost scale) on every pair."""
    costs = np.ascontiguousarray(costs, dtype=np.float64)
    a = np.ascontiguousarray(a, dtype=np.float64).reshape(-1)
    b = np.ascontiguousarray(b, dtype=np.float64).reshape(-1)
    n, m = costs.shape
    if a.size != n or b.size != m:
        raise ValueError("masses must match the cost matrix shape")
    rows = np.empty(n + m, np.int32)
    cols = np.empty(n + m, np.int32)
    flows = np.empty(n + m, np.float64)
    count = np.zeros(1, np.int64)
    u = np.empty(n, np.float64)
    v = np.empty(m, np.float64)
    pivots = np.zeros(1, np.int64)
    p = lambda x: ctypes.c_void_p(x.ctypes.data)  # noqa: E731
    rc = _lib.load().hm_transport_simplex(n, m, p(costs), p(a), p(b), int(max_pivots), p(rows), p(cols), p(flows),
                                          p(count), p(u), p(v), p(pivots))
    _lib.check(rc, "hm_transport_simplex")
    k = int(count[0])
    return rows[:k], cols[:k], flows[:k], u, v, int(pivots[0])


def solve_coarsest(cost, a: torch.Tensor, b: torch.Tensor, level_index: int):
    """Exact coarsest level: (support, duals, LevelResult)."""
    started = time.perf_counter()
    n, m = cost.shape
    dev = a.device
    rows = torch.arange(n, device=dev).repeat_interleave(m)
    cols = torch.arange(m, device=dev).repeat(n)
    matrix = cost.pairs(rows, cols).view(n, m).cpu().numpy()
    r, c, x, u, v, _ = transport_simplex(matrix, a.cpu().numpy(), b.cpu().numpy())
    keep = x > PLAN_THRESHOLD
    r, c, x = r[keep], c[keep], x[keep]
    objective = float(matrix[r, c] @ x)
    support = ActiveSet.from_plan(torch.as_tensor(r, device=dev), torch.as_tensor(c, device=dev),
                                  torch.as_tensor(x, device=dev), n, m)
    dual = torch.as_tensor(np.concatenate((u, v)), device=dev)
    elapsed = time.perf_counter() - started
    level = LevelResult(level_index, "coarsest", n, m, None, CoarsestSolveStats(elapsed, objective, len(support)),
                        elapsed)
    return support, dual, level


__all__ = ["solve_coarsest", "transport_simplex"]
