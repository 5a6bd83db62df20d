"""Device-resident active support of one hierarchy level.

The role of ``gpu_resident/support.py:15-138`` in the reference. Edges are int64 keys row * m + col kept sorted
(unique), with fp64 flows and a "structural" flag for the northwest-corner basis edges that pruning must keep.
Restricted LPs run in the HIP Halpern-PDHG (``hm_pdhg_solve``); costs come from the HIP pair-cost kernels.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from ..config import POSITIVE_SUPPORT_TOLERANCE
from ..lp import NativeRestrictedOTPDLP


def normalize_masses(a: torch.Tensor, b: torch.Tensor):
    """Normalise both marginals to sum 1 and move the total-mass roundoff onto the largest entry of the lighter
    side, twice (gpu_resident/support.py:15-25)."""
    a, b = a / a.sum(), b / b.sum()
    for _ in range(2):
        gap = a.sum() - b.sum()
        a[a.argmax()] -= gap.clamp_max(0)
        b[b.argmax()] += gap.clamp_min(0)
    return a, b


def northwest(a: torch.Tensor, b: torch.Tensor):
    """Northwest-corner basis (n + m - 1 edges, degenerate zero-flow edges kept) from the merged cumulative
    boundaries of the two marginals (gpu_resident/support.py:28-42): sorting the n - 1 source and m - 1 target
    boundaries, each boundary steps the row (source) or the column (target); the flow of an edge is the gap
    between consecutive boundaries."""
    n, m, device = len(a), len(b), a.device
    bounds = torch.cat((a.cumsum(0)[:-1], b.cumsum(0)[:-1]))
    order = torch.argsort(bounds, stable=True)
    is_source = order < n - 1
    zero = torch.zeros(1, dtype=torch.int64, device=device)
    rows = torch.cat((zero, is_source.long().cumsum(0)))
    cols = torch.cat((zero, (~is_source).long().cumsum(0)))
    edges = torch.cat((torch.zeros(1, dtype=torch.float64, device=device), bounds[order], a.sum().reshape(1)))
    return rows * m + cols, edges.diff().clamp_min(0)


@dataclass
class Support:
    keys: torch.Tensor
    values: torch.Tensor
    structural: torch.Tensor
    n: int
    m: int

    @classmethod
    def initial(cls, candidates: torch.Tensor, a: torch.Tensor, b: torch.Tensor) -> "Support":
        """Candidates plus the northwest-corner basis carrying the northwest flows."""
        nw, flows = northwest(a, b)
        keys = torch.unique(torch.cat((candidates, nw)), sorted=True)
        values = torch.zeros(len(keys), dtype=torch.float64, device=a.device)
        structural = torch.zeros(len(keys), dtype=torch.bool, device=a.device)
        positions = torch.searchsorted(keys, nw)
        values.index_add_(0, positions, flows)
        structural[positions] = True
        return cls(keys, values, structural, len(a), len(b))

    def rows_cols(self):
        return torch.div(self.keys, self.m, rounding_mode="floor"), self.keys.remainder(self.m)

    def extend(self, candidates: torch.Tensor) -> torch.Tensor:
        """Add candidate keys (zero flow); returns the mask of new entries."""
        keys = torch.unique(torch.cat((self.keys, candidates)), sorted=True)
        old = torch.searchsorted(keys, self.keys)
        values = torch.zeros(len(keys), dtype=torch.float64, device=keys.device)
        structural = torch.zeros(len(keys), dtype=torch.bool, device=keys.device)
        fresh = torch.ones(len(keys), dtype=torch.bool, device=keys.device)
        values[old], structural[old], fresh[old] = self.values, self.structural, False
        self.keys, self.values, self.structural = keys, values, structural
        return fresh

    def prune(self, cost, dual: torch.Tensor, fresh: torch.Tensor, budget: int) -> torch.Tensor:
        """Budgeted pruning (refinement/budgeted_pruning.py:27-58): when the support exceeds the budget, drop the
        old, non-structural, zero-flow edges with the largest reduced cost. Returns the removed keys."""
        remove = max(0, len(self.keys) - budget)
        if not remove:
            return self.keys[:0]
        rows, cols = self.rows_cols()
        eligible = (~self.structural) & (~fresh) & (self.values.abs() <= POSITIVE_SUPPORT_TOLERANCE)
        candidates = torch.nonzero(eligible).flatten()
        if len(candidates) < remove:
            raise RuntimeError("GPU budgeted pruning has insufficient old zero-flow edges")
        rr, cc = rows[candidates], cols[candidates]
        reduced = cost.pairs(rr, cc) - dual[rr] - dual[self.n + cc]
        removed = candidates[torch.argsort(reduced, descending=True, stable=True)[:remove]]
        removed_keys = self.keys[removed]
        keep = torch.ones(len(self.keys), dtype=torch.bool, device=self.keys.device)
        keep[removed] = False
        self.keys, self.values, self.structural = self.keys[keep], self.values[keep], self.structural[keep]
        return removed_keys

    def solve_lp(self, cost, a: torch.Tensor, b: torch.Tensor, dual: torch.Tensor, tolerance: float):
        """Restricted LP on the support, warm-started from the current flows and duals."""
        rows, cols = self.rows_cols()
        costs = cost.pairs(rows, cols)
        solver = NativeRestrictedOTPDLP(device=a.device, evaluation_frequency=200)
        result = solver.solve_restricted(rows=rows, cols=cols, costs=costs, source_mass=a, target_mass=b,
                                         warm_start_primal=self.values, warm_start_dual=dual, tolerance=tolerance)
        if not result.success:
            raise RuntimeError(f"GPU restricted LP failed: {result.termination_reason}")
        self.values = result.x
        result.obj_val = float(costs @ result.x)
        return result.y, result


__all__ = ["Support", "normalize_masses", "northwest"]
