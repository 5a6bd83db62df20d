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
from .sparsify import sparsify_transport_support


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
    last_sparsification: object = None
    sparsification_log: list | None = None

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

    def solve_lp(self, cost, a: torch.Tensor, b: torch.Tensor, dual: torch.Tensor, tolerance: float,
                 primal_cap: int | None = None):
        """Restricted LP on the support, warm-started from the current flows and duals. When the solution keeps
        more than ``primal_cap`` positive edges, its support is sparsified by cycle cancelling (cost never
        increases) and the duals are shifted down by half the new primal-dual gap per unit mass, as the reference
        does (gpu_resident/support.py:121-137). ``self.last_sparsification`` holds that step's result or None."""
        rows, cols = self.rows_cols()
        costs = cost.pairs(rows, cols)
        solver = NativeRestrictedOTPDLP(device=a.device, evaluation_frequency=200)
        result = solver.solve_restricted(rows=rows, cols=cols, costs=costs, source_mass=a, target_mass=b,
                                         warm_start_primal=self.values, warm_start_dual=dual, tolerance=tolerance)
        if not result.success:
            raise RuntimeError(f"GPU restricted LP failed: {result.termination_reason}")
        self.values = result.x
        result.obj_val = float(costs @ result.x)
        dual = result.y
        self.last_sparsification = None
        if primal_cap is not None and int(torch.count_nonzero(self.values > POSITIVE_SUPPORT_TOLERANCE)) > primal_cap:
            sparse = sparsify_transport_support(rows.cpu().numpy(), cols.cpu().numpy(), self.values.cpu().numpy(),
                                                costs.cpu().numpy(), n_source=self.n, n_target=self.m,
                                                target_nnz=primal_cap)
            self.values = torch.as_tensor(sparse.values, device=a.device)
            self.last_sparsification = sparse
            result.x = self.values
            result.obj_val = float(costs @ self.values)
            rhs = torch.cat((a, b))
            shift = ((rhs @ dual - result.obj_val) / a.sum()).clamp_min(0)
            dual = dual - 0.5 * shift
            result.y = dual
            result.dual_obj_val = float(rhs @ dual)
            result.gap = abs(result.obj_val - result.dual_obj_val) / (1 + abs(result.obj_val) + abs(result.dual_obj_val))
        return dual, result


__all__ = ["Support", "normalize_masses", "northwest"]
