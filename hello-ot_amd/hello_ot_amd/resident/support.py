"""Device-resident active support of one hierarchy level (the role of ``gpu_resident/support.py:15-138``).

Layout. The support is a sorted set of int64 edge keys ``row * n_target + col`` -- row-major, so the edge list is
already in the source order the PDHG's first pass walks -- with three per-edge columns: the fp64 flow, a ``pinned``
flag for the northwest-corner basis edges that pruning must keep, and ``born``, the refinement iteration that added
the edge (-1 for the initial support). Everything stays on the device; only the support sparsifier, a host
algorithm, sees host copies.

Updates never re-sort the whole set. New candidate keys arrive sorted and unique; ``absorb`` drops those already
present and interleaves the rest by rank: with ``searchsorted`` in both directions, every old edge moves up by the
number of new keys below it and every new key lands at its own index plus the number of old keys below it, so the
merge is two binary searches and two scatters instead of a sort of the union.
"""
from __future__ import annotations

import torch

from ..config import POSITIVE_SUPPORT_TOLERANCE
from .. import _lib
from ..lp import NativeRestrictedOTPDLP
from .sparsify import sparsify_transport_support


def balanced_masses(a: torch.Tensor, b: torch.Tensor):
    """Both marginals scaled to total 1, then the leftover total-mass mismatch (fp roundoff) added twice to the
    largest entry of the lighter side (the level masses of ``gpu_resident/support.py:15-25``)."""
    a = a / a.sum()
    b = b / b.sum()
    for _ in range(2):
        excess = a.sum() - b.sum()                 # > 0: targets are light; < 0: sources are light
        a[a.argmax()] += torch.clamp(-excess, min=0.0)
        b[b.argmax()] += torch.clamp(excess, min=0.0)
    return a, b


def staircase(a: torch.Tensor, b: torch.Tensor):
    """Northwest-corner basis of the transport polytope (``gpu_resident/support.py:28-42``): its n + m - 1 edges,
    including degenerate zero-flow ones, as keys and flows.

    The interior cumulative boundaries of the two marginals, merged into one increasing sequence (a source boundary
    before an equal target boundary), cut [0, total] into n + m - 1 pieces; piece t is the edge (number of source
    boundaries before it, number of target boundaries before it) and carries the piece's length. The merged
    position of each boundary is its own index plus the count of the other side's boundaries strictly below it
    (source) or at or below it (target)."""
    n, m, dev = a.numel(), b.numel(), a.device
    sa, sb = a.cumsum(0)[:-1], b.cumsum(0)[:-1]
    at_a = torch.arange(n - 1, device=dev) + torch.searchsorted(sb, sa, right=False)
    at_b = torch.arange(m - 1, device=dev) + torch.searchsorted(sa, sb, right=True)
    cuts = torch.empty(n + m, dtype=torch.float64, device=dev)
    cuts[0] = 0.0
    cuts[-1] = a.sum()
    cuts[1 + at_a] = sa
    cuts[1 + at_b] = sb
    source_cut = torch.zeros(n + m - 1, dtype=torch.int64, device=dev)
    source_cut[1 + at_a] = 1
    row = source_cut.cumsum(0)
    col = torch.arange(n + m - 1, device=dev) - row
    return row * m + col, (cuts[1:] - cuts[:-1]).clamp_min(0.0)


def _member(sorted_keys: torch.Tensor, queries: torch.Tensor) -> torch.Tensor:
    """Mask of the queries found in a sorted key set."""
    if sorted_keys.numel() == 0:
        return torch.zeros(queries.numel(), dtype=torch.bool, device=queries.device)
    at = torch.searchsorted(sorted_keys, queries).clamp_max(sorted_keys.numel() - 1)
    return sorted_keys[at] == queries


class ActiveSet:
    """Sorted edge keys with per-edge flow, pinned flag and birth iteration."""

    def __init__(self, keys, flow, pinned, born, n_source: int, n_target: int):
        self.keys, self.flow, self.pinned, self.born = keys, flow, pinned, born
        self.n_source, self.n_target = int(n_source), int(n_target)
        self.last_sparsification = None
        self.sparsification_log = []

    # -- construction -----------------------------------------------------------------------------------
    @classmethod
    def seeded(cls, candidates: torch.Tensor, a: torch.Tensor, b: torch.Tensor) -> "ActiveSet":
        """The staircase basis (pinned, carrying its flows) plus sorted unique candidate keys at zero flow."""
        basis, flows = staircase(a, b)      # distinct keys, already increasing: row and column never decrease
        dev = a.device
        support = cls(basis, flows, torch.ones(basis.numel(), dtype=torch.bool, device=dev),
                      torch.full((basis.numel(),), -1, dtype=torch.int32, device=dev), a.numel(), b.numel())
        support.absorb(candidates, born=-1)
        return support

    @classmethod
    def from_plan(cls, rows, cols, flows, n_source: int, n_target: int) -> "ActiveSet":
        """A support holding a given plan (nothing pinned)."""
        keys = rows.long() * int(n_target) + cols.long()
        order = torch.argsort(keys)
        keys, flows = keys[order], flows[order].double()
        dev = keys.device
        return cls(keys, flows, torch.zeros(keys.numel(), dtype=torch.bool, device=dev),
                   torch.full((keys.numel(),), -1, dtype=torch.int32, device=dev), n_source, n_target)

    # -- views ------------------------------------------------------------------------------------------
    def __len__(self) -> int:
        return int(self.keys.numel())

    def endpoints(self):
        return torch.div(self.keys, self.n_target, rounding_mode="floor"), self.keys.remainder(self.n_target)

    # -- updates ----------------------------------------------------------------------------------------
    def absorb(self, candidates: torch.Tensor, *, born: int) -> torch.Tensor:
        """Merge sorted unique candidate keys (zero flow, stamped ``born``); returns the keys that were new."""
        new = candidates[~_member(self.keys, candidates)]
        if new.numel() == 0:
            return new
        old_count, dev = self.keys.numel(), self.keys.device
        to_old = torch.arange(old_count, device=dev) + torch.searchsorted(new, self.keys)
        to_new = torch.arange(new.numel(), device=dev) + torch.searchsorted(self.keys, new)
        total = old_count + new.numel()
        keys = torch.empty(total, dtype=torch.int64, device=dev)
        flow = torch.zeros(total, dtype=torch.float64, device=dev)
        pinned = torch.zeros(total, dtype=torch.bool, device=dev)
        stamp = torch.full((total,), int(born), dtype=torch.int32, device=dev)
        keys[to_old], keys[to_new] = self.keys, new
        flow[to_old], pinned[to_old], stamp[to_old] = self.flow, self.pinned, self.born
        self.keys, self.flow, self.pinned, self.born = keys, flow, pinned, stamp
        return new

    def trim(self, cost, dual: torch.Tensor, budget: int, iteration: int) -> torch.Tensor:
        """Budgeted pruning (``refinement/budgeted_pruning.py:27-58``): past the budget, remove that many edges among
        those that are neither pinned nor added in this iteration and carry no flow, largest reduced cost
        c_ij - f_i - g_j first, equal reduced costs in key order. Returns the removed keys (sorted).

        The selection takes the ``excess`` largest reduced costs with a partial top-k, then settles the ties at the
        threshold by position."""
        excess = len(self) - int(budget)
        if excess <= 0:
            return self.keys[:0]
        idle = (~self.pinned) & (self.born < iteration) & (self.flow.abs() <= POSITIVE_SUPPORT_TOLERANCE)
        slots = torch.nonzero(idle).flatten()
        if slots.numel() < excess:
            raise RuntimeError("GPU budgeted pruning has insufficient old zero-flow edges")
        rows, cols = self.endpoints()
        r, c = rows[slots], cols[slots]
        reduced = cost.pairs(r, c) - dual[r] - dual[self.n_source + c]
        threshold = torch.topk(reduced, excess, largest=True, sorted=False).values.min()
        above = reduced > threshold
        tied = torch.nonzero(reduced == threshold).flatten()
        take = torch.cat((torch.nonzero(above).flatten(), tied[: excess - int(above.sum())]))
        drop = slots[take]
        keep = torch.ones(len(self), dtype=torch.bool, device=self.keys.device)
        keep[drop] = False
        removed = self.keys[drop].sort().values
        self.keys, self.flow, self.pinned, self.born = (self.keys[keep], self.flow[keep], self.pinned[keep],
                                                        self.born[keep])
        return removed

    # -- restricted LP ----------------------------------------------------------------------------------
    def solve_lp(self, cost, a: torch.Tensor, b: torch.Tensor, dual: torch.Tensor, tolerance: float,
                 primal_cap: int | None = None):
        """Restricted LP on the support, warm-started from the current flows and duals (HIP Halpern-PDHG).

        When the solution keeps more than ``primal_cap`` positive edges, its positive support is thinned by cycle
        cancelling on the host (cost never increases), and the duals are lowered by half the primal-dual gap that
        leaves per unit of source mass, so that the reported gap stays consistent
        (``gpu_resident/support.py:121-137``). ``last_sparsification`` records that step (or None)."""
        rows, cols = self.endpoints()
        costs = cost.pairs(rows, cols)
        solver = NativeRestrictedOTPDLP(device=a.device, evaluation_frequency=200)
        passes = _lib.profile_query("pdhg_iteration") if _lib.profiling() else None
        result = solver.solve_restricted(rows=rows, cols=cols, costs=costs, source_mass=a, target_mass=b,
                                         warm_start_primal=self.flow, warm_start_dual=dual, tolerance=tolerance)
        if passes is not None:
            # with the library's kernel timing on: the iterations' own device time (no pair costs, no set-up)
            ms, count = _lib.profile_query("pdhg_iteration")
            result.solver_diag["pdhg_pass_ms"] = ms - passes[0]
            result.solver_diag["pdhg_passes"] = count - passes[1]
        if not result.success:
            raise RuntimeError(f"GPU restricted LP failed: {result.termination_reason}")
        self.flow = result.x
        result.obj_val = float(costs @ self.flow)
        dual = result.y
        self.last_sparsification = None
        positive = int(torch.count_nonzero(self.flow > POSITIVE_SUPPORT_TOLERANCE))
        if primal_cap is None or positive <= primal_cap:
            return dual, result
        thinned = sparsify_transport_support(rows.cpu().numpy(), cols.cpu().numpy(), self.flow.cpu().numpy(),
                                             costs.cpu().numpy(), n_source=self.n_source, n_target=self.n_target,
                                             target_nnz=primal_cap)
        self.flow = torch.as_tensor(thinned.values, device=a.device)
        self.last_sparsification = thinned
        self.sparsification_log.append(thinned)
        primal = float(costs @ self.flow)
        masses = torch.cat((a, b))
        gap_per_mass = torch.clamp((masses @ dual - primal) / a.sum(), min=0.0)
        dual = dual - 0.5 * gap_per_mass
        dual_objective = float(masses @ dual)
        result.x, result.y = self.flow, dual
        result.obj_val, result.dual_obj_val = primal, dual_objective
        result.gap = abs(primal - dual_objective) / (1.0 + abs(primal) + abs(dual_objective))
        return dual, result


__all__ = ["ActiveSet", "balanced_masses", "staircase"]
