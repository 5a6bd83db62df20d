"""HELLO driver on the device: hierarchy chain, exact coarsest level, and per-level seeding and refinement.

What each level does is HELLO's algorithm as the reference's GPU-resident solver runs it
(``gpu_resident/solver.py:27-398``):

* one global shuffle per side (``hierarchy/plan.py:73-87``); level l keeps the first n_l source and m_l target
  points; going coarser, the larger side is divided by ``split_count`` until both fit ``coarsest_size_threshold``;
* the coarsest level is solved exactly (network simplex, ``resident/leaf.py``), as the reference does with POT's
  ``emd`` (``gpu_resident/solver.py:168-191``);
* each finer level inherits the duals of the side it shares with the coarser level and completes the other side
  by a c-transform (a directional top-1 scan); both directions' ``assignment_topk`` best pairs plus the
  northwest-corner basis seed the support; then the refinement loop runs ``LP -> pricing scan with certificate ->
  add violated pairs -> budgeted pruning`` until the relative dual infeasibility is at most the tolerance.

Cost perturbation (``cost_perturbation="auto"``) is detected as the reference detects it (a pruned edge coming back)
but not applied: the level keeps refining on the original cost and the trigger is recorded.

The refinement is a small state machine (``LevelRefinement``): ``seed`` builds the support and duals, ``step`` runs
one iteration and returns its record, ``run`` loops and assembles the level result.
"""
from __future__ import annotations

import sys
import time

import numpy as np
import torch

from ..config import active_support_budget, level_stopping_norm, primal_support_cap
from ..types import (ActiveSupportStats, BudgetedPruningStats, ConvergenceStats, DualViolationStats,
                     HelloSolveError, InitializationStats, IterationStats, LevelResult, RefinementResult,
                     RefinementSummary, SolveLPStats)
from .cost import Cost
from .support import ActiveSet


def derive_hierarchy_seeds(seed: int, num_children: int):
    """Source-split, target-split and child seeds of a hierarchy node (hierarchy/utilities.py:56-65)."""
    rng = np.random.default_rng(int(seed))
    draws = [int(rng.integers(0, 2**31 - 1)) for _ in range(2 + int(num_children))]
    return draws[0], draws[1], draws[2:]


def shuffle_once_permutation(n_source: int, n_target: int, seed: int, split_count: int):
    """One global random permutation per side (hierarchy/plan.py:73-87)."""
    source_seed, target_seed, _ = derive_hierarchy_seeds(seed, split_count)
    return (np.random.default_rng(source_seed).permutation(int(n_source)).astype(np.int64),
            np.random.default_rng(target_seed).permutation(int(n_target)).astype(np.int64))


def level_sizes(n: int, m: int, threshold: int, split: int):
    """Finest-first chain of (n_l, m_l): the larger side is divided by ``split`` until both fit ``threshold``."""
    sizes = [(n, m)]
    while max(sizes[-1]) > threshold:
        nn, mm = sizes[-1]
        if nn >= mm:
            nn = -(-nn // split)
        else:
            mm = -(-mm // split)
        sizes.append((nn, mm))
    return sizes


def candidate_keys(row_values, row_index, col_values, col_index, dual, n, m, positive=False):
    """Sorted unique keys row * m + col of the pairs the scans proposed (gpu_resident/solver.py:27-35).

    ``row_index[i]`` lists the columns proposed for source row i and ``col_index[j]`` the rows proposed for target
    column j (-1 = empty slot). The stored values exclude the row's own dual (a row list holds g_j - c_ij, a
    column list f_i - c_ij), so with ``positive`` a pair is kept only when adding that dual back gives a violated
    pair, sigma_ij = f_i + g_j - c_ij > 0."""
    pieces = []
    for values, index, own, count, by_row in ((row_values, row_index, dual[:n], n, True),
                                              (col_values, col_index, dual[n:], m, False)):
        if index is None:
            continue
        owner = torch.arange(count, device=dual.device).unsqueeze(1).expand_as(index)
        keep = index >= 0
        if positive:
            keep = keep & ((values + own.unsqueeze(1)) > 0)
        partner = index.long()
        pieces.append(((owner * m + partner) if by_row else (partner * m + owner))[keep])
    return torch.unique(torch.cat(pieces), sorted=True)


def _progress(options, message: str) -> None:
    """A progress line (verbose="detailed"), with the peak device memory of the solve so far."""
    if options.verbose == "detailed":
        peak = torch.cuda.max_memory_allocated() / 2**30
        print(f"[hello-mi355x] {message} peak={peak:.1f}GiB", file=sys.stderr, flush=True)


class _Stopwatch:
    """Wall-clock laps (host time; device work is synchronised by the readbacks the steps already do)."""

    def __init__(self):
        self.origin = self.mark = time.perf_counter()

    def lap(self) -> float:
        now = time.perf_counter()
        elapsed, self.mark = now - self.mark, now
        return elapsed

    def total(self) -> float:
        return time.perf_counter() - self.origin


class LevelRefinement:
    """One refined hierarchy level: seeding from the coarser level's duals, then the refinement iterations."""

    def __init__(self, cost: Cost, a, b, options, index: int, detect_reentry: bool):
        self.cost, self.a, self.b, self.options, self.index = cost, a, b, options, index
        self.n, self.m = cost.shape
        self.detect_reentry = detect_reentry
        self.budget = active_support_budget(options.support_budget_factor, self.n, self.m)
        self.cap = primal_support_cap(options.support_budget_factor, options.pricing_topk, self.n, self.m)
        self.support = None
        self.dual = None
        self.peak = 0
        self.recently_pruned = None       # sorted keys removed by the last pruning
        self.reentry_seen = False         # a pruned edge came back in the last iteration
        self.perturbation_triggered = False
        self.records = []
        self.lp = None
        self.lp_device = {"seconds": 0.0, "iterations": 0}  # hm_pdhg_solve time of the level's LP solves

    # -- seeding ----------------------------------------------------------------------------------------
    def seed(self, previous: torch.Tensor, inherited: str | None) -> InitializationStats:
        """Inherit the shared side's duals, c-transform the other side, gather both directions' best pairs and
        complete them with the northwest basis (gpu_resident/solver.py:38-64)."""
        watch = _Stopwatch()
        n, m, k = self.n, self.m, self.options.assignment_topk
        dual = torch.zeros(n + m, dtype=torch.float64, device=self.a.device)
        rows_best = cols_best = (None, None)
        propagation = 0.0
        if inherited == "target":
            dual[n:] = previous[-m:]
            rows_best = self.cost.scan(dual, k, direction="source")[:2]
            dual[:n] = -rows_best[0][:, 0]          # f_i = min_j (c_ij - g_j)
            propagation = watch.lap()
            _progress(self.options, f"init {n}x{m}: source c-transform scan {propagation:.3f}s")
            cols_best = self.cost.scan(dual, k, direction="target")[2:4]
        elif inherited == "source":
            dual[:n] = previous[:n]
            cols_best = self.cost.scan(dual, k, direction="target")[2:4]
            dual[n:] = -cols_best[0][:, 0]          # g_j = min_i (c_ij - f_i)
            propagation = watch.lap()
            _progress(self.options, f"init {n}x{m}: target c-transform scan {propagation:.3f}s")
            rows_best = self.cost.scan(dual, k, direction="source")[:2]
        else:
            dual = previous.clone()
            both = self.cost.scan(dual, k)
            rows_best, cols_best = both[:2], both[2:4]
        candidates = candidate_keys(*rows_best, *cols_best, dual, n, m)
        assignment = watch.lap()
        self.support = ActiveSet.seeded(candidates, self.a, self.b)
        self.dual = dual
        self.peak = len(self.support)
        torch.cuda.synchronize()
        basis = watch.lap()
        total = watch.total()
        _progress(self.options, f"init {n}x{m}: {len(self.support)} initial edges {total:.3f}s")
        # support sizes as the reference reports them: the forward (row) assignment's n * min(m, k) slots, then the
        # deduplicated union of both directions, then the basis edges that were not already candidates
        return InitializationStats(total, propagation, propagation + assignment, basis, inherited, k,
                                   n * min(m, k), len(candidates), len(self.support) - len(candidates),
                                   len(self.support))

    # -- one iteration ----------------------------------------------------------------------------------
    def step(self, iteration: int) -> bool:
        """LP, pricing with certificate, and (unless converged) support growth and pruning. Returns convergence."""
        options, tol = self.options, self.options.tolerance
        watch = _Stopwatch()
        support = self.support
        size_before = len(support)
        self.dual, lp = support.solve_lp(self.cost, self.a, self.b, self.dual, tol, primal_cap=self.cap)
        self.lp = lp
        lp_seconds = watch.lap()
        diag = lp.solver_diag or {}
        self.lp_device["seconds"] += float(diag.get("device_loop_sec", 0.0))
        self.lp_device["iterations"] += int(lp.iterations)
        if "pdhg_pass_ms" in diag:
            self.lp_device["pass_ms"] = self.lp_device.get("pass_ms", 0.0) + diag["pdhg_pass_ms"]
            self.lp_device["passes"] = self.lp_device.get("passes", 0) + diag["pdhg_passes"]
        thinned = support.last_sparsification
        _progress(options, f"level={self.index} iteration={iteration} lp {lp_seconds:.3f}s support={size_before} "
                           f"pdhg_iters={lp.iterations}"
                           + (f" sparsified {thinned.input_nnz}->{thinned.output_nnz}" if thinned else ""))
        xv, xi, yv, yi, metrics = self.cost.scan(self.dual, options.pricing_topk, certificate=True)
        scan_seconds = watch.lap()
        norm = level_stopping_norm(options.stopping_norm, self.index)   # gpu_resident/solver.py:86, 100
        converged = metrics[norm] <= tol
        if not converged and self.detect_reentry and self.reentry_seen:
            self.perturbation_triggered = True
        grown = size_before
        added = 0
        prune_seconds = 0.0
        if not converged:
            fresh = support.absorb(candidate_keys(xv, xi, yv, yi, self.dual, self.n, self.m, positive=True),
                                   born=iteration)
            added, grown = int(fresh.numel()), len(support)
            if not added:
                raise HelloSolveError("GPU full optimality check failed without new candidate edges")
            self.peak = max(self.peak, grown)
            pruned_before = self.recently_pruned
            self.reentry_seen = pruned_before is not None and bool(_contains_any(pruned_before, fresh))
            watch.lap()
            self.recently_pruned = support.trim(self.cost, self.dual, self.budget, iteration)
            prune_seconds = watch.lap()
        self.records.append(IterationStats(
            iteration, float(lp.obj_val), watch.total(), 0.0, scan_seconds,
            SolveLPStats(lp_seconds, lp.iterations, lp.primal_feas, lp.gap, "l2", lp.termination_reason,
                         lp.primal_feas, lp.dual_feas, lp.dual_feas),
            DualViolationStats(scan_seconds, metrics["count"], added),
            BudgetedPruningStats(prune_seconds, grown, len(support), self.budget, grown > self.budget),
            ActiveSupportStats(size_before, grown, len(support), self.peak),
            ConvergenceStats(metrics[norm], tol, converged, metrics["l2"], metrics["linf"], metrics["max"], norm)))
        _progress(options, f"level={self.index} iteration={iteration} scan {scan_seconds:.3f}s "
                           f"dual_{norm}={metrics[norm]:.3e} added={added} support={len(support)}")
        return converged

    def run(self, max_iterations: int, initialization: InitializationStats, started: float) -> LevelResult:
        converged = False
        for iteration in range(max_iterations):
            if self.step(iteration):
                converged = True
                break
        summary = RefinementSummary(time.perf_counter() - started, len(self.records), float(self.lp.obj_val),
                                    len(self.support), self.peak,
                                    "converged" if converged else "max_refinement_iterations", converged)
        return LevelResult(self.index, "refined", self.n, self.m, initialization,
                           RefinementResult(tuple(self.records), summary), time.perf_counter() - started)


def _contains_any(sorted_keys: torch.Tensor, queries: torch.Tensor) -> bool:
    if sorted_keys.numel() == 0 or queries.numel() == 0:
        return False
    at = torch.searchsorted(sorted_keys, queries).clamp_max(sorted_keys.numel() - 1)
    return bool((sorted_keys[at] == queries).any())


def refine_level(cost: Cost, a, b, previous, inherited, options, level_index, max_iterations, detect_reentry):
    """Seed and refine one level; returns (support, duals, LevelResult, perturbation trigger, LP device time:
    seconds inside hm_pdhg_solve, PDHG iterations, and with the library's kernel timing on the iterations' own
    milliseconds and count)."""
    started = time.perf_counter()
    level = LevelRefinement(cost, a, b, options, level_index, detect_reentry)
    initialization = level.seed(previous, inherited)
    result = level.run(max_iterations, initialization, started)
    return level.support, level.dual, result, level.perturbation_triggered, dict(level.lp_device)


__all__ = ["LevelRefinement", "candidate_keys", "derive_hierarchy_seeds", "level_sizes", "refine_level",
           "shuffle_once_permutation"]
