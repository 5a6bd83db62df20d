"""HELLO driver: hierarchy chain, coarsest solve, per-level initialization and refinement, all on the GPU.

Follows the reference's GPU-resident algorithm (``gpu_resident/solver.py:27-398``):

* one global shuffle of each side (``hierarchy/plan.py:73-87``); level l keeps the first n_l / m_l points;
  going coarser, the larger side is divided by ``split_count`` until both are <= ``coarsest_size_threshold``;
* coarsest level: refined from zero duals like any other level (the reference calls POT ``emd`` on the CPU);
* each finer level: the side shared with the coarser level keeps its duals, the other side is completed by a
  c-transform (directional top-1 scan), both directions contribute their ``assignment_topk`` best pairs and
  the northwest-corner basis completes an initial support; then ``solve_lp -> pricing scan with certificate ->
  add violating pairs -> budgeted pruning`` until the relative dual infeasibility is <= tolerance.

Cost perturbation (``cost_perturbation="auto"``) is detected as in the reference (re-entry of pruned edges) but
not applied: the level keeps refining on the original cost and the trigger is recorded in the metadata.
"""
from __future__ import annotations

import sys
import time

import numpy as np
import torch

from ..config import active_support_budget, primal_support_cap
from ..types import (ActiveSupportStats, BudgetedPruningStats, CoarsestSolveStats, ConvergenceStats,
                     DualViolationStats, HelloSolveError, InitializationStats, IterationStats, LevelResult,
                     RefinementResult, RefinementSummary, SolveLPStats)
from .cost import Cost
from .support import Support, normalize_masses


def derive_hierarchy_seeds(seed: int, num_children: int):
    """Source-split, target-split and child seeds of a hierarchy node (hierarchy/utilities.py:56-65)."""
    rng = np.random.default_rng(int(seed))
    src = int(rng.integers(0, 2**31 - 1))
    tgt = int(rng.integers(0, 2**31 - 1))
    children = [int(rng.integers(0, 2**31 - 1)) for _ in range(int(num_children))]
    return src, tgt, children


def shuffle_once_permutation(n_source: int, n_target: int, seed: int, split_count: int):
    """One global random permutation per side (hierarchy/plan.py:73-87)."""
    src, tgt, _ = derive_hierarchy_seeds(seed, split_count)
    return (np.random.default_rng(src).permutation(int(n_source)).astype(np.int64),
            np.random.default_rng(tgt).permutation(int(n_target)).astype(np.int64))


def level_sizes(n: int, m: int, threshold: int, split: int):
    """Finest-first chain of (n_l, m_l): the larger side is divided by ``split`` until both fit ``threshold``."""
    sizes = [(n, m)]
    while max(sizes[-1]) > threshold:
        nn, mm = sizes[-1]
        sizes.append(((nn + split - 1) // split, mm) if nn >= mm else (nn, (mm + split - 1) // split))
    return sizes


def candidate_keys(xv, xi, yv, yi, dual, n, m, positive=False):
    """Keys row * m + col of the row-direction and column-direction candidates (gpu_resident/solver.py:27-35);
    with ``positive`` only pairs whose dual score sigma = f_i + g_j - c_ij is > 0."""
    parts = []
    if xi is not None:
        rows = torch.arange(n, device=dual.device)[:, None].expand_as(xi)
        mask = xi >= 0
        if positive:
            mask &= xv + dual[:n, None] > 0
        parts.append((rows * m + xi.long())[mask])
    if yi is not None:
        cols = torch.arange(m, device=dual.device)[:, None].expand_as(yi)
        mask = yi >= 0
        if positive:
            mask &= yv + dual[n:, None] > 0
        parts.append((yi.long() * m + cols)[mask])
    return torch.unique(torch.cat(parts), sorted=True)


def _sync():
    torch.cuda.synchronize()


def solve_leaf(cost: Cost, a, b, level_index: int, options, max_iterations: int):
    """Coarsest level. The reference solves it exactly with POT ``emd`` on the CPU (gpu_resident/solver.py:168-191);
    here it is refined like every other level, from zero duals: both directions' ``assignment_topk`` nearest
    pairs plus the northwest basis, then LP / pricing / support updates until the certificate passes. The
    result is optimal to the same tolerance as the finer levels and stays on the device."""
    started = time.perf_counter()
    n, m = cost.shape
    zeros = torch.zeros(n + m, dtype=torch.float64, device=a.device)
    support, dual, level, _ = refine(cost, a, b, zeros, None, options, level_index, max_iterations, False)
    summary = level.solve.summary
    if not summary.converged:
        raise HelloSolveError(f"coarsest level did not converge in {max_iterations} iterations")
    _sync()
    elapsed = time.perf_counter() - started
    stats = CoarsestSolveStats(elapsed, float(summary.final_objective), len(support.keys))
    return support, dual, LevelResult(level_index, "coarsest", n, m, level.initialization, stats, elapsed), level


def _progress(options, message: str) -> None:
    if options.verbose == "detailed":
        print(f"[hello-mi355x] {message}", file=sys.stderr, flush=True)


def initialize(cost: Cost, a, b, previous, known_side, options):
    """Dual propagation + directional assignment + northwest basis (gpu_resident/solver.py:38-64)."""
    started = time.perf_counter()
    n, m = cost.shape
    device = a.device
    k = options.assignment_topk
    dual = torch.zeros(n + m, dtype=torch.float64, device=device)
    if known_side == "target":
        dual[n:] = previous[-m:]
    elif known_side == "source":
        dual[:n] = previous[:n]
    else:
        dual = previous.clone()
    xv = xi = yv = yi = None
    if known_side == "target":
        xv, xi, _, _, _ = cost.scan(dual, k, direction="source")
        dual[:n] = -xv[:, 0]               # c-transform: f_i = min_j (c_ij - g_j)
        propagation = time.perf_counter() - started
        _progress(options, f"init {n}x{m}: source c-transform scan {propagation:.3f}s")
        _, _, yv, yi, _ = cost.scan(dual, k, direction="target")
    elif known_side == "source":
        _, _, yv, yi, _ = cost.scan(dual, k, direction="target")
        dual[n:] = -yv[:, 0]
        propagation = time.perf_counter() - started
        _progress(options, f"init {n}x{m}: target c-transform scan {propagation:.3f}s")
        xv, xi, _, _, _ = cost.scan(dual, k, direction="source")
    else:
        propagation = 0.0
        xv, xi, yv, yi, _ = cost.scan(dual, k)
    candidates = candidate_keys(xv, xi, yv, yi, dual, n, m)
    assigned = time.perf_counter() - started
    support = Support.initial(candidates, a, b)
    _sync()
    total = time.perf_counter() - started
    _progress(options, f"init {n}x{m}: {len(support.keys)} initial edges {total:.3f}s")
    stats = InitializationStats(total, propagation, assigned, total - assigned, known_side, k, len(candidates),
                                None, len(support.keys) - len(candidates), len(support.keys))
    return support, dual, stats


def refine(cost: Cost, a, b, previous, known_side, options, level_index, max_iterations, detect_reentry):
    """One level: initialization, then the SolveLP -> CheckOptimality -> UpdateSupport loop
    (gpu_resident/solver.py:67-165)."""
    started = time.perf_counter()
    support, dual, init_stats = initialize(cost, a, b, previous, known_side, options)
    n, m = cost.shape
    tol = options.tolerance
    budget = active_support_budget(options.support_budget_factor, n, m)
    cap = primal_support_cap(options.support_budget_factor, options.pricing_topk, n, m)
    peak = len(support.keys)
    previous_pruned, reentered, triggered = None, False, False
    history = []
    sparsifications = []
    lp = None
    for index in range(max_iterations):
        it_started = time.perf_counter()
        before = len(support.keys)
        t0 = time.perf_counter()
        dual, lp = support.solve_lp(cost, a, b, dual, tol, primal_cap=cap)
        lp_seconds = time.perf_counter() - t0
        if support.last_sparsification is not None:
            sparsifications.append(support.last_sparsification)
        _progress(options, f"level={level_index} iteration={index} lp {lp_seconds:.3f}s support={before} "
                           f"pdhg_iters={lp.iterations}"
                           + (f" sparsified {support.last_sparsification.input_nnz}->"
                              f"{support.last_sparsification.output_nnz}" if support.last_sparsification else ""))
        t0 = time.perf_counter()
        xv, xi, yv, yi, metrics = cost.scan(dual, options.pricing_topk, certificate=True)
        scan_seconds = time.perf_counter() - t0
        converged = metrics["l2"] <= tol
        if not converged and detect_reentry and reentered:
            triggered = True
        after, added_count, prune_seconds = before, 0, 0.0
        if not converged:
            candidates = candidate_keys(xv, xi, yv, yi, dual, n, m, positive=True)
            fresh = support.extend(candidates)
            added = support.keys[fresh]
            added_count, after = len(added), len(support.keys)
            peak = max(peak, after)
            reentered = previous_pruned is not None and bool(torch.isin(added, previous_pruned).any())
            t0 = time.perf_counter()
            previous_pruned = support.prune(cost, dual, fresh, budget)
            prune_seconds = time.perf_counter() - t0
            if not added_count:
                raise HelloSolveError("GPU full optimality check failed without new candidate edges")
        history.append(IterationStats(
            index, float(lp.obj_val), time.perf_counter() - it_started, 0.0, scan_seconds,
            SolveLPStats(lp_seconds, lp.iterations, lp.primal_feas, lp.gap, "l2", lp.termination_reason,
                         lp.primal_feas, lp.dual_feas, lp.dual_feas),
            DualViolationStats(scan_seconds, metrics["count"], added_count),
            BudgetedPruningStats(prune_seconds, after, len(support.keys), budget, after > budget),
            ActiveSupportStats(before, after, len(support.keys), peak),
            ConvergenceStats(metrics["l2"], tol, converged, metrics["l2"], metrics["linf"], metrics["max"], "l2")))
        _progress(options, f"level={level_index} iteration={index} scan {scan_seconds:.3f}s "
                           f"dual_l2={metrics['l2']:.3e} added={added_count} support={len(support.keys)}")
        if converged:
            break
    converged = bool(history and history[-1].convergence.passed)
    summary = RefinementSummary(time.perf_counter() - started, len(history), float(lp.obj_val), len(support.keys),
                                peak, "converged" if converged else "max_refinement_iterations", converged)
    level = LevelResult(level_index, "refined", n, m, init_stats, RefinementResult(tuple(history), summary),
                        time.perf_counter() - started)
    support.sparsification_log = sparsifications
    return support, dual, level, triggered


__all__ = ["candidate_keys", "derive_hierarchy_seeds", "initialize", "level_sizes", "refine",
           "shuffle_once_permutation", "solve_leaf"]
