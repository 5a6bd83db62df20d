"""``solve`` -- the HELLO front end of the MI355X build (``src/hello_ot/__init__.py:40-90``, ``api.py:353-372``).

Array calls default to squared-Euclidean cost and uniform masses; ``max_iterations`` bounds the refinement
iterations per level and ``random_seed`` fixes the global shuffle. Inputs may be numpy arrays or tensors; the
solve runs on ``cuda:0`` (or the device of CUDA input tensors) and returns a device-resident ``Result``.
"""
from __future__ import annotations

import os
import sys
import time
from typing import Any, Optional

import numpy as np
import torch

from ._native_compat import require_native_runtime_compatibility
from .config import SolverOptions, level_precision
from .resident.cost import Cost
from .resident import host as _host
from .resident.host import HostRows, permute_rows_inplace, shuffled_rows
from .resident.leaf import solve_coarsest
from .resident.solver import level_sizes, refine_level, shuffle_once_permutation
from .resident.support import balanced_masses
from .types import CostStageResult, Problem, Result, SolveStageResult, SparseOTSolution


def solve(source_points: Problem | Any, target_points: Any | None = None, *, source_mass: Any | None = None,
          target_mass: Any | None = None, cost: str | None = None, max_iterations: int = 100,
          random_seed: int = 42, options: SolverOptions | None = None) -> Result:
    if isinstance(source_points, Problem):
        if target_points is not None or source_mass is not None or target_mass is not None or cost is not None:
            raise TypeError("When the first argument is Problem, target_points, masses, and cost must not be repeated.")
        problem = source_points
    else:
        if target_points is None:
            raise TypeError("target_points is required when solving from arrays")
        problem = Problem(source_points, target_points, "l2^2" if cost is None else cost, source_mass, target_mass)
    if int(max_iterations) < 1:
        raise ValueError("max_iterations must be >= 1")
    if not isinstance(random_seed, int):
        raise TypeError("random_seed must be an int")
    options = SolverOptions() if options is None else options
    if not isinstance(options, SolverOptions):
        raise TypeError("options must be SolverOptions or None")
    return solve_problem(problem, options, max_iterations=int(max_iterations), random_seed=int(random_seed))


def _device_of(problem: Problem) -> torch.device:
    for value in (problem.source_points, problem.target_points):
        if torch.is_tensor(value) and value.is_cuda:
            return value.device
    return torch.device("cuda", 0)


def _to_device(value, device, dtype):
    if torch.is_tensor(value):
        return value.to(device=device, dtype=dtype)
    return torch.as_tensor(np.asarray(value), dtype=dtype, device=device)


def _permute_in_place(value, perm, device, bounded: bool):
    """value[i] = (old value)[perm[i]] in place: through one full temporary, or, with ``bounded`` (a
    memory-bounded solve) or when the device has no room for the temporary, with one block of extra device memory
    (``permute_rows_inplace``, which walks the permutation's cycles on the device)."""
    nbytes = 4 * value.numel()
    if nbytes > _host.STREAM_MIN_BYTES and (bounded or torch.cuda.mem_get_info(device)[0] < nbytes + (4 << 30)):
        permute_rows_inplace(value, perm)
    else:
        value.copy_(value[perm])


def _shuffled_features(value, perm, device, consume: bool, restore: list, bounded: bool = False):
    """Rows of ``value`` in shuffle order as contiguous fp32 on ``device``. With ``consume`` a contiguous fp32
    tensor already on the device is reordered in place, and (tensor, inverse permutation, bounded) is appended to
    ``restore`` so that the caller's order comes back when the solve ends, as the reference's in-place reorder
    does (``gpu_resident/storage.py:74-120``, ``prewarm.py:177-214``)."""
    if consume and torch.is_tensor(value) and value.device == device and value.dtype == torch.float32 \
            and value.is_contiguous():
        _permute_in_place(value, perm, device, bounded)
        inverse = torch.empty_like(perm)
        inverse[perm] = torch.arange(perm.numel(), device=perm.device, dtype=perm.dtype)
        restore.append((value, inverse, bounded))
        return value
    return _to_device(value, device, torch.float32)[perm].contiguous()


def _stream_source(value, target, cost_type: str, device, options: SolverOptions) -> bool:
    """Whether the source side stays in host memory and is streamed in chunks (the reference's non-resident path:
    kernels/bilinear_topk.py:255-368). ``gpu_resident=True`` keeps both sides on the device. Otherwise a source side
    of more than STREAM_MIN_BYTES of fp32 features is streamed when the resident plan would take more than
    RESIDENT_BUDGET of the device's memory (``STREAM_POLICY`` / HELLOOT_STREAM_SOURCE can force either way), which
    leaves the device one side's features plus bounded chunk staging. A streamed side is read from the caller's
    host matrix, chunk by chunk in the shuffled order (``consume_input_features`` then applies to the target side
    only)."""
    if options.gpu_resident:
        return False
    rows, d = (int(s) for s in value.shape)
    if 4 * rows * d <= _host.STREAM_MIN_BYTES:
        return False
    policy = os.environ.get("HELLOOT_STREAM_SOURCE", _host.STREAM_POLICY)
    if policy not in ("auto", "always", "never"):
        raise ValueError("HELLOOT_STREAM_SOURCE must be one of: auto, always, never")
    if policy != "auto":
        return policy == "always"
    # the resident plan: both fp32 sides, the l2^2 sweep's int8 copy of the larger side, the scan's list budget
    # (12 GiB) and the LP / support state
    other = int(target.shape[0])
    need = 4 * (rows + other) * d + (2 * max(rows, other) * d if cost_type == "l2^2" else 0) + (16 << 30)
    total = torch.cuda.get_device_properties(device).total_memory
    return need > _host.RESIDENT_BUDGET * total


def _streamed_side(value, perm, device) -> HostRows:
    """The streamed source side: a contiguous fp32 host matrix (torch, or numpy without a conversion) is read in
    place, its chunks gathered in shuffle order as they are streamed; anything else (device tensors, other dtypes or
    layouts) is first copied into a host matrix in shuffle order."""
    host = value
    if isinstance(host, np.ndarray) and host.dtype == np.float32 and host.ndim == 2 and host.flags.c_contiguous:
        host = torch.from_numpy(host)
    if torch.is_tensor(host) and host.device.type == "cpu" and host.dtype == torch.float32 and host.ndim == 2 \
            and host.is_contiguous():
        return HostRows(host, device, order=perm)
    return HostRows(shuffled_rows(value, perm), device)


@torch.no_grad()
def solve_problem(problem: Problem, options: SolverOptions, *, max_iterations: int = 100,
                  random_seed: int = 42) -> Result:
    options.check_supported()
    if options.stopping_norm == "finest_linf" and problem.cost_type != "l2^2":
        raise ValueError("finest_linf currently requires l2^2")   # gpu_resident/solver.py:235-236
    require_native_runtime_compatibility()
    device = _device_of(problem)
    n, m = problem.shape
    if options.gpu_resident:
        # the reference's GPU-resident entry takes both sides as device tensors (gpu_resident/solver.py:230-234)
        x, y = problem.source_points, problem.target_points
        if not all(torch.is_tensor(v) and v.is_cuda for v in (x, y)) or x.device != y.device:
            raise ValueError("gpu_resident requires source and target CUDA tensors on the same device")
        if any(v.dtype != torch.float32 or not v.is_contiguous() for v in (x, y)):
            raise ValueError("gpu_resident requires contiguous FP32 input features")
    consume = bool(options.consume_input_features)
    if consume and all(torch.is_tensor(v) for v in (problem.source_points, problem.target_points)) and \
            problem.source_points.untyped_storage().data_ptr() == problem.target_points.untyped_storage().data_ptr():
        raise ValueError("consume_input_features requires source and target with disjoint storage")
    with torch.cuda.device(device):
        torch.cuda.synchronize(device)
        torch.cuda.reset_peak_memory_stats(device)
        started = time.perf_counter()
        perm_s, perm_t = shuffle_once_permutation(n, m, random_seed, options.split_count)
        si = torch.as_tensor(perm_s, device=device)
        ti = torch.as_tensor(perm_t, device=device)
        a = (torch.full((n,), 1.0 / n, dtype=torch.float64, device=device) if problem.source_mass is None
             else _to_device(problem.source_mass, device, torch.float64))[si]
        b = (torch.full((m,), 1.0 / m, dtype=torch.float64, device=device) if problem.target_mass is None
             else _to_device(problem.target_mass, device, torch.float64))[ti]
        restore = []  # tensors reordered in place: the caller's order comes back when the solve ends, or fails
        try:
            run = _solve_levels(problem, options, device, si, ti, a, b, consume, restore, max_iterations)
        finally:
            for value, inverse, bounded in reversed(restore):
                _permute_in_place(value, inverse, device, bounded)
        torch.cuda.synchronize(device)
        wall = time.perf_counter() - started
        peak = torch.cuda.max_memory_allocated(device) / 2**20
    levels = run["levels"]
    stage = SolveStageResult(tuple(levels), wall)
    sparsified = run["sparsified"]
    metadata = {
        "gpu_resident": not run["streamed"], "streamed_source": run["streamed"],
        "backend": "native", "device": str(device), "cost_type": problem.cost_type,
        "cost_precision": options.cost_precision, "stopping_norm": options.stopping_norm,
        "coarsest_solver": "mi355x_network_simplex", "lp_solver": "mi355x_halpern_pdhg",
        "hierarchy_sizes": [list(s) for s in run["sizes"]],
        "total_refinement_iterations": sum(len(l.solve.iterations) for l in levels if l.kind == "refined"),
        "total_lp_solve_time": sum(i.solve_lp.wall_time for l in levels if l.kind == "refined"
                                   for i in l.solve.iterations),
        "total_scan_time": sum(i.full_scan_time for l in levels if l.kind == "refined" for i in l.solve.iterations),
        "cost_perturbation": {"policy": options.cost_perturbation, "activated": False,
                              "reentry_trigger_levels": run["triggers"]},
        "lp_device_by_level": run["lp_device"],
        "support_sparsification": {"events": len(sparsified),
                                   "cycle_updates": sum(r.cycle_updates for r in sparsified),
                                   "removed_edges": sum(r.input_nnz - r.output_nnz for r in sparsified),
                                   "wall_time": sum(r.wall_time for r in sparsified)},
    }
    result = Result(run["objective"], run["solution"], stage, wall, peak, None, metadata,
                    (CostStageResult("original", stage),))
    if options.verbose != "off":
        finest = levels[-1]
        state = finest.solve.summary.stop_reason if finest.kind == "refined" else "coarsest"
        print(f"[hello-mi355x] n={n} m={m} cost={problem.cost_type} objective={run['objective']:.12g} "
              f"time={wall:.3f}s levels={len(levels)} finest={state}", file=sys.stderr)
    return result


def _solve_levels(problem, options, device, si, ti, a, b, consume, restore, max_iterations) -> dict:
    """The hierarchy on the shuffled features, coarsest level first; the plan and duals come back in the caller's
    numbering."""
    n, m = problem.shape
    if _stream_source(problem.source_points, problem.target_points, problem.cost_type, device, options):
        x = _streamed_side(problem.source_points, si, device)
    else:
        x = _shuffled_features(problem.source_points, si, device, consume, restore)
    y = _shuffled_features(problem.target_points, ti, device, consume, restore, bounded=isinstance(x, HostRows))
    full = Cost.create(x, y, problem.cost_type)
    sizes = level_sizes(n, m, options.coarsest_size_threshold, options.split_count)
    levels, previous, triggers = [], None, []
    support = dual = None
    sparsified, lp_device = [], []
    for level_index in reversed(range(len(sizes))):
        nn, mm = sizes[level_index]
        cost = full.sliced(nn, mm, level_precision(options.cost_precision, level_index))
        aa, bb = balanced_masses(a[:nn].clone(), b[:mm].clone())
        if previous is None:
            support, dual, level = solve_coarsest(cost, aa, bb, level_index)
        else:
            inherited = "target" if nn >= mm else "source"
            support, dual, level, triggered, lp_time = refine_level(cost, aa, bb, previous, inherited, options,
                                                                    level_index, max_iterations,
                                                                    options.cost_perturbation == "auto")
            lp_device.append({"level": level_index, **lp_time})
            if triggered:
                triggers.append(level_index)
        levels.append(level)
        sparsified.extend(support.sparsification_log)
        previous = dual
    rows, cols = support.endpoints()
    objective = float(full.pairs(rows, cols) @ support.flow)
    keys = si[rows] * m + ti[cols]
    order = torch.argsort(keys, stable=True)
    f = torch.empty(n, dtype=torch.float64, device=device)
    g = torch.empty(m, dtype=torch.float64, device=device)
    f[si], g[ti] = dual[:n], dual[n:]
    solution = SparseOTSolution((n, m), si[rows][order], ti[cols][order], support.flow[order], f, g)
    return {"levels": levels, "sizes": sizes, "streamed": isinstance(x, HostRows), "objective": objective,
            "solution": solution, "triggers": triggers, "sparsified": sparsified, "lp_device": lp_device}


__all__ = ["solve", "solve_problem"]
