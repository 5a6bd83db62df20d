"""``hello_ot_native.pycupdlpx`` served by the MI355X restricted-OT Halpern-PDHG (``hm_pdhg_solve``).

The reference loads this module as its LP engine (``load_native_module("hello_ot_native.pycupdlpx")``,
``src/hello_ot/_source_build.py:174-178``, ``gpu_resident/solver.py:239-241``) and drives it through
``CuPDLPxSolver.solve`` (``_internal/lp/cupdlpx.py:658``): ``cupdlpx()`` -> ``loadData_device_csr(...)`` ->
``setInitSol(x0, y0)`` -> ``solve(params)`` -> ``getSolution()`` (binding ``cupdlpx_bindings.cpp:711-1093,
2069-2121``). HELLO's LPs are restricted transport problems, and so is what this module accepts: an all-equality
LP whose constraint matrix is the bipartite incidence matrix of the support (each variable has one entry in a source
row and one in a target row, rows 0..n_source-1 the sources), x >= 0, given on the device-CSR path with either the
plain incidence values (all ones) or the values of a pre-applied diagonal rescaling (``has_precomputed_rescaling``:
1 / (row scale * column scale), with ``c / column scale`` and ``rhs / row scale``, and optionally the scalar
bound / objective rescalings; ``cupdlpx.py:314-530``). The module recovers the support, the costs and the masses
from it, solves the LP with the library's PDHG (degree-sqrt scaling, constant step 0.998, Halpern, restarts and PID
as the reference's restricted-OT solver, ``_native/cpp/solver.cpp:39-378``), and returns the solution unscaled, as
the binding does with ``do_unscale``. Any other LP or option that selects a different algorithm raises
``NotImplementedError``.
"""
from __future__ import annotations

import math
import time

import numpy as np
import torch

from hello_ot_amd import _lib
from hello_ot_amd.lp.native_pdlp import run_pdhg

GPU_ARRAY_IO_VERSION = 1

_DEFAULTS = {
    "termination_evaluation_frequency": 200, "termination_norm": "l2", "iteration_limit": 2**31 - 1,
    "time_sec_limit": 3600.0, "eps_optimal_relative": 1e-4, "eps_feasible_relative_primal": 1e-4,
    "eps_feasible_relative_dual": 1e-4, "step_size_method": 3, "step_size_safety": 0.998,
    "l_inf_ruiz_iterations": 0, "has_pock_chambolle_alpha": False, "bound_objective_rescaling": False,
    "return_device": "cpu", "vector_sum_mode": "direct_reduce",
}


def make_default_params() -> dict:
    """The parameter keys this module reads, with their defaults."""
    return dict(_DEFAULTS)


def set_free_mode(mode: int) -> None:
    """Memory-release policy of the CUDA binding; device buffers here are freed with the solver object."""
    if int(mode) not in (0, 1, 2):
        raise ValueError("free mode must be 0, 1 or 2")


def reset_cuda_device() -> None:
    """The binding resets its CUDA context; the MI355X module keeps none of its own."""


def _scalar_or_all(value, target: float) -> bool:
    if value is None:
        return False
    if torch.is_tensor(value):
        return bool(torch.all(value == target)) if value.numel() else True
    if isinstance(value, np.ndarray):
        return bool(np.all(value == target))
    return float(value) == target


def _unsupported(what: str):
    raise NotImplementedError(f"hello_ot_native.pycupdlpx on MI355X solves HELLO's restricted transport LPs only: {what}")


class cupdlpx:  # noqa: N801 - the reference binding's class name
    """One restricted transport LP at a time, as the binding's ``cupdlpx`` holder."""

    def __init__(self):
        self._problem = None
        self._x0 = self._y0 = None
        self._last = None
        self._load_stats = {}

    # -- loaders ------------------------------------------------------------------------------------------
    def loadData_device_csr(self, row_ptr, col_ind, values, m, n, c, rhs, lb, ub, nEqs,
                            variable_bound_mode="explicit", matrix_value_mode="explicit", constraint_rescaling=None,
                            variable_rescaling=None, constraint_bound_rescaling=1.0, objective_vector_rescaling=1.0,
                            original_objective_vector_norm=None, original_constraint_bound_norm=None,
                            has_precomputed_rescaling=False, original_objective_vector_linf_norm=None,
                            original_constraint_bound_linf_norm=None):
        started = time.perf_counter()
        if not all(torch.is_tensor(t) and t.is_cuda for t in (row_ptr, col_ind, c, rhs)):
            raise TypeError("loadData_device_csr requires CUDA tensors for row_ptr, col_ind, c and rhs")
        dev = row_ptr.device
        vertices, edges = int(m), int(n)
        if int(nEqs) != vertices:
            _unsupported("every constraint must be an equality (nEqs == m)")
        if str(variable_bound_mode) not in ("explicit", "constant"):
            raise ValueError("variable_bound_mode must be explicit or constant")
        if not (_scalar_or_all(lb, 0.0) and _scalar_or_all(ub, math.inf)):
            _unsupported("variable bounds must be 0 <= x < inf")
        row_ptr = row_ptr.to(torch.int64)
        col_ind = col_ind.to(torch.int64)
        if row_ptr.numel() != vertices + 1 or int(row_ptr[0]) != 0 or int(row_ptr[-1]) != col_ind.numel():
            raise ValueError("row_ptr must have m + 1 entries from 0 to nnz")
        if col_ind.numel() != 2 * edges or c.numel() != edges or rhs.numel() != vertices:
            _unsupported("the constraint matrix must be a bipartite incidence matrix (two entries per variable)")
        if edges == 0 or int(col_ind.min()) < 0 or int(col_ind.max()) >= edges:
            raise ValueError("col_ind must hold variable indices in [0, n)")
        if not bool(torch.all(torch.bincount(col_ind, minlength=edges) == 2)):
            _unsupported("the constraint matrix must be a bipartite incidence matrix (two entries per variable)")
        counts = row_ptr[1:] - row_ptr[:-1]
        row_of = torch.repeat_interleave(torch.arange(vertices, device=dev), counts)
        first = torch.full((edges,), vertices, dtype=torch.int64, device=dev).scatter_reduce(
            0, col_ind, row_of, reduce="amin")
        second = torch.zeros(edges, dtype=torch.int64, device=dev).scatter_reduce(0, col_ind, row_of, reduce="amax")
        # the source rows come first and hold one entry of every variable: they end where row_ptr reaches n
        n_source = int(torch.searchsorted(row_ptr, torch.tensor([edges], device=dev)).item())
        if n_source > vertices or int(row_ptr[n_source]) != edges or not bool(torch.all(first < n_source)) \
                or not bool(torch.all(second >= n_source)):
            _unsupported("every variable must join one source row (rows 0..n_source-1) and one target row")
        con = torch.ones(vertices, dtype=torch.float64, device=dev) if constraint_rescaling is None else \
            torch.as_tensor(constraint_rescaling, dtype=torch.float64, device=dev).view(-1)
        var = torch.ones(edges, dtype=torch.float64, device=dev) if variable_rescaling is None else \
            torch.as_tensor(variable_rescaling, dtype=torch.float64, device=dev).view(-1)
        if not has_precomputed_rescaling:
            con, var = torch.ones_like(con), torch.ones_like(var)
            constraint_bound_rescaling = objective_vector_rescaling = 1.0
        if values is not None:
            expected = 1.0 / (con[row_of] * var[col_ind])
            if values.numel() != col_ind.numel() or not bool(torch.allclose(values.to(torch.float64), expected,
                                                                              rtol=1e-12, atol=0.0)):
                _unsupported("the matrix values must be the (rescaled) incidence values")
        bound_scale, objective_scale = float(constraint_bound_rescaling), float(objective_vector_rescaling)
        costs = c.to(torch.float64) * var / objective_scale
        masses = rhs.to(torch.float64) * con / bound_scale
        self._problem = {
            "rows": first.contiguous(), "cols": (second - n_source).contiguous(), "costs": costs.contiguous(),
            "source": masses[:n_source].contiguous(), "target": masses[n_source:].contiguous(), "device": dev,
            "scalar_rescaling": bound_scale != 1.0 or objective_scale != 1.0,
        }
        self._x0 = self._y0 = None
        self._last = None
        self._load_stats = {"sparse_format": "device_csr", "n_source": n_source, "n_target": vertices - n_source,
                            "edges": edges, "total_time_sec": time.perf_counter() - started}

    def _host_loader(self, *args, **kwargs):
        _unsupported("HELLO's LPs arrive on the device-CSR path (loadData_device_csr)")

    loadData = loadData_csr = loadData_csc = _host_loader

    def getLoadStats(self) -> dict:
        return dict(self._load_stats)

    def setInitSol(self, x0, y0):
        if self._problem is None:
            raise RuntimeError("No problem loaded. Call loadData_device_csr first.")
        dev = self._problem["device"]
        self._x0 = torch.as_tensor(x0, dtype=torch.float64, device=dev).contiguous().view(-1)
        self._y0 = torch.as_tensor(y0, dtype=torch.float64, device=dev).contiguous().view(-1)

    # -- solve --------------------------------------------------------------------------------------------
    def solve(self, params=None) -> dict:
        if self._problem is None:
            raise RuntimeError("No problem loaded. Call loadData_device_csr first.")
        p = make_default_params()
        p.update(dict(params or {}))
        if str(p["termination_norm"]).lower() != "l2":
            _unsupported("termination_norm must be l2")
        if int(p["step_size_method"]) != 3:
            _unsupported("step_size_method must be 3 (constant steps)")
        # Pock-Chambolle with alpha = 1 on a 0/1 incidence matrix scales rows and columns by sqrt(degree): the
        # diagonal scaling the PDHG applies anyway (and the one a pre-rescaled payload already carries)
        if int(p.get("l_inf_ruiz_iterations", 0) or 0) != 0 or (
                bool(p.get("has_pock_chambolle_alpha")) and float(p.get("pock_chambolle_alpha", 1.0)) != 1.0):
            _unsupported("the only scaling is the degree-sqrt diagonal one (no Ruiz passes, Pock-Chambolle alpha 1)")
        if str(p["return_device"]) not in ("cpu", "cuda"):
            raise ValueError("return_device must be cpu or cuda")
        prob = self._problem
        dev = prob["device"]
        edges, vertices = prob["costs"].numel(), prob["source"].numel() + prob["target"].numel()
        x0 = self._x0 if self._x0 is not None and self._x0.numel() == edges else None
        y0 = self._y0 if self._y0 is not None and self._y0.numel() == vertices else None
        started = time.perf_counter()
        torch.cuda.reset_peak_memory_stats(dev)
        x, y, res = run_pdhg(prob["rows"], prob["cols"], prob["costs"], prob["source"], prob["target"], x0, y0,
                             evaluation_frequency=int(p["termination_evaluation_frequency"]),
                             rescale=bool(p.get("bound_objective_rescaling")) or prob["scalar_rescaling"],
                             iteration_limit=int(p["iteration_limit"]),
                             objective_tolerance=float(p["eps_optimal_relative"]),
                             primal_tolerance=float(p["eps_feasible_relative_primal"]),
                             dual_tolerance=float(p["eps_feasible_relative_dual"]),
                             time_limit_seconds=float(p["time_sec_limit"]), device=dev)
        runtime = time.perf_counter() - started
        reason = _lib.REASONS[int(res.reason)]
        if p["return_device"] == "cpu":
            x, y = x.cpu().numpy(), y.cpu().numpy()
        out = {
            "termination_reason": reason, "iterations": int(res.iterations),
            "primal_objective": res.primal_objective, "dual_objective": res.dual_objective,
            "abs_primal_res": res.abs_primal, "rel_primal_res": res.rel_primal,
            "abs_dual_res": res.abs_dual, "rel_dual_res": res.rel_dual,
            "termination_norm": "l2", "termination_abs_primal_res": res.abs_primal,
            "termination_rel_primal_res": res.rel_primal, "termination_abs_dual_res": res.abs_dual,
            "termination_rel_dual_res": res.rel_dual,
            "abs_obj_gap": abs(res.primal_objective - res.dual_objective), "rel_obj_gap": res.rel_gap,
            "restart_count": int(res.restarts), "primal_weight": res.primal_weight,
            "matrix_value_mode": "implicit_aty", "implicit_ax_enabled": False, "implicit_aty_enabled": True,
            "implicit_ax_agg": "none", "vector_sum_mode": str(p["vector_sum_mode"]),
            "peak_gpu_mem_mib": torch.cuda.max_memory_allocated(dev) / 2**20,
            "runtime_sec": runtime, "cumulative_time_sec": res.seconds, "x": x, "y": y,
        }
        self._last = out
        return out

    def getSolution(self) -> dict:
        if self._last is None:
            raise RuntimeError("No solution yet. Call solve first.")
        r = self._last
        return {"x": r["x"], "y": r["y"], "PrimalObj": r["primal_objective"], "DualObj": r["dual_objective"],
                "iters": r["iterations"], "solve_time": r["runtime_sec"], "PrimalFeas": r["abs_primal_res"],
                "DualFeas": r["abs_dual_res"], "DualityGap": r["abs_obj_gap"], "PrimalFeasRel": r["rel_primal_res"],
                "DualFeasRel": r["rel_dual_res"], "RelObjGap": r["rel_obj_gap"], "PrimalFeasAvg": None,
                "DualFeasAvg": None, "DualityGapAvg": None, "PrimalFeasAvgRel": None, "DualFeasAvgRel": None,
                "RelObjGapAverage": None, "SaveInfo": 0, "LastRestartIter": -1, "PrimalStep": 0.0}


__all__ = ["GPU_ARRAY_IO_VERSION", "cupdlpx", "make_default_params", "reset_cuda_device", "set_free_mode"]
