"""Restricted-OT Halpern-PDHG on MI355X behind the reference's restricted-OT solver interface.

Mirrors ``TorchRestrictedOTPDLP`` / ``CppRestrictedOTPDLP`` (``_internal/lp/torch_restricted_ot.py:105-393``,
``_internal/lp/cpp_restricted_ot.py:25-72``) and their shared contract ``RestrictedOTPDLP``
(``_internal/lp/restricted_ot_pdlp.py:12-100``): constructor options, ``solve_restricted`` arguments,
validation errors, the one-shot NUMERICAL_DIVERGENCE retry with scalar rescaling, and ``SolverResult``.
The iteration itself runs in ``hm_pdhg_solve`` (HIP kernels); nothing is computed on the CPU.
"""
from __future__ import annotations

import time
from typing import Any, Dict, Optional

import numpy as np
import torch

from .. import _lib
from .wrapper import SolverResult


def _as_1d(value: Any, *, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
    if torch.is_tensor(value):
        return value.detach().to(device=device, dtype=dtype).contiguous().view(-1)
    return torch.as_tensor(np.asarray(value), device=device, dtype=dtype).contiguous().view(-1)


def run_pdhg(rows_t, cols_t, costs_t, source_t, target_t, x0, y0, *, evaluation_frequency: int, rescale: bool,
             iteration_limit: int, objective_tolerance: float, primal_tolerance: float, dual_tolerance: float,
             time_limit_seconds: float, device: torch.device):
    """One ``hm_pdhg_solve`` call on validated device tensors (int64 endpoints, fp64 costs / masses / warm starts
    or None): returns (x, y, PdhgResult)."""
    n_source, n_target, e = int(source_t.numel()), int(target_t.numel()), int(costs_t.numel())
    masses_t = torch.cat((source_t, target_t))
    x_out = torch.empty(e, dtype=torch.float64, device=device)
    y_out = torch.empty(n_source + n_target, dtype=torch.float64, device=device)
    lib = _lib.load()
    ws = torch.empty(max(int(lib.hm_pdhg_workspace_bytes(n_source, n_target, e)), 256), dtype=torch.uint8,
                     device=device)
    params = _lib.PdhgParams(int(evaluation_frequency), int(bool(rescale)), int(iteration_limit),
                             float(objective_tolerance), float(primal_tolerance), float(dual_tolerance),
                             float(time_limit_seconds))
    res = _lib.PdhgResult()
    with torch.cuda.device(device):
        rc = lib.hm_pdhg_solve(_lib.stream_handle(device), _lib.ptr(rows_t), _lib.ptr(cols_t), _lib.ptr(costs_t),
                               _lib.ptr(masses_t), _lib.ptr(x0), _lib.ptr(y0), n_source, n_target, e, params,
                               _lib.ptr(x_out), _lib.ptr(y_out), res, _lib.ptr(ws), ws.numel())
    _lib.check(rc, "hm_pdhg_solve")
    return x_out, y_out, res


class NativeRestrictedOTPDLP:
    """FP64 Halpern-PDHG restricted OT solver for HELLO active supports, on MI355X."""

    def __init__(self, *, device: str | torch.device = "cuda", evaluation_frequency: int = 200,
                 time_limit_seconds: float = 3600.0, iteration_limit: int = np.iinfo(np.int32).max,
                 record_state_trace: bool = False) -> None:
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("NativeRestrictedOTPDLP runs on a ROCm GPU device")
        self.evaluation_frequency = int(evaluation_frequency)
        self.time_limit_seconds = float(time_limit_seconds)
        self.iteration_limit = int(iteration_limit)
        self.record_state_trace = bool(record_state_trace)
        if self.evaluation_frequency < 1:
            raise ValueError("evaluation_frequency must be >= 1")
        if self.time_limit_seconds <= 0.0 or self.iteration_limit < 1:
            raise ValueError("time_limit_seconds and iteration_limit must be positive")

    def solve_restricted(self, *, rows: Any, cols: Any, costs: Any, source_mass: Any, target_mass: Any,
                         warm_start_primal: Optional[Any] = None, warm_start_dual: Optional[Any] = None,
                         tolerance: float | Dict[str, float] = 1e-6, verbose: bool = False) -> SolverResult:
        if isinstance(tolerance, dict):
            objective_tolerance = float(tolerance.get("objective", 1e-6))
            primal_tolerance = float(tolerance.get("primal", objective_tolerance))
            dual_tolerance = float(tolerance.get("dual", objective_tolerance))
        else:
            objective_tolerance = primal_tolerance = dual_tolerance = float(tolerance)
        kwargs = dict(rows=rows, cols=cols, costs=costs, source_mass=source_mass, target_mass=target_mass,
                      warm_start_primal=warm_start_primal, warm_start_dual=warm_start_dual,
                      objective_tolerance=objective_tolerance, primal_tolerance=primal_tolerance,
                      dual_tolerance=dual_tolerance, verbose=bool(verbose))
        first = self._solve_once(scalar_rescaling=False, **kwargs)
        if first.termination_reason != "NUMERICAL_DIVERGENCE":
            return first
        retry = self._solve_once(scalar_rescaling=True, **kwargs)
        retry.solver_diag = dict(retry.solver_diag or {})
        retry.solver_diag.update({
            "numerical_rescaling_retry": True,
            "numerical_rescaling_first_termination_reason": first.termination_reason,
            "numerical_rescaling_first_iterations": int(first.iterations),
        })
        return retry

    def _solve_once(self, *, rows, cols, costs, source_mass, target_mass, warm_start_primal, warm_start_dual,
                    objective_tolerance, primal_tolerance, dual_tolerance, scalar_rescaling, verbose) -> SolverResult:
        started = time.perf_counter()
        dev = self.device
        rows_t = _as_1d(rows, dtype=torch.int64, device=dev)
        cols_t = _as_1d(cols, dtype=torch.int64, device=dev)
        costs_t = _as_1d(costs, dtype=torch.float64, device=dev)
        source_t = _as_1d(source_mass, dtype=torch.float64, device=dev)
        target_t = _as_1d(target_mass, dtype=torch.float64, device=dev)
        masses_t = torch.cat((source_t, target_t))
        n_source, n_target, e = int(source_t.numel()), int(target_t.numel()), int(costs_t.numel())
        if rows_t.numel() != e or cols_t.numel() != e:
            raise ValueError("rows, cols, and costs must have equal lengths")
        if e == 0:
            raise ValueError("restricted OT active support must not be empty")
        if bool(torch.any(rows_t < 0)) or bool(torch.any(rows_t >= n_source)):
            raise ValueError("source endpoint index is out of bounds")
        if bool(torch.any(cols_t < 0)) or bool(torch.any(cols_t >= n_target)):
            raise ValueError("target endpoint index is out of bounds")
        mass_scale = max(1.0, float(torch.max(torch.abs(masses_t)).item()))
        if abs(float(source_t.sum().item()) - float(target_t.sum().item())) > 1e-12 * mass_scale:
            raise ValueError("balanced restricted OT requires equal source and target total mass")
        x0 = None if warm_start_primal is None else _as_1d(warm_start_primal, dtype=torch.float64, device=dev)
        y0 = None if warm_start_dual is None else _as_1d(warm_start_dual, dtype=torch.float64, device=dev)
        if (x0 is not None and x0.numel() != e) or (y0 is not None and y0.numel() != n_source + n_target):
            raise ValueError("warm-start dimensions do not match the restricted OT problem")
        x_out, y_out, res = run_pdhg(rows_t, cols_t, costs_t, source_t, target_t, x0, y0,
                                     evaluation_frequency=self.evaluation_frequency, rescale=scalar_rescaling,
                                     iteration_limit=self.iteration_limit, objective_tolerance=objective_tolerance,
                                     primal_tolerance=primal_tolerance, dual_tolerance=dual_tolerance,
                                     time_limit_seconds=self.time_limit_seconds, device=dev)
        reason = _lib.REASONS[int(res.reason)]
        duration = float(time.perf_counter() - started)
        diag = {
            "backend": "mi355x_hip", "device": str(dev), "dtype": "float64",
            "scaling_mode": "degree_sqrt" + ("_with_scalar_retry" if scalar_rescaling else ""),
            "step_size": 0.998, "termination_norm": "l2",
            "termination_abs_primal_res": res.abs_primal, "termination_rel_primal_res": res.rel_primal,
            "termination_abs_dual_res": res.abs_dual, "termination_rel_dual_res": res.rel_dual,
            "relative_primal_dual_gap": res.rel_gap, "primal_weight": res.primal_weight,
            "restart_count": int(res.restarts), "runtime_sec": duration, "device_loop_sec": res.seconds,
            "termination_reason": reason, "numerical_rescaling_retry": bool(scalar_rescaling),
        }
        if verbose:
            print(f"[NativeRestrictedOTPDLP] termination={reason} iterations={res.iterations} "
                  f"rel_primal={res.rel_primal:.3e} rel_dual={res.rel_dual:.3e} gap={res.rel_gap:.3e}")
        return SolverResult(success=reason == "OPTIMAL", x=x_out, y=y_out, obj_val=res.primal_objective,
                            dual_obj_val=res.dual_objective, duration=duration, iterations=int(res.iterations),
                            peak_mem=0.0, termination_reason=reason, primal_feas=res.rel_primal,
                            dual_feas=res.rel_dual, gap=res.rel_gap, solver_diag=diag)


__all__ = ["NativeRestrictedOTPDLP", "run_pdhg"]
