"""Public problem / result records of the MI355X HELLO front end.

Field for field as the reference's records (``src/hello_ot/types.py:19-414``): ``Problem``, the per-iteration
statistics, ``LevelResult``, ``SparseOTSolution`` and ``Result``. Solutions of the GPU-resident path stay on
the device; ``SparseOTSolution.to_cpu`` exports them explicitly.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Literal, Mapping, Optional, Tuple, Union

import numpy as np
import torch

COST_TYPES = ("l2^2", "l1", "l2", "linf")


class HelloSolveError(RuntimeError):
    """A HELLO solve could not make progress (types.py:19)."""


def _points(value, name):
    """Point matrices as the reference's ``_float32_matrix`` (types.py:26-39) keeps them: a device tensor as it is
    (its dtype and layout are checked where they matter), anything else as contiguous fp32 on the host."""
    if torch.is_tensor(value):
        value = value.detach()
        if value.is_cuda:
            if value.ndim != 2 or min(value.shape) < 1:
                raise ValueError(f"{name} must be a non-empty 2D matrix")
            return value
        value = value.float().numpy()
    array = np.asarray(value, dtype=np.float32)
    if array.ndim != 2:
        raise ValueError(f"{name} must be a 2D array; got shape={array.shape}.")
    if array.shape[0] < 1 or array.shape[1] < 1:
        raise ValueError(f"{name} must be non-empty; got shape={array.shape}.")
    array = np.ascontiguousarray(array)
    if not np.all(np.isfinite(array)):
        raise ValueError(f"{name} must contain only finite values.")
    return array


def _mass(value, size, name):
    """Masses as the reference's ``_mass_vector`` (types.py:49-63): uniform when absent, a device tensor kept on its
    device in fp64, anything else a host fp64 vector; finite and strictly positive."""
    if torch.is_tensor(value):
        value = value.detach()
        if value.is_cuda:
            value = value.to(dtype=torch.float64).reshape(-1).contiguous()
            if value.numel() != size or not bool(torch.all(torch.isfinite(value) & (value > 0))):
                raise ValueError(f"{name} must have length {size} and finite, strictly positive values")
            return value
        value = value.double().numpy()
    if value is None:
        return np.full(int(size), 1.0 / float(size), dtype=np.float64)
    array = np.ascontiguousarray(np.asarray(value, dtype=np.float64).reshape(-1))
    if array.size != size:
        raise ValueError(f"{name} must have length {size}; got {array.size}.")
    if not np.all(np.isfinite(array)) or np.any(array <= 0.0):
        raise ValueError(f"{name} must contain only finite, strictly positive values.")
    return array


@dataclass(frozen=True)
class Problem:
    """Balanced point-cloud OT input (types.py:66-95): fp32 points, a cost type, optional positive masses."""

    source_points: Any
    target_points: Any
    cost_type: str
    source_mass: Optional[Any] = None
    target_mass: Optional[Any] = None

    def __post_init__(self) -> None:
        source = _points(self.source_points, "source_points")
        target = _points(self.target_points, "target_points")
        if source.shape[1] != target.shape[1]:
            raise ValueError("source_points and target_points must have the same feature dimension.")
        cost_type = str(self.cost_type).strip().lower()
        if cost_type not in COST_TYPES:
            raise ValueError("cost_type must be one of: l2^2, l1, l2, linf")
        object.__setattr__(self, "source_points", source)
        object.__setattr__(self, "target_points", target)
        object.__setattr__(self, "cost_type", cost_type)
        object.__setattr__(self, "source_mass", _mass(self.source_mass, source.shape[0], "source_mass"))
        object.__setattr__(self, "target_mass", _mass(self.target_mass, target.shape[0], "target_mass"))

    @property
    def shape(self) -> Tuple[int, int]:
        return int(self.source_points.shape[0]), int(self.target_points.shape[0])


@dataclass(frozen=True)
class SolveLPStats:
    wall_time: float
    backend_iterations: Optional[int]
    primal_feasibility: Optional[float]
    primal_dual_gap: Optional[float]
    termination_norm: Optional[Literal["l2", "linf"]] = None
    termination_reason: Optional[str] = None
    termination_primal_feasibility: Optional[float] = None
    termination_dual_feasibility: Optional[float] = None
    algorithm_dual_feasibility: Optional[float] = None


@dataclass(frozen=True)
class DualViolationStats:
    wall_time: float
    violations_found: int
    edges_added: int


@dataclass(frozen=True)
class BudgetedPruningStats:
    wall_time: float
    support_before: int
    support_after: int
    budget: int
    budget_exceeded: bool


@dataclass(frozen=True)
class ActiveSupportStats:
    before_lp: int
    after_dual_violation: int
    after_budgeted_pruning: int
    peak: int


@dataclass(frozen=True)
class ConvergenceStats:
    dual_feasibility: Optional[float]
    tolerance: float
    passed: bool
    relative_full_dual_feasibility: Optional[float] = None
    relative_linf_dual_feasibility: Optional[float] = None
    max_dual_violation: Optional[float] = None
    norm: Optional[Literal["l2", "linf"]] = None


@dataclass(frozen=True)
class IterationStats:
    index: int
    objective: float
    wall_time: float
    bookkeeping_time: float
    full_scan_time: float
    solve_lp: SolveLPStats
    dual_violation: DualViolationStats
    budgeted_pruning: BudgetedPruningStats
    support: ActiveSupportStats
    convergence: ConvergenceStats


@dataclass(frozen=True)
class InitializationStats:
    wall_time: float
    dual_propagation_time: float
    dual_assignment_time: float
    northwest_augmentation_time: float
    inherited_dual_side: Optional[Literal["source", "target"]]
    assignment_topk: int
    support_after_forward: int
    support_after_reverse: Optional[int]
    northwest_edges_added: int
    initial_active_support_size: int


@dataclass(frozen=True)
class RefinementSummary:
    wall_time: float
    iterations: int
    final_objective: float
    final_active_support_size: int
    peak_active_support_size: int
    stop_reason: str
    converged: bool


@dataclass(frozen=True)
class RefinementResult:
    iterations: Tuple[IterationStats, ...]
    summary: RefinementSummary
    solution: Optional["SparseOTSolution"] = None


@dataclass(frozen=True)
class CoarsestSolveStats:
    wall_time: float
    objective: float
    support_size: int


LevelSolveResult = Union[CoarsestSolveStats, RefinementResult]


@dataclass(frozen=True)
class LevelResult:
    level_index: int
    kind: Literal["coarsest", "refined"]
    n_source: int
    n_target: int
    initialization: Optional[InitializationStats]
    solve: LevelSolveResult
    wall_time: float


@dataclass(frozen=True)
class SolveStageResult:
    levels: Tuple[LevelResult, ...]
    wall_time: float


@dataclass(frozen=True)
class SparseOTSolution:
    """Sparse coupling (rows, cols, values) with the source / target duals; entries <= 1e-12 are dropped
    (types.py:264-338)."""

    shape: Tuple[int, int]
    rows: Any
    cols: Any
    values: Any
    source_dual: Any
    target_dual: Any

    def __post_init__(self) -> None:
        keys = ("rows", "cols", "values", "source_dual", "target_dual")
        if torch.is_tensor(self.values):
            if not all(torch.is_tensor(getattr(self, k)) and getattr(self, k).device == self.values.device for k in keys):
                raise ValueError("GPU solution arrays must share one device")
            rows, cols, values, f, g = (getattr(self, k).detach().to(torch.int64 if k in ("rows", "cols") else
                                                                     torch.float64).reshape(-1).contiguous()
                                        for k in keys)
            keep = values > 1e-12
            rows, cols, values = rows[keep], cols[keep], values[keep]
        else:
            rows = np.asarray(self.rows, np.int64).reshape(-1)
            cols = np.asarray(self.cols, np.int64).reshape(-1)
            values = np.asarray(self.values, np.float64).reshape(-1)
            f = np.asarray(self.source_dual, np.float64).reshape(-1)
            g = np.asarray(self.target_dual, np.float64).reshape(-1)
            keep = values > 1e-12
            rows, cols, values = rows[keep], cols[keep], values[keep]
        if not (len(rows) == len(cols) == len(values)):
            raise ValueError("rows, cols, and values must have equal lengths")
        if len(f) != int(self.shape[0]) or len(g) != int(self.shape[1]):
            raise ValueError("dual lengths must match solution shape")
        for key, value in zip(keys, (rows, cols, values, f, g)):
            object.__setattr__(self, key, value)

    def to_cpu(self) -> "SparseOTSolution":
        if not torch.is_tensor(self.values):
            return self
        return SparseOTSolution(self.shape, *(getattr(self, k).cpu().numpy() for k in
                                              ("rows", "cols", "values", "source_dual", "target_dual")))

    def to_sparse_matrix(self):
        if torch.is_tensor(self.values):
            return torch.sparse_coo_tensor(torch.stack((self.rows, self.cols)), self.values, self.shape).coalesce()
        from scipy import sparse

        return sparse.coo_matrix((self.values, (self.rows, self.cols)), shape=self.shape)

    def to_warm_start_state(self) -> "WarmStartState | GPUWarmStartState":
        """The plan and duals as a warm-start state (state.py:11-40): device tensors stay on their device."""
        if torch.is_tensor(self.values):
            return GPUWarmStartState(self.rows.int().clone(), self.cols.int().clone(), self.values.clone(),
                                     torch.cat((self.source_dual, self.target_dual)), int(self.shape[0]),
                                     int(self.shape[1]), str(self.values.device))
        return WarmStartState(self.rows.astype(np.int32), self.cols.astype(np.int32), self.values.astype(np.float64),
                              np.concatenate((self.source_dual, self.target_dual)).astype(np.float64),
                              int(self.shape[0]), int(self.shape[1]), None)


@dataclass(frozen=True)
class WarmStartState:
    """A host-side sparse plan with its duals (the reference's ``state.WarmStartState``)."""
    rows: np.ndarray
    cols: np.ndarray
    x_prev: np.ndarray
    dual_uv: Optional[np.ndarray]
    n_source: int
    n_target: int
    northwest_positions: Optional[np.ndarray] = None


@dataclass(frozen=True)
class GPUWarmStartState:
    """A device-side sparse plan with its duals (the reference's ``state.GPUWarmStartState``)."""
    rows: torch.Tensor
    cols: torch.Tensor
    x_prev: torch.Tensor
    dual_uv: Optional[torch.Tensor]
    n_source: int
    n_target: int
    device: str = "cuda"


@dataclass(frozen=True)
class CostStageResult:
    """One cost stage in execution order and its per-level statistics (types.py:352-359)."""
    name: str
    solve: SolveStageResult


@dataclass(frozen=True)
class Result:
    objective: float
    solution: SparseOTSolution
    solve_stage: SolveStageResult
    total_wall_time: float
    peak_gpu_memory_mib: Optional[float] = None
    trace: Optional[Any] = None
    metadata: Mapping[str, Any] = field(default_factory=dict)
    cost_stages: tuple = ()

    @property
    def original_cost_stage(self) -> SolveStageResult:
        return self.solve_stage

    @property
    def perturbed_cost_stage(self) -> Optional[SolveStageResult]:
        return next((stage.solve for stage in self.cost_stages if stage.name == "perturbed"), None)


__all__ = [
    "ActiveSupportStats", "BudgetedPruningStats", "COST_TYPES", "CoarsestSolveStats", "ConvergenceStats",
    "CostStageResult", "DualViolationStats", "GPUWarmStartState", "HelloSolveError", "InitializationStats",
    "IterationStats", "LevelResult", "Problem", "RefinementResult", "RefinementSummary", "Result", "SolveLPStats",
    "SolveStageResult", "SparseOTSolution", "WarmStartState",
]
