"""``SolverOptions`` of the MI355X HELLO front end.

Same fields, defaults and validation messages as the reference's public options (``src/hello_ot/config.py:50-115``)
so callers can switch without edits. Only the native GPU-resident path exists here:

* ``backend`` must be ``"native"`` (the reference's torch / cpp CPU backends are not part of this build);
* ``cost_perturbation="on"`` raises ``NotImplementedError``, and ``"auto"`` records a re-entry trigger but keeps
  refining on the original cost (the perturbed cost stage is outside this build's scope);
* ``cost_precision``: the kernels read fp32 features and rank squared-Euclidean pairs by fp64 scores (fp64 dots
  re-evaluated for every candidate near a list's cut; pair costs in fp64), which is what ``"fp64"`` and
  ``"finest_fp64"`` ask for, so all three run the same ℓ2² path. The ℓ1 / ℓ2 / ℓ∞ costs follow the level's
  precision (``level_precision``, ``config.py:23-28`` of the reference): fp32 chunked costs, or fp64 costs in the
  scans (the reference's ``compute_precision = 1``) and fp64 pair costs on the support.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Literal, Optional

POSITIVE_SUPPORT_TOLERANCE = 1e-15


def finest_stopping_norm(policy: str) -> str:
    """The norm the finest level stops on under ``stopping_norm`` (config.py:31-36)."""
    if policy not in {"l2", "finest_linf"}:
        raise ValueError("stopping_norm must be one of: l2, finest_linf")
    return "linf" if policy == "finest_linf" else "l2"


def level_stopping_norm(policy: str, level_index: int) -> str:
    """The norm hierarchy level ``level_index`` (0 = finest) stops on (config.py:39-46): coarser levels always l2."""
    return finest_stopping_norm(policy) if int(level_index) == 0 else "l2"


def level_precision(policy: str, level_index: int) -> str:
    """Cost arithmetic of hierarchy level ``level_index`` (0 = finest) under ``cost_precision`` (config.py:23-28)."""
    if policy not in {"fp32", "fp64", "finest_fp64"}:
        raise ValueError("cost_precision must be one of: fp32, fp64, finest_fp64")
    return "fp64" if policy == "fp64" or (policy == "finest_fp64" and int(level_index) == 0) else "fp32"


def normalize_pricing_topk(value) -> int:
    """refinement/support_budget.py:10-24."""
    if isinstance(value, bool):
        raise ValueError("pricing_topk must be a positive integer")
    try:
        parsed = float(value)
    except (TypeError, ValueError) as error:
        raise ValueError("pricing_topk must be a positive integer") from error
    if not math.isfinite(parsed) or parsed < 1.0 or not parsed.is_integer():
        raise ValueError("pricing_topk must be a positive integer")
    return int(parsed)


def validate_support_budget_factor(beta, gamma: int) -> float:
    """HELLO requires beta >= gamma + 2 (refinement/support_budget.py:27-46)."""
    if isinstance(beta, bool):
        raise ValueError("support_budget_factor must be finite and positive")
    try:
        parsed = float(beta)
    except (TypeError, ValueError) as error:
        raise ValueError("support_budget_factor must be finite and positive") from error
    if not math.isfinite(parsed) or parsed <= 0.0:
        raise ValueError("support_budget_factor must be finite and positive")
    if parsed < int(gamma) + 2:
        raise ValueError("HELLO requires support_budget_factor >= pricing_topk + 2 "
                         f"(beta={parsed:g}, gamma={int(gamma)}, required beta>={int(gamma) + 2})")
    return parsed


def active_support_budget(beta: float, n_source: int, n_target: int) -> int:
    """ceil(beta * (m + n)) (refinement/support_budget.py:49-53)."""
    return int(math.ceil(float(beta) * (int(n_source) + int(n_target))))


def primal_support_cap(beta: float, gamma: int, n_source: int, n_target: int) -> int:
    """Positive edges an LP solution may keep: the budget minus room for a basis (V - 1) and gamma * V new
    violations (refinement/support_budget.py:56-67)."""
    vertices = int(n_source) + int(n_target)
    return active_support_budget(beta, n_source, n_target) - (vertices - 1) - int(gamma) * vertices


@dataclass(frozen=True)
class SolverOptions:
    split_count: int = 4
    coarsest_size_threshold: int = 1024
    assignment_topk: int = 16
    pricing_topk: int = 2
    support_budget_factor: float = 10.0
    fused_scan_memory_floor_mib: float = 768.0
    stopping_norm: Literal["l2", "finest_linf"] = "l2"
    verbose: Literal["off", "compact", "detailed"] = "compact"
    record_trace: bool = False
    profile_memory: bool = False
    consume_input_features: bool = False
    backend: Literal["native", "torch", "cpp"] = "native"
    torch_device: Literal["auto", "cpu", "cuda"] = "auto"
    cost_perturbation: Literal["on", "off", "auto"] = "auto"
    cost_perturbation_relative_scale: float = 0.01
    cost_precision: Literal["fp32", "fp64", "finest_fp64"] = "fp32"
    gpu_resident: bool = False
    num_threads: Optional[int] = 16
    tolerance: float = 1e-6

    def __post_init__(self) -> None:
        if isinstance(self.tolerance, bool) or not math.isfinite(self.tolerance) or self.tolerance <= 0:
            raise ValueError("tolerance must be finite and > 0")
        if not isinstance(self.gpu_resident, bool):
            raise ValueError("gpu_resident must be a boolean")
        if not isinstance(self.verbose, str) or self.verbose not in {"off", "compact", "detailed"}:
            raise ValueError("verbose must be one of: off, compact, detailed; boolean values are not supported")
        if self.stopping_norm not in {"l2", "finest_linf"}:
            raise ValueError("stopping_norm must be one of: l2, finest_linf")
        if self.cost_perturbation not in {"on", "off", "auto"}:
            raise ValueError("cost_perturbation must be one of: on, off, auto")
        if not math.isfinite(self.cost_perturbation_relative_scale) or self.cost_perturbation_relative_scale <= 0:
            raise ValueError("cost_perturbation_relative_scale must be finite and > 0; use 'off' to disable")
        if self.cost_precision not in {"fp32", "fp64", "finest_fp64"}:
            raise ValueError("cost_precision must be one of: fp32, fp64, finest_fp64")
        if self.split_count not in {2, 4, 8}:
            raise ValueError("split_count must be one of: 2, 4, 8")
        if self.coarsest_size_threshold < 1:
            raise ValueError("coarsest_size_threshold must be >= 1")
        if isinstance(self.assignment_topk, bool) or self.assignment_topk < 1:
            raise ValueError("assignment_topk must be >= 1")
        pricing_topk = normalize_pricing_topk(self.pricing_topk)
        object.__setattr__(self, "pricing_topk", pricing_topk)
        object.__setattr__(self, "support_budget_factor",
                           validate_support_budget_factor(self.support_budget_factor, pricing_topk))
        if self.fused_scan_memory_floor_mib <= 0.0:
            raise ValueError("fused_scan_memory_floor_mib must be > 0")
        if self.backend not in {"native", "torch", "cpp"}:
            raise ValueError("backend must be one of: native, torch, cpp")
        if self.num_threads is not None and (isinstance(self.num_threads, bool) or not isinstance(self.num_threads, int)
                                             or self.num_threads < 1):
            raise ValueError("num_threads must be a positive integer or None")
        if self.torch_device not in {"auto", "cpu", "cuda"}:
            raise ValueError("torch_device must be one of: auto, cpu, cuda")

    def check_supported(self) -> None:
        """Raise for options whose code path is not part of the MI355X build."""
        if self.backend != "native":
            raise NotImplementedError("the MI355X build implements backend='native' only")
        if self.torch_device == "cpu":
            raise NotImplementedError("the MI355X build runs on the GPU only (torch_device='cpu' is unsupported)")
        if self.cost_perturbation == "on":
            raise NotImplementedError("cost_perturbation='on' is not part of the MI355X build; use 'auto' or 'off'")
        if self.assignment_topk > 32 or self.pricing_topk > 32:
            raise NotImplementedError("the MI355X scans keep at most 32 candidates per row")


__all__ = ["POSITIVE_SUPPORT_TOLERANCE", "SolverOptions", "active_support_budget", "finest_stopping_norm",
           "level_precision", "level_stopping_norm", "normalize_pricing_topk", "primal_support_cap",
           "validate_support_budget_factor"]
