"""Restricted-LP result record, field for field as ``_internal/lp/wrapper.py:9-37``."""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Dict


@dataclass
class SolverResult:
    success: bool
    x: Any = None
    y: Any = None
    obj_val: float = 0.0
    dual_obj_val: float = None
    duration: float = 0.0
    iterations: int = 0
    peak_mem: float = 0.0
    termination_reason: str = None
    primal_feas: float = None
    dual_feas: float = None
    gap: float = None
    solver_diag: Dict = None
