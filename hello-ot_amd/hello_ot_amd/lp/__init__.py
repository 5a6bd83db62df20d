"""Restricted-OT LP solver (Halpern-PDHG) on MI355X."""
from .native_pdlp import NativeRestrictedOTPDLP
from .wrapper import SolverResult

__all__ = ["NativeRestrictedOTPDLP", "SolverResult"]
