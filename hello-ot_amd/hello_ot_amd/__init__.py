"""MI355X-native HELLO hot path: pricing scan, SDDMM cost evaluation and restricted-LP Halpern-PDHG.

Host-side mirror of the reference's native operator interfaces over ``libhelloot_hip.so``:

* ``kernels.generic_scan.ScanExtension`` -- pricing scans (``hello_ot/kernels/generic_scan.py:468-597``)
* ``costs.pairs`` -- SDDMM / pair costs on the active support (``hello_ot/costs/pairs.py:221-437``)
* ``lp.NativeRestrictedOTPDLP`` -- restricted-OT PDHG (``hello_ot/_internal/lp/torch_restricted_ot.py``)

and the HELLO front end that drives them on the GPU: ``solve`` / ``SolverOptions`` / ``Problem`` / ``Result``
(``hello_ot/__init__.py:40-90``).
"""
from ._lib import NativeUnavailableError, header_symbols, load as load_library
from ._native_compat import native_runtime_compatibility, require_native_runtime_compatibility
from .api import solve, solve_problem
from .config import SolverOptions
from .types import HelloSolveError, Problem, Result, SparseOTSolution

__version__ = "0.2.0"
API_VERSION = 1

__all__ = ["HelloSolveError", "NativeUnavailableError", "Problem", "Result", "SolverOptions", "SparseOTSolution",
           "header_symbols", "load_library", "native_runtime_compatibility", "require_native_runtime_compatibility",
           "solve", "solve_problem", "API_VERSION"]
