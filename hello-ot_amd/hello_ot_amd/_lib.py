"""ctypes binding of ``libhelloot_hip.so`` (the C ABI declared in ``include/helloot_hip.h``).

The product path has no fallback: if the HIP library is missing or cannot be loaded, every entry point
raises ``NativeUnavailableError`` instead of computing anything on the CPU.
"""
from __future__ import annotations

import ctypes
import os
import re
from pathlib import Path

LIB_NAME = "libhelloot_hip.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME
HEADER_PATH = Path(__file__).resolve().parents[2] / "include" / "helloot_hip.h"

HM_OK, HM_EINVAL, HM_EHIP, HM_ENOSPC, HM_ESOLVE = 0, 1, 2, 3, 4
HM_ROWS, HM_COLS, HM_STATS, HM_LINF, HM_BF16X3, HM_INT8X3, HM_FP64 = 1, 2, 4, 8, 16, 32, 64
COST_KINDS = {"l1": 0, "linf": 1, "l2": 2}

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_U32 = ctypes.c_uint32
_D = ctypes.c_double
_SZ = ctypes.c_size_t


class NativeUnavailableError(RuntimeError):
    """The MI355X HIP library is not built or not loadable; there is no CPU fallback."""


class PdhgParams(ctypes.Structure):
    _fields_ = [
        ("evaluation_frequency", _I32), ("rescale", _I32), ("iteration_limit", _I64),
        ("tol_objective", _D), ("tol_primal", _D), ("tol_dual", _D), ("time_limit_seconds", _D),
    ]


class PdhgResult(ctypes.Structure):
    _fields_ = [
        ("iterations", _I64), ("restarts", _I64), ("reason", _I32), ("pad", _I32),
        ("primal_objective", _D), ("dual_objective", _D), ("abs_primal", _D), ("rel_primal", _D),
        ("abs_dual", _D), ("rel_dual", _D), ("rel_gap", _D), ("primal_weight", _D), ("seconds", _D),
    ]


REASONS = {0: "UNSPECIFIED", 1: "OPTIMAL", 2: "ITERATION_LIMIT", 3: "NUMERICAL_DIVERGENCE", 4: "TIME_LIMIT"}

# name -> (restype, argtypes)
SIGNATURES = {
    "hm_last_error": (ctypes.c_char_p, []),
    "hm_abi_version": (ctypes.c_int, []),
    "hm_profile_enable": (None, [ctypes.c_int]),
    "hm_profile_reset": (None, []),
    "hm_profile_query": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(_D), ctypes.POINTER(_I64)]),
    "hm_pricing_l2sq_workspace_bytes": (_SZ, [_I64, _I64, _I32, _I32, _U32]),
    "hm_pricing_l2sq": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I32, _I32, _D, _U32,
                                       _P, _P, _P, _P, _P, _P, _SZ]),
    "hm_l2sq_resident_bytes": (_SZ, [_I64, _I32, _U32]),
    "hm_l2sq_resident_prepare": (ctypes.c_int, [_P, _P, _I64, _I32, _U32, _P, _SZ]),
    "hm_pricing_l2sq_resident_workspace_bytes": (_SZ, [_I64, _I64, _I32, _I32, _U32]),
    "hm_pricing_l2sq_resident": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I32, _I32, _D, _U32,
                                                _P, _P, _P, _P, _P, _P, _SZ, _P, _SZ]),
    "hm_pricing_l2sq_resident_floor": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I32, _I32, _D,
                                                      _U32, _P, _P, _P, _P, _P, _P, _P, _SZ, _P, _SZ]),
    "hm_pricing_norm_workspace_bytes": (_SZ, [_I64, _I64, _I32, _I32, _U32]),
    "hm_pricing_norm": (ctypes.c_int, [_P, _P, _P, _P, _P, _I64, _I64, _I32, _I32, _I32, _U32,
                                       _P, _P, _P, _P, _P, _P, _SZ]),
    "hm_pricing_norm_noalloc_max_bytes": (_SZ, []),
    "hm_pricing_norm_noalloc": (ctypes.c_int, [_P, _P, _P, _P, _P, _I64, _I64, _I32, _I32, _I32, _U32,
                                               _P, _P, _P, _P, _P]),
    "hm_sddmm_l2sq_csr": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I32, _D, _P]),
    "hm_pair_costs_l2sq": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _I64, _I32, _D, _P]),
    "hm_pair_costs_norm": (ctypes.c_int, [_P, _P, _P, _P, _P, _I64, _I32, _I32, _P]),
    "hm_pair_costs_norm_fp32": (ctypes.c_int, [_P, _P, _P, _P, _P, _I64, _I32, _I32, _P]),
    "hm_sparsify_support": (ctypes.c_int, [_I64, _I64, _I64, _P, _P, _P, _P, _I64, _D, _P]),
    "hm_transport_simplex": (ctypes.c_int, [_I64, _I64, _P, _P, _P, _I64, _P, _P, _P, _P, _P, _P, _P]),
    "hm_pdhg_workspace_bytes": (_SZ, [_I64, _I64, _I64]),
    "hm_pdhg_solve": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, ctypes.POINTER(PdhgParams),
                                     _P, _P, ctypes.POINTER(PdhgResult), _P, _SZ]),
}

_LIB = None


def header_symbols() -> list[str]:
    """Every function the C header declares (used by the export test)."""
    text = HEADER_PATH.read_text()
    return sorted(set(re.findall(r"\b(hm_[a-z0-9_]+)\s*\(", text)))


def load() -> ctypes.CDLL:
    global _LIB
    if _LIB is not None:
        return _LIB
    path = Path(os.environ.get("HELLOOT_HIP_LIB", LIB_PATH))
    if not path.exists():
        raise NativeUnavailableError(
            f"{path} is not built; run __graft_entry__.build() (make -C hello-ot_amd). "
            "The native backend has no CPU fallback.")
    try:
        lib = ctypes.CDLL(str(path))
    except OSError as exc:  # pragma: no cover - depends on the host
        raise NativeUnavailableError(f"cannot load {path}: {exc}") from exc
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.hm_abi_version() != 1:
        raise NativeUnavailableError("libhelloot_hip ABI version mismatch; rebuild the package")
    _LIB = lib
    return lib


def last_error() -> str:
    return load().hm_last_error().decode(errors="replace")


def check(rc: int, what: str) -> None:
    if rc == HM_OK:
        return
    message = f"{what}: {last_error()}"
    if rc == HM_EINVAL:
        raise ValueError(message)
    raise RuntimeError(message)


def ptr(t) -> ctypes.c_void_p:
    """Device (or host) address of a tensor, or NULL for None."""
    if t is None:
        return ctypes.c_void_p(0)
    return ctypes.c_void_p(int(t.data_ptr()))


_PROFILING = False


def profile_enable(on: bool = True) -> None:
    global _PROFILING
    load().hm_profile_enable(int(bool(on)))
    _PROFILING = bool(on)


def profiling() -> bool:
    """Whether the library's kernel timing is on (profile_enable)."""
    return _PROFILING


def profile_reset() -> None:
    load().hm_profile_reset()


def profile_query(name: str) -> tuple[float, int]:
    """(total milliseconds, launches) of one kernel since the last reset (waits for pending events)."""
    ms = _D(0.0)
    n = _I64(0)
    load().hm_profile_query(name.encode(), ctypes.byref(ms), ctypes.byref(n))
    return float(ms.value), int(n.value)


def stream_handle(device) -> ctypes.c_void_p:
    import torch

    return ctypes.c_void_p(int(torch.cuda.current_stream(device).cuda_stream))
