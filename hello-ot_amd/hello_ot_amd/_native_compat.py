"""Native-runtime gate for the MI355X backend.

Replaces ``hello_ot._native_compat`` (``_native_compat.py:6-46``), which pins torch 2.7.1 + CUDA 11.8: the
native backend here needs a ROCm build of PyTorch, a visible gfx950 device and the in-tree HIP library.
"""
from __future__ import annotations

import torch

from . import _lib

NATIVE_ARCH = "gfx950"


def native_runtime_compatibility() -> tuple[bool, str]:
    if getattr(torch.version, "hip", None) is None:
        return False, f"expected a ROCm build of PyTorch; found torch={torch.__version__} without HIP"
    if not _lib.LIB_PATH.exists():
        return False, f"{_lib.LIB_PATH.name} is not built (run __graft_entry__.build())"
    if not torch.cuda.is_available():
        return False, "no ROCm GPU is visible"
    arch = torch.cuda.get_device_properties(0).gcnArchName.split(":")[0]
    if arch != NATIVE_ARCH:
        return False, f"expected a {NATIVE_ARCH} (MI355X) device; found {arch}"
    return True, f"torch={torch.__version__} hip={torch.version.hip} arch={arch}"


def require_native_runtime_compatibility() -> None:
    compatible, detail = native_runtime_compatibility()
    if not compatible:
        raise RuntimeError(
            "The native backend requires the MI355X (gfx950) ROCm stack: "
            f"{detail}. The explicit torch backend remains available.")
