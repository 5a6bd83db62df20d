"""C-ABI library checks that need no GPU: it loads, exports every declared symbol, and rejects invalid
arguments before touching a device."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from hello_ot_amd import _lib


def test_library_exports_every_header_symbol():
    lib = _lib.load()
    declared = _lib.header_symbols()
    assert len(declared) >= 11
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_lib.SIGNATURES)
    assert lib.hm_abi_version() == 1


def test_invalid_arguments_fail_before_any_device_work():
    lib = _lib.load()
    one = ctypes.c_void_p(16)  # never dereferenced: validation rejects the call first
    rc = lib.hm_pricing_l2sq(None, one, one, one, one, one, one, 10, 10, 4, 0, 2.0, 1, one, one, one, one, one,
                             one, 1 << 20)
    assert rc == _lib.HM_EINVAL and "1 <= k <= 32" in _lib.last_error()
    rc = lib.hm_pricing_l2sq(None, one, one, one, one, one, one, 10, 10, 4, 2, 3.0, 1, one, one, one, one, one,
                             one, 1 << 20)
    assert rc == _lib.HM_EINVAL and "dot_scale" in _lib.last_error()
    rc = lib.hm_pricing_l2sq(None, one, one, one, one, one, one, 10, 10, 4, 2, 2.0, 1, one, one, one, one, one,
                             one, 16)
    assert rc == _lib.HM_ENOSPC
    rc = lib.hm_pricing_norm(None, one, one, one, one, 10, 10, 4, 2, 7, 1, one, one, one, one, one, one, 1 << 20)
    assert rc == _lib.HM_EINVAL and "unsupported norm cost" in _lib.last_error()
    rc = lib.hm_sddmm_l2sq_csr(None, one, one, one, one, one, one, 10, 10, 4, 3.0, one)
    assert rc == _lib.HM_EINVAL
    assert lib.hm_sddmm_l2sq_csr(None, None, None, None, None, None, None, 0, 0, 4, 2.0, None) == _lib.HM_OK
    assert lib.hm_pair_costs_norm(None, None, None, None, None, 0, 4, 0, None) == _lib.HM_OK
    params = _lib.PdhgParams(0, 0, 10, 1e-6, 1e-6, 1e-6, 1.0)
    res = _lib.PdhgResult()
    rc = lib.hm_pdhg_solve(None, one, one, one, one, None, None, 2, 2, 4, params, one, one, res, one, 1 << 20)
    assert rc == _lib.HM_EINVAL and "runtime limits" in _lib.last_error()


def test_workspace_queries_are_host_arithmetic():
    lib = _lib.load()
    small = lib.hm_pricing_l2sq_workspace_bytes(1000, 1000, 64, 8, 7)
    big = lib.hm_pricing_l2sq_workspace_bytes(131072, 131072, 64, 8, 7)
    assert 0 < small < big
    # C5: the per-chunk column partial lists are capped at 12 GiB (query chunks shrink to fit), the rest is
    # small next to the 2 x 39 GiB feature matrices
    c5 = lib.hm_pricing_l2sq_workspace_bytes(1_280_000, 1_280_000, 8192, 2, 7)
    assert 12 << 30 < c5 < 14 << 30
    c5_rows = lib.hm_pricing_l2sq_workspace_bytes(1_280_000, 1_280_000, 8192, 2, 5)  # rows + stats only
    assert c5_rows < 1 << 30
    assert lib.hm_pricing_l2sq_workspace_bytes(0, 10, 4, 2, 7) == 0
    assert lib.hm_pricing_norm_workspace_bytes(524288, 524288, 8, 2, 7) > 0


def test_resident_side_sizes_and_validation():
    """A resident Y side holds its norms and sweep copy (two bytes per feature for the int8 split, four for
    split-bf16, none for fp32); a call against it needs that much less workspace. Invalid calls fail before any
    device work."""
    lib = _lib.load()
    n, d = 1_280_000, 8192
    i8, bf = _lib.HM_INT8X3, _lib.HM_BF16X3
    r_i8, r_bf, r_32 = (lib.hm_l2sq_resident_bytes(n, d, f) for f in (i8, bf, 0))
    assert 2 * n * d < r_i8 < 2 * n * d * 1.02 + (64 << 20)
    assert 4 * n * d < r_bf < 4 * n * d * 1.02 + (64 << 20)
    assert 8 * n <= r_32 < 8 * n + (1 << 20)
    full = lib.hm_pricing_l2sq_workspace_bytes(8192, n, d, 2, 7 | i8)
    part = lib.hm_pricing_l2sq_resident_workspace_bytes(8192, n, d, 2, 7 | i8)
    assert full - part >= 2 * n * d
    assert lib.hm_l2sq_resident_bytes(0, d, i8) == 0
    one = ctypes.c_void_p(16)  # never dereferenced
    rc = lib.hm_l2sq_resident_prepare(None, one, 10, 4, i8 | bf, one, 1 << 20)
    assert rc == _lib.HM_EINVAL and "exclude each other" in _lib.last_error()
    rc = lib.hm_l2sq_resident_prepare(None, one, 10, 4, i8, one, 16)
    assert rc == _lib.HM_ENOSPC
    rc = lib.hm_pricing_l2sq_resident(None, one, one, one, one, one, one, 10, 10, 4, 2, 2.0, 1, one, one, one, one,
                                      one, None, 1 << 20, one, 1 << 20)
    assert rc == _lib.HM_EINVAL and "resident side buffer" in _lib.last_error()
    rc = lib.hm_pricing_l2sq_resident(None, one, one, one, one, one, one, 10, 10, 4, 2, 2.0, 1, one, one, one, one,
                                      one, one, 8, one, 1 << 20)
    assert rc == _lib.HM_EINVAL and "resident buffer smaller" in _lib.last_error()
    rc = lib.hm_pricing_l2sq_resident_floor(None, one, one, one, one, one, one, 10, 10, 4, 2, 2.0, 1, one, one, one,
                                            one, one, one, one, 1 << 20, one, 1 << 20)
    assert rc == _lib.HM_EINVAL and "column floor needs HM_COLS" in _lib.last_error()


def test_python_mirror_rejects_host_tensors_like_the_reference():
    from hello_ot_amd.kernels.generic_scan import ScanExtension

    x = torch.zeros(4, 2)
    v = torch.zeros(4, dtype=torch.float64)
    with pytest.raises(ValueError, match="CUDA FP32/FP64 feature matrices"):
        ScanExtension().fused_bidir_topk_stats_raw(x, x, v, v, v, v, 4, 4, 256, 2, True, False, False, 2, 2.0)
    with pytest.raises(ValueError, match="power-of-two bucket"):
        ScanExtension().fused_bidir_topk_stats_raw(x, x, v, v, v, v, 4, 4, 256, 3, True, False, False, 0, 2.0)


def test_pdlp_mirror_contract_on_host():
    from hello_ot_amd.lp import NativeRestrictedOTPDLP, SolverResult

    with pytest.raises(ValueError):
        NativeRestrictedOTPDLP(device="cpu")
    fields = set(SolverResult.__dataclass_fields__)
    assert {"success", "x", "y", "obj_val", "dual_obj_val", "iterations", "termination_reason", "primal_feas",
            "dual_feas", "gap", "solver_diag"} <= fields


def test_native_gate_reports_missing_gpu():
    from hello_ot_amd import native_runtime_compatibility

    ok, detail = native_runtime_compatibility()
    if not torch.cuda.is_available():
        assert not ok and detail
