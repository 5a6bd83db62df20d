"""SDDMM cost evaluation on the active support (MI355X HIP kernels).

* ``lowrank_pair_costs``: l2^2 ("lowrank") costs c_e = (p_i + q_j) - s*<x_i, y_j> for arbitrary pairs, the
  role of ``costs/pairs._cost_pairs_lowrank_batched`` (``costs/pairs.py:221-437``) and
  ``gpu_resident.cost.Cost.pairs`` (``gpu_resident/cost.py:59-71``), with fp64 accumulation.
* ``lowrank_csr_costs``: the same on a CSR support (rows sorted, ``rowptr``/``col``), the layout the
  reference builds on the host before ``torch.sparse.sampled_addmm`` (``costs/pairs.py:309-407``).
* ``norm_pair_costs``: fp64 l1 / linf / l2 costs, ``fused_gcost_pairs`` without perturbation
  (``_native/norm_cost_scan/norm_cost_scan_kernel.cu:233-275``).
"""
from __future__ import annotations

import torch

from .. import _lib


def _features(x, y):
    if (not x.is_cuda or x.device != y.device or x.dtype != torch.float32 or y.dtype != torch.float32
            or x.ndim != 2 or y.ndim != 2 or x.shape[1] != y.shape[1] or x.shape[1] < 1):
        raise ValueError("pair costs require matching CUDA FP32 feature matrices")
    return x.contiguous(), y.contiguous()


def lowrank_pair_costs(source_feat, target_feat, source_offset, target_offset, rows, cols, *, dot_scale=2.0):
    x, y = _features(source_feat, target_feat)
    if dot_scale not in (1.0, 2.0):
        raise ValueError("dot_scale must be exactly 1 or 2")
    rows = torch.as_tensor(rows, device=x.device).to(torch.int64).contiguous().view(-1)
    cols = torch.as_tensor(cols, device=x.device).to(torch.int64).contiguous().view(-1)
    if rows.numel() != cols.numel():
        raise ValueError("pair indices must be matching int64 arrays")
    p = source_offset.to(device=x.device, dtype=torch.float64).contiguous()
    q = target_offset.to(device=x.device, dtype=torch.float64).contiguous()
    if p.numel() != x.shape[0] or q.numel() != y.shape[0]:
        raise ValueError("offsets must match the feature rows")
    out = torch.empty(rows.numel(), dtype=torch.float64, device=x.device)
    if rows.numel() == 0:
        return out
    if int(rows.min()) < 0 or int(rows.max()) >= x.shape[0] or int(cols.min()) < 0 or int(cols.max()) >= y.shape[0]:
        raise ValueError("pair index is out of bounds")
    lib = _lib.load()
    with torch.cuda.device(x.device):
        rc = lib.hm_pair_costs_l2sq(_lib.stream_handle(x.device), _lib.ptr(x), _lib.ptr(y), _lib.ptr(p), _lib.ptr(q),
                                    _lib.ptr(rows), _lib.ptr(cols), rows.numel(), x.shape[1], float(dot_scale),
                                    _lib.ptr(out))
    _lib.check(rc, "hm_pair_costs_l2sq")
    return out


def lowrank_csr_costs(source_feat, target_feat, source_offset, target_offset, rowptr, col, *, dot_scale=2.0):
    x, y = _features(source_feat, target_feat)
    if dot_scale not in (1.0, 2.0):
        raise ValueError("dot_scale must be exactly 1 or 2")
    rowptr = rowptr.to(device=x.device, dtype=torch.int32).contiguous()
    col = col.to(device=x.device, dtype=torch.int32).contiguous()
    if rowptr.numel() != x.shape[0] + 1:
        raise ValueError("rowptr must have m + 1 entries")
    p = source_offset.to(device=x.device, dtype=torch.float64).contiguous()
    q = target_offset.to(device=x.device, dtype=torch.float64).contiguous()
    out = torch.empty(col.numel(), dtype=torch.float64, device=x.device)
    if int(rowptr[0]) != 0 or int(rowptr[-1]) != col.numel() or bool((rowptr[1:] < rowptr[:-1]).any()):
        raise ValueError("rowptr must start at 0, end at nnz and be non-decreasing")
    if col.numel() == 0:
        return out
    if int(col.min()) < 0 or int(col.max()) >= y.shape[0]:
        raise ValueError("CSR column index is out of bounds")
    lib = _lib.load()
    with torch.cuda.device(x.device):
        rc = lib.hm_sddmm_l2sq_csr(_lib.stream_handle(x.device), _lib.ptr(x), _lib.ptr(y), _lib.ptr(p), _lib.ptr(q),
                                   _lib.ptr(rowptr), _lib.ptr(col), x.shape[0], col.numel(), x.shape[1],
                                   float(dot_scale), _lib.ptr(out))
    _lib.check(rc, "hm_sddmm_l2sq_csr")
    return out


def norm_pair_costs(query, db, rows, cols, cost_type, *, precision="fp64"):
    """fp64 norm costs (``precision="fp64"``), or the fp32 cost the norm pricing scan ranks with, widened to fp64
    (``precision="fp32"``: 32-feature chunks accumulated in fp32, as ``costs/pairs.py:88-218`` evaluates
    pairs for ``cost_precision="fp32"``)."""
    x, y = _features(query, db)
    if precision not in ("fp32", "fp64"):
        raise ValueError("precision must be fp32 or fp64")
    if cost_type not in (0, 1, 2):
        raise ValueError("unsupported norm cost")
    rows = torch.as_tensor(rows, device=x.device).to(torch.int64).contiguous().view(-1)
    cols = torch.as_tensor(cols, device=x.device).to(torch.int64).contiguous().view(-1)
    if rows.numel() != cols.numel():
        raise ValueError("pair indices must be matching int64 arrays")
    out = torch.empty(rows.numel(), dtype=torch.float64, device=x.device)
    if rows.numel() == 0:
        return out
    if int(rows.min()) < 0 or int(rows.max()) >= x.shape[0] or int(cols.min()) < 0 or int(cols.max()) >= y.shape[0]:
        raise ValueError("pair index is out of bounds")
    lib = _lib.load()
    fn = lib.hm_pair_costs_norm if precision == "fp64" else lib.hm_pair_costs_norm_fp32
    with torch.cuda.device(x.device):
        rc = fn(_lib.stream_handle(x.device), _lib.ptr(x), _lib.ptr(y), _lib.ptr(rows), _lib.ptr(cols), rows.numel(),
                x.shape[1], int(cost_type), _lib.ptr(out))
    _lib.check(rc, "hm_pair_costs_norm")
    return out


__all__ = ["lowrank_pair_costs", "lowrank_csr_costs", "norm_pair_costs"]
