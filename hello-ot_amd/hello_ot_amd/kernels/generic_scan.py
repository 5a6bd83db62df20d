"""MI355X pricing scans behind the reference's ``ScanExtension`` interface.

Mirrors ``hello_ot.kernels.generic_scan.ScanExtension`` (``kernels/generic_scan.py:468-597``): same method
names, argument meaning, return shapes and validation errors. Each method calls one C-ABI entry point of
``libhelloot_hip.so``; there is no CPU or PyTorch fallback.
"""
from __future__ import annotations

from collections import Counter

import torch

from .. import _lib

_ROUTES = Counter()
_BUCKETS = (1, 2, 4, 8, 16, 32)


def scan_routes(*, reset=False):
    """Route counters, as ``generic_scan.scan_routes`` (generic_scan.py:22-30)."""
    result = dict(_ROUTES)
    if reset:
        _ROUTES.clear()
    return result


def _check(x, y, k, *vectors):
    """Validation of ``generic_scan._check`` (generic_scan.py:42-56), restricted to fp32 features."""
    if k not in _BUCKETS:
        raise ValueError("generic scan requires a power-of-two bucket in [1,32]")
    if (not x.is_cuda or not y.is_cuda or x.device != y.device
            or x.dtype not in (torch.float32, torch.float64) or y.dtype != x.dtype
            or x.ndim != 2 or y.ndim != 2 or x.shape[1] != y.shape[1]
            or min(*x.shape, *y.shape) < 1 or max(*x.shape, *y.shape) >= 2**31):
        raise ValueError("generic scan requires nonempty matching CUDA FP32/FP64 feature matrices with int32 dimensions")
    if x.dtype != torch.float32:
        raise ValueError("the MI355X scan computes from FP32 feature storage (compute_precision='fp32')")
    for v, count in vectors:
        if v.device != x.device or v.dtype != torch.float64 or v.numel() != count:
            raise ValueError("generic scan requires matching CUDA FP64 bias vectors")


def _c(t):
    return t.contiguous()


def _workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


SWEEP_PRECISIONS = ("auto", "fp32", "bf16x3", "int8x3")
SPLIT_MIN_D = 64    # "auto" sweeps on split-bf16 MFMA from this feature count on (faster than fp32 at d = 64)
INT8_MIN_D = 256    # ... and on the int8 split from this one on (MI355X, whole calls: 1.05x at d = 256, 1.30x at
                    # 1024, 1.46x at 4096; the C5 sweep 1.85x at 8192)
INT8_MAX_D = 65536  # the int8 sweep's int32 sums hold up to this many features


def sweep_precision(precision: str, d: int) -> str:
    if precision not in SWEEP_PRECISIONS:
        raise ValueError(f"precision must be one of {SWEEP_PRECISIONS}")
    if precision == "auto":
        if INT8_MIN_D <= d <= INT8_MAX_D:
            return "int8x3"
        return "bf16x3" if d >= SPLIT_MIN_D else "fp32"
    if precision == "int8x3" and d > INT8_MAX_D:
        raise ValueError(f"the int8 sweep supports d <= {INT8_MAX_D}")
    return precision


def _precision_flags(precision: str) -> int:
    return (_lib.HM_BF16X3 if precision == "bf16x3" else 0) | (_lib.HM_INT8X3 if precision == "int8x3" else 0)


class ResidentSide:
    """The Y side of chunked l2^2 scans prepared once on the device (``hm_l2sq_resident_prepare``): its norms, its
    sweep copy for ``precision`` and the int8 scales and error terms. The reference's chunked check places one side
    on the device the same way and streams query chunks against it (kernels/bilinear_topk.py:255-293).
    ``pricing_l2sq(..., resident=side)`` then skips the side's preparation; ``y`` must stay unchanged."""

    def __init__(self, y, precision: str = "auto"):
        lib = _lib.load()
        self.y = _c(y)
        self.n, self.d = int(self.y.shape[0]), int(self.y.shape[1])
        self.precision = sweep_precision(precision, self.d)
        flags = _precision_flags(self.precision)
        dev = self.y.device
        self.buffer = _workspace(lib.hm_l2sq_resident_bytes(self.n, self.d, flags), dev)
        with torch.cuda.device(dev):
            rc = lib.hm_l2sq_resident_prepare(_lib.stream_handle(dev), _lib.ptr(self.y), self.n, self.d, flags,
                                              _lib.ptr(self.buffer), self.buffer.numel())
        _lib.check(rc, "hm_l2sq_resident_prepare")


def pricing_l2sq(x, y, nx, ny, qb, dbb, k, *, dot_scale=2.0, rows=True, cols=True, stats=True, linf=False,
                 precision="auto", resident: ResidentSide | None = None, col_floor=None):
    """Raw l2^2 pricing: returns (row_vals, row_idx, col_vals, col_idx, stats5) with None for skipped parts.

    ``stats5`` = (num, den, count, max sigma+, max|cost|); max|cost| is 0 unless ``linf``. ``precision`` picks the
    candidate sweep: ``"fp32"`` MFMA, ``"bf16x3"`` split-bf16 MFMA (three products), ``"int8x3"`` int8 MFMA over a
    16-bit fixed-point split (three exact int32 products, d <= 65536) or ``"auto"`` (split-bf16 from d = SPLIT_MIN_D
    on); all feed the same exact fp64 re-evaluation, so the outputs are identical and only the speed (and the
    rescan rate) differs. With ``resident`` (a ``ResidentSide`` of ``y``) the side's preparation is reused and the
    precision is the side's.

    ``col_floor`` (with ``resident`` and ``cols``): fp64 per column of ``y``, a score the caller's own list of that
    column already reaches k times. Column entries scoring below it may then be left out (padded with -inf / -1);
    merging the outputs into the caller's lists gives what the full lists give.
    """
    if col_floor is not None and (resident is None or not cols):
        raise ValueError("col_floor needs a resident side and the column lists")
    if resident is not None:
        if precision not in ("auto", resident.precision):
            raise ValueError(f"the resident side was prepared for precision {resident.precision!r}")
        if y.data_ptr() != resident.y.data_ptr() or tuple(y.shape) != (resident.n, resident.d):
            raise ValueError("pricing against a resident side needs the tensor it was prepared from")
        precision, y = resident.precision, resident.y
    precision = sweep_precision(precision, int(x.shape[1]))
    lib = _lib.load()
    x, y, nx, ny, qb, dbb = map(_c, (x, y, nx, ny, qb, dbb))
    m, n, d = x.shape[0], y.shape[0], x.shape[1]
    flags = (_lib.HM_ROWS if rows else 0) | (_lib.HM_COLS if cols else 0) | (_lib.HM_STATS if stats else 0) \
        | (_lib.HM_LINF if (stats and linf) else 0) | _precision_flags(precision)
    dev = x.device
    rv = torch.empty((m, k), dtype=torch.float64, device=dev) if rows else None
    ri = torch.empty((m, k), dtype=torch.int32, device=dev) if rows else None
    cv = torch.empty((n, k), dtype=torch.float64, device=dev) if cols else None
    ci = torch.empty((n, k), dtype=torch.int32, device=dev) if cols else None
    st = torch.zeros(5, dtype=torch.float64, device=dev) if stats else None
    if resident is None:
        ws = _workspace(lib.hm_pricing_l2sq_workspace_bytes(m, n, d, k, flags), dev)
        with torch.cuda.device(dev):
            rc = lib.hm_pricing_l2sq(_lib.stream_handle(dev), _lib.ptr(x), _lib.ptr(y), _lib.ptr(nx), _lib.ptr(ny),
                                     _lib.ptr(qb), _lib.ptr(dbb), m, n, d, k, float(dot_scale), flags, _lib.ptr(rv),
                                     _lib.ptr(ri), _lib.ptr(cv), _lib.ptr(ci), _lib.ptr(st), _lib.ptr(ws), ws.numel())
        _lib.check(rc, "hm_pricing_l2sq")
        return rv, ri, cv, ci, st
    if col_floor is not None:
        col_floor = _c(col_floor)
        if col_floor.dtype != torch.float64 or tuple(col_floor.shape) != (n,) or col_floor.device != dev:
            raise ValueError(f"col_floor must be a float64 vector of {n} values on {dev}")
    ws = _workspace(lib.hm_pricing_l2sq_resident_workspace_bytes(m, n, d, k, flags), dev)
    with torch.cuda.device(dev):
        rc = lib.hm_pricing_l2sq_resident_floor(_lib.stream_handle(dev), _lib.ptr(x), _lib.ptr(y), _lib.ptr(nx),
                                                _lib.ptr(ny), _lib.ptr(qb), _lib.ptr(dbb), m, n, d, k,
                                                float(dot_scale), flags, _lib.ptr(col_floor), _lib.ptr(rv),
                                                _lib.ptr(ri), _lib.ptr(cv), _lib.ptr(ci), _lib.ptr(st),
                                                _lib.ptr(resident.buffer), resident.buffer.numel(), _lib.ptr(ws),
                                                ws.numel())
    _lib.check(rc, "hm_pricing_l2sq_resident_floor")
    return rv, ri, cv, ci, st


NORM_PRECISIONS = ("fp32", "fp64")


def pricing_norm(x, y, f, g, k, cost_type, *, rows=True, cols=True, stats=True, linf=True, precision="fp32"):
    """l1 / linf / l2 pricing (cost_type 0/1/2): (row_vals, row_idx, col_vals, col_idx, stats5). ``precision``
    "fp32" ranks by the reference's fp32 chunked costs, "fp64" by its fp64 costs (compute_precision = 1)."""
    if precision not in NORM_PRECISIONS:
        raise ValueError(f"precision must be one of {NORM_PRECISIONS}")
    lib = _lib.load()
    x, y, f, g = map(_c, (x, y, f, g))
    m, n, d = x.shape[0], y.shape[0], x.shape[1]
    flags = (_lib.HM_ROWS if (rows or stats) else 0) | (_lib.HM_COLS if cols else 0) \
        | (_lib.HM_STATS if stats else 0) | (_lib.HM_LINF if (stats and linf) else 0) \
        | (_lib.HM_FP64 if precision == "fp64" else 0)
    dev = x.device
    need_rows = bool(flags & _lib.HM_ROWS)
    rv = torch.empty((m, k), dtype=torch.float64, device=dev) if need_rows else None
    ri = torch.empty((m, k), dtype=torch.int32, device=dev) if need_rows else None
    cv = torch.empty((n, k), dtype=torch.float64, device=dev) if cols else None
    ci = torch.empty((n, k), dtype=torch.int32, device=dev) if cols else None
    st = torch.zeros(5, dtype=torch.float64, device=dev) if stats else None
    ws = _workspace(lib.hm_pricing_norm_workspace_bytes(m, n, d, k, flags), dev)
    with torch.cuda.device(dev):
        rc = lib.hm_pricing_norm(_lib.stream_handle(dev), _lib.ptr(x), _lib.ptr(y), _lib.ptr(f), _lib.ptr(g), m, n, d,
                                 k, int(cost_type), flags, _lib.ptr(rv), _lib.ptr(ri), _lib.ptr(cv), _lib.ptr(ci),
                                 _lib.ptr(st), _lib.ptr(ws), ws.numel())
    _lib.check(rc, "hm_pricing_norm")
    return (rv if rows else None), (ri if rows else None), cv, ci, st


_NORM_PRECISION = {0: "fp32", 1: "fp64"}  # compute_precision of the reference's norm scans


class ScanExtension:
    """Unified scan entry points (generic_scan.py:468-597) on MI355X HIP kernels."""

    supports_assignment_statistics = False
    supports_cost_perturbation = False
    supports_fp64_accumulation = True
    index_hash_arithmetic = None

    def __init__(self):
        self.routes = Counter()
        self.last_backend = "mi355x"

    def _record(self, name):
        key = name + ":mi355x"
        self.routes[key] += 1
        _ROUTES[key] += 1

    # -- (a) l2^2 pricing -------------------------------------------------------------------------------
    def fused_bidir_topk_stats_raw(self, query_feat, db_feat, query_cost, db_cost, query_bias, db_bias,
                                   query_tile, db_tile, col_reduce_tile, k, compute_stats,
                                   collect_linf_stats, collect_timing, col_kernel, dot_scale):
        """generic_scan.py:577-597 -> [q_vals f64(q,k), q_idx i32(q,k), r_vals f64(n,k), r_idx i32(n,k),
        stats f64(4) = (num, den, count, max|cost| if collect_linf_stats), timing f64(4) on CPU (zeros)]."""
        x, y, nx, ny, qb, dbb = query_feat, db_feat, query_cost, db_cost, query_bias, db_bias
        if x.dtype != y.dtype:
            raise RuntimeError("query/db feature dtypes must match")
        _check(x, y, k, (nx, len(x)), (ny, len(y)), (qb, len(x)), (dbb, len(y)))
        if (query_tile <= 0 or db_tile <= 0 or not 0 < col_reduce_tile <= 256 or dot_scale not in (1., 2.)
                or col_kernel not in (0, 1, 2) or (col_kernel == 1 and k != 4) or (col_kernel == 2 and k != 2)):
            raise ValueError("invalid raw pricing tile, scale or column mode")
        self._record("raw_pricing")
        rv, ri, cv, ci, st = pricing_l2sq(x, y, nx, ny, qb, dbb, k, dot_scale=float(dot_scale), rows=True, cols=True,
                                          stats=bool(compute_stats), linf=bool(collect_linf_stats))
        if compute_stats:
            stats = torch.stack((st[0], st[1], st[2], st[4] if collect_linf_stats else st[4].new_zeros(())))
        else:
            stats = torch.zeros(4, dtype=torch.float64, device=x.device)
        return [rv, ri, cv, ci, stats, torch.zeros(4, dtype=torch.float64, device="cpu")]

    def raw_lowrank_stats_only(self, x, y, nx, ny, f, g, query_tile, db_tile, dot_scale):
        """Certificate only (generic_scan.py:502-510): f64(5) = (num, den, count, max, costmax)."""
        if query_tile <= 0 or db_tile <= 0:
            raise ValueError("tile sizes must be positive")
        _check(x, y, 1, (nx, len(x)), (ny, len(y)), (f, len(x)), (g, len(y)))
        if dot_scale not in (1., 2.):
            raise ValueError("invalid raw certificate scale or precision")
        self._record("raw_certificate")
        qb, dbb = f - nx, g - ny
        _, _, _, _, st = pricing_l2sq(x, y, nx, ny, qb, dbb, 1, dot_scale=float(dot_scale), rows=False, cols=False,
                                      stats=True, linf=True)
        return st

    def initialization_directional_topk_raw(self, query_feat, db_feat, query_bias, db_bias, query_tile, db_tile, k,
                                            dot_scale):
        """generic_scan.py:560-575 -> [values f64(q,k), indices i32(q,k)]: per query row the k largest raw scores
        (dot_scale * <x_i, y_j> + query_bias_i) + db_bias_j, descending, the lowest index first among equal scores
        (the rows-only l2^2 sweep; the query tile sizes are planning hints there and here)."""
        x, y, qb, dbb = query_feat, db_feat, query_bias, db_bias
        if x.dtype != y.dtype:
            raise RuntimeError("query/db feature dtypes must match")
        _check(x, y, k, (qb, len(x)), (dbb, len(y)))
        if query_tile <= 0 or db_tile <= 0 or dot_scale not in (1., 2.):
            raise ValueError("invalid raw directional tile or scale")
        self._record("raw_initial")
        zx = torch.zeros(len(x), dtype=torch.float64, device=x.device)   # costs enter only the certificate
        zy = torch.zeros(len(y), dtype=torch.float64, device=x.device)
        rv, ri, _, _, _ = pricing_l2sq(x, y, zx, zy, qb, dbb, k, dot_scale=float(dot_scale), rows=True, cols=False,
                                       stats=False, linf=False)
        return [rv, ri]

    def fused_directional_topk_raw(self, query_feat, db_feat, query_bias, db_bias, query_tile, db_tile, k, dot_scale):
        """generic_scan.py:512-518: the directional compatibility name of initialization_directional_topk_raw."""
        self._record("raw_directional")
        return self.initialization_directional_topk_raw(query_feat, db_feat, query_bias, db_bias, query_tile, db_tile,
                                                        k, dot_scale)

    # -- (a) norm pricing -----------------------------------------------------------------------------
    def fused_gcost_topk(self, query, db, dual_db, k, cost_type, query_global_index=None, database_global_index=None,
                         sigma=0., seed=0, perturb_mode=1, row_is_source=True, index_hash_coeffs=None,
                         compute_precision=0, collect_statistics=False):
        """generic_scan.py:520-531 -> [values f64(q,k), indices i64(q,k)]: per query row the k smallest
        cost_ij - dual_db_j, ascending, the lowest index first among equal values (the rows-only norm sweep with zero
        query duals: its scores are dual_db_j - cost_ij exactly, so their negations are cost - dual exactly)."""
        _check(query, db, k, (dual_db, len(db)))
        if cost_type not in (0, 1, 2):
            raise ValueError("generic directional cost must be l1, linf, l2 or raw")
        if compute_precision not in (0, 1):
            raise ValueError("norm scans require FP32 coordinate storage and precision 0 or 1")
        if float(sigma) != 0.0:
            raise NotImplementedError("cost perturbation is not part of the MI355X native pricing path")
        if collect_statistics:
            raise NotImplementedError("assignment statistics are not collected by the MI355X norm scan")
        self._record("norm_initial")
        zero = torch.zeros(len(query), dtype=torch.float64, device=query.device)
        rv, ri, _, _, _ = pricing_norm(query, db, zero, dual_db, k, cost_type, rows=True, cols=False, stats=False,
                                       linf=False, precision=_NORM_PRECISION[compute_precision])
        return [rv.neg(), ri.long()]

    def fused_gcost_certificate(self, query, db, query_dual, db_dual, cost_type, query_global_index=None,
                                database_global_index=None, sigma=0., seed=0, perturb_mode=1, row_is_source=True,
                                index_hash_coeffs=None, compute_denominator=1, compute_precision=0):
        """generic_scan.py:545-558 -> [num, den, max, costmax, count i64] of the norm certificate over all pairs
        (den is zero when compute_denominator is off); the six-argument form passes compute_denominator sixth."""
        if isinstance(query_global_index, (int, bool)) and database_global_index is None:
            compute_denominator, query_global_index = query_global_index, None
        _check(query, db, 1, (query_dual, len(query)), (db_dual, len(db)))
        if cost_type not in (0, 1, 2):
            raise ValueError("certificate-only requires a norm or raw cost")
        if compute_precision not in (0, 1):
            raise ValueError("norm scans require FP32 coordinate storage and precision 0 or 1")
        if float(sigma) != 0.0:
            raise NotImplementedError("cost perturbation is not part of the MI355X native pricing path")
        self._record("norm_certificate")
        _, _, _, _, st = pricing_norm(query, db, query_dual, db_dual, 1, cost_type, rows=True, cols=False, stats=True,
                                      linf=True, precision=_NORM_PRECISION[compute_precision])
        den = st[1] if compute_denominator else torch.zeros_like(st[1])
        return [st[0], den, st[3], st[4], st[2].long()]

    def fused_gcost_bidir_certificate(self, query, db, query_dual, db_dual, k, cost_type,
                                      query_global_index=None, database_global_index=None, sigma=0., seed=0,
                                      perturb_mode=1, row_is_source=True, index_hash_coeffs=None,
                                      compute_precision=0, rows_per_block_hint=8):
        """generic_scan.py:533-543 -> [q_vals, q_idx i64, r_vals, r_idx i64, num, den, max, costmax, count]."""
        _check(query, db, k, (query_dual, len(query)), (db_dual, len(db)))
        if cost_type not in (0, 1, 2):
            raise ValueError("generic bidirectional cost must be l1, linf, l2 or raw")
        if compute_precision not in (0, 1):
            raise ValueError("norm scans require FP32 coordinate storage and precision 0 or 1")
        if float(sigma) != 0.0:
            raise NotImplementedError("cost perturbation is not part of the MI355X native pricing path")
        self._record("norm_pricing")
        rv, ri, cv, ci, st = pricing_norm(query, db, query_dual, db_dual, k, cost_type, rows=True, cols=True,
                                          stats=True, linf=True, precision=_NORM_PRECISION[compute_precision])
        return [rv, ri.long(), cv, ci.long(), st[0], st[1], st[3], st[4], st[2].long()]

    # -- (b) SDDMM / pair costs -------------------------------------------------------------------------
    def fused_gcost_pairs(self, query, db, rows, cols, cost_type, source_index=None, target_index=None,
                          sigma=0.0, seed=0, mode=1, coefficients=None):
        """fp64 norm costs of selected pairs (norm_cost_scan_kernel.cu:249-275), without perturbation."""
        if float(sigma) != 0.0:
            raise NotImplementedError("cost perturbation is not part of the MI355X native pair-cost path")
        from ..costs.pairs import norm_pair_costs

        self._record("norm_pairs")
        return norm_pair_costs(query, db, rows, cols, cost_type)


__all__ = ["ResidentSide", "ScanExtension", "pricing_l2sq", "pricing_norm", "scan_routes"]
