"""``hierot_generic_pricing_small_ext`` (reference ``_native/generic_scan/pricing_small.cu:230-319``) on MI355X."""
from __future__ import annotations

from hello_ot_amd.kernels.generic_scan import ScanExtension

from ._unsupported import missing

_EXT = ScanExtension()


def raw_scan_tiled(x, y, nx, ny, qb, dbb, k, scale, stats_enabled, linf, query_tile, db_tile):
    """pricing_small.cu:298-304 -> [row_vals f64(q,k), row_idx i32(q,k), col_vals f64(n,k), col_idx i32(n,k),
    stats f64(4) = (num, den, count, max|cost| when linf), timing f64(4) on the CPU (zeros)]; k in {1, 2}.
    Scores are (scale * <x_i, y_j> + qb_i) + dbb_j and costs (nx_i + ny_j) - scale * <x_i, y_j>; the tile sizes
    are the caller's plan, which the fused MI355X sweep replaces with its own."""
    if query_tile <= 0 or db_tile <= 0 or k not in (1, 2):
        raise RuntimeError("Invalid raw pricing tile or bucket")
    return _EXT.fused_bidir_topk_stats_raw(x, y, nx, ny, qb, dbb, query_tile, db_tile, 256, k, bool(stats_enabled),
                                           bool(linf), False, 0, float(scale))


__getattr__ = missing("hierot_generic_pricing_small_ext",
                      {"raw_scan": "raw_scan_tiled", "scan": "hello_ot_amd.kernels.generic_scan.pricing_l2sq",
                       "merge": "hello_ot_amd.kernels.generic_scan.pricing_l2sq",
                       "matrix_initial": "hierot_generic_cost_ext.raw_initial"})
