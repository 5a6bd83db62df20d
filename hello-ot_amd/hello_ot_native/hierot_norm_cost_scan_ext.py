"""``hierot_norm_cost_scan_ext`` (reference ``_native/norm_cost_scan/norm_cost_scan_ext.cpp:1-10``) on MI355X."""
from __future__ import annotations

from hello_ot_amd.kernels.generic_scan import ScanExtension

_EXT = ScanExtension()


def fused_gcost_pairs(query, db, rows, cols, cost_type, source_index=None, target_index=None, sigma=0.0, seed=0,
                      mode=1, coefficients=None):
    """norm_cost_scan_kernel.cu:249-275 -> f64(E): l1 / linf / l2 costs of the pairs (rows[e], cols[e])."""
    return _EXT.fused_gcost_pairs(query, db, rows, cols, cost_type, source_index, target_index, sigma, seed, mode,
                                  coefficients)
