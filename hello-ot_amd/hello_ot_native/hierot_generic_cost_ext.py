"""``hierot_generic_cost_ext`` (reference ``_native/generic_scan/cost.cu:615-620``) on MI355X."""
from __future__ import annotations

import torch

from hello_ot_amd.kernels.generic_scan import ScanExtension
from hello_ot_amd.resident.cost import offsets

from ._unsupported import missing

_EXT = ScanExtension()


def raw_initial(x, y, qb, dbb, k, query_tile, database_tile, scale):
    """cost.cu:305-348 -> [values f64(q,k), indices i32(q,k)]: per query row the k largest
    (scale * <x_i, y_j> + qb_i) + dbb_j, the lowest index first among equal scores."""
    return _EXT.initialization_directional_topk_raw(x, y, qb, dbb, query_tile, database_tile, k, float(scale))


def raw_certificate_tiled(x, y, nx, ny, f, g, qt, nt, scale, denominator, fp64, caller_layout):
    """cost.cu:557-613 -> f64(5): the l2^2 certificate over all pairs without candidates. caller_layout gives the
    ScanExtension order (num, den, count, max, costmax); without it the certificate kernel's own order
    (num, den, max, costmax, count). fp64 dots are not offered (the sweep's certificate is fp32-grade)."""
    if fp64:
        raise ValueError("the MI355X certificate computes its dots from FP32 features (fp64=False)")
    st = _EXT.raw_lowrank_stats_only(x, y, nx, ny, f, g, qt, nt, float(scale))
    if not denominator:
        st = st.clone()
        st[1] = 0.0
    if caller_layout:
        return st
    return torch.stack((st[0], st[1], st[3], st[4], st[2]))


def norms(x):
    """cost.cu:173-179 -> f64(rows): squared row norms of an FP32 matrix."""
    if not (x.is_cuda and x.is_contiguous() and x.dtype == torch.float32 and x.dim() == 2):
        raise RuntimeError("Expected CUDA FP32 matrix")
    return offsets(x)


__getattr__ = missing("hierot_generic_cost_ext",
                      {"raw_certificate": "raw_certificate_tiled", "certificate": "raw_certificate_tiled",
                       "dots": "raw_initial", "dots_fp64": None, "direct_norm": None, "direct_norm_fp64": None,
                       "finish": None, "perturb_cost": None})
