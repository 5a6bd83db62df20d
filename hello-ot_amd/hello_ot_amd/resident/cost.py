"""Point-cloud costs on the device and the scans HELLO runs on them.

The role of ``gpu_resident/cost.py:9-161`` in the reference: one object holding the (globally shuffled)
source / target features, the l2^2 offsets p = ||x||^2, q = ||y||^2, prefix slicing per hierarchy level,
pair costs on the active support and the pricing / directional scans. Every evaluation runs in the HIP
library (``hm_pricing_l2sq``, ``hm_pricing_norm``, ``hm_pair_costs_*``); nothing falls back to PyTorch math.

The source side may be streamed (``HostRows``: pinned host memory, read in row chunks), as in the reference's
resident / streamed scan (``kernels/bilinear_topk.py:255-368``): the target side stays on the device, each source
chunk is priced against it (l2^2: against its sweep copy, prepared once per scan), row lists are written per chunk,
column lists are merged across chunks in exact fp64 with the lowest row index first among equal values, and the
certificate sums add up (its maxima take the maximum). Pair costs are evaluated chunk by chunk over the pairs sorted
by source row. The results are the same as with both sides on the device.
"""
from __future__ import annotations

from dataclasses import dataclass, replace

import torch

from ..costs.pairs import lowrank_pair_costs, norm_pair_costs
from .. import _lib
from ..kernels.generic_scan import ResidentSide, _precision_flags, pricing_l2sq, pricing_norm
from . import host as _host
from .host import HostRows

NORM_KINDS = {"l1": 0, "linf": 1, "l2": 2}


def _sq_rows(part: torch.Tensor) -> torch.Tensor:
    part = part.double()
    return (part * part).sum(-1)


def offsets(features) -> torch.Tensor:
    """fp64 squared row norms, in bounded chunks (gpu_resident/cost.py:91-101); a streamed side is read once."""
    if isinstance(features, HostRows):
        out = torch.empty(len(features), device=features.device, dtype=torch.float64)
        block = max(1, (64 << 20) // (8 * features.d))
        for s, e, x in features.chunks():
            for b in range(0, e - s, block):
                part = x[b:b + block]
                out[s + b:s + b + len(part)] = _sq_rows(part)
        return out
    out = torch.empty(len(features), device=features.device, dtype=torch.float64)
    block = max(1, (64 << 20) // (8 * features.shape[1]))
    for start in range(0, len(features), block):
        out[start:start + block] = _sq_rows(features[start:start + block])
    return out


# device bytes a streamed l2^2 scan's library call may take for its workspace: a call with both directions keeps
# column lists per 256-row panel of its chunk for every column (6.6 GiB for 19968 x 1.28M), so such scans read the
# streamed side in smaller chunks (8192 rows for the C5 certificate, 2.9 GiB)
STREAMED_WORKSPACE_BYTES = 3 << 30


def fused_chunk_rows(chunk: int, n: int, d: int, k: int, certificate: bool, precision: str) -> int:
    """Source rows per call of a streamed scan with both directions: ``chunk``, or when its workspace against n
    resident columns exceeds STREAMED_WORKSPACE_BYTES the largest multiple of 2048 rows whose workspace fits (at
    least 2048). 2048 rows are 8 of the sweep's 256-row panels: with a multiple of 8 panels (up to 64) its
    panel-major workgroup order keeps each panel on one XCD (25 panels run 7% slower than 24)."""
    lib = _lib.load()
    flags = _lib.HM_ROWS | _lib.HM_COLS | (_lib.HM_STATS | _lib.HM_LINF if certificate else 0) \
        | _precision_flags(precision)
    step = 2048

    def fits(rows):
        return lib.hm_pricing_l2sq_resident_workspace_bytes(rows, n, d, k, flags) <= STREAMED_WORKSPACE_BYTES

    if chunk <= step or fits(chunk):
        return chunk
    lo, hi = 1, chunk // step             # step * lo rows are taken when nothing larger fits
    while lo < hi:
        mid = (lo + hi + 1) // 2
        if fits(step * mid):
            lo = mid
        else:
            hi = mid - 1
    return step * lo


def merge_columns(best, new, k: int):
    """Best k per column of two exact lists, each sorted (values descending, equal values by row index) and ``best``
    holding only lower row indices than ``new``: the merged order puts ``best``'s entry first among equal values,
    which is the lowest row index. Each entry's merged rank is its own position plus the entries of the other list
    ahead of it (strictly greater values from ``new``, greater or equal ones from ``best``), found by binary search
    in the other row; every entry is scattered to its rank, those of rank k or more into one spare column that is
    dropped (no data-dependent sizes, so nothing waits for the device)."""
    if best is None:
        return new
    av, ai = best
    bv, bi = new
    pos = torch.arange(av.shape[1], device=av.device).expand_as(av)
    na, nb = (-av).contiguous(), (-bv).contiguous()          # ascending rows for the binary searches
    rank_a = pos + torch.searchsorted(nb, na, right=False)   # entries of `new` strictly greater
    rank_b = pos[:, : bv.shape[1]] + torch.searchsorted(na, nb, right=True)   # entries of `best` greater or equal
    out_v = torch.empty((av.shape[0], k + 1), dtype=av.dtype, device=av.device)
    out_i = torch.empty((av.shape[0], k + 1), dtype=ai.dtype, device=av.device)
    for rank, v, i in ((rank_a, av, ai), (rank_b, bv, bi)):
        r = rank.clamp(max=k)
        out_v.scatter_(1, r, v)
        out_i.scatter_(1, r, i)
    return out_v[:, :k].contiguous(), out_i[:, :k].contiguous()


@dataclass
class Cost:
    source: object                 # device fp32 tensor, or HostRows (streamed)
    target: torch.Tensor
    kind: str
    source_offset: torch.Tensor | None = None
    target_offset: torch.Tensor | None = None
    precision: str = "fp32"   # cost arithmetic of the norm costs: "fp32" or "fp64" (l2^2 is fp64-exact in both)

    @classmethod
    def create(cls, source, target: torch.Tensor, kind: str) -> "Cost":
        if kind == "l2^2":
            return cls(source, target, kind, offsets(source), offsets(target))
        if kind not in NORM_KINDS:
            raise ValueError(f"unsupported cost type {kind!r}")
        return cls(source, target, kind)

    def sliced(self, n: int, m: int, precision: str = "fp32") -> "Cost":
        """The first n source and m target points: a hierarchy level after the global shuffle, with that level's
        cost precision (gpu_resident/cost.py:31-37). A streamed source prefix small enough is copied to the device."""
        source = self.source[:n] if torch.is_tensor(self.source) else self.source.prefix(n)
        if isinstance(source, HostRows) and source.nbytes() <= _host.STREAM_MIN_BYTES:
            source = source.to_device()
        return replace(self, source=source, target=self.target[:m],
                       source_offset=None if self.source_offset is None else self.source_offset[:n],
                       target_offset=None if self.target_offset is None else self.target_offset[:m],
                       precision=precision)

    @property
    def shape(self):
        return len(self.source), len(self.target)

    @property
    def streamed(self) -> bool:
        return isinstance(self.source, HostRows)

    def _pairs_with(self, x, p, rows, cols):
        if self.kind == "l2^2":
            return lowrank_pair_costs(x, self.target, p, self.target_offset, rows, cols)
        return norm_pair_costs(x, self.target, rows, cols, NORM_KINDS[self.kind], precision=self.precision)

    def pairs(self, rows: torch.Tensor, cols: torch.Tensor) -> torch.Tensor:
        """fp64 costs of (rows[e], cols[e]): exact p + q - 2<x, y> for l2^2; for the norms the pricing scan's fp32
        cost, or at fp64 precision the fp64 norm of the reference's pair-cost kernel (costs/metric.py:94-118)."""
        if not self.streamed:
            return self._pairs_with(self.source, self.source_offset, rows, cols)
        rows, cols = rows.reshape(-1).long(), cols.reshape(-1).long()
        out = torch.empty(rows.numel(), dtype=torch.float64, device=self.target.device)
        if rows.numel() == 0:
            return out
        order = torch.argsort(rows, stable=True)
        rs, cs = rows[order], cols[order]
        starts = torch.arange(0, len(self.source), self.source.chunk, device=rows.device)
        edges = torch.searchsorted(rs, torch.cat((starts, starts.new_tensor([len(self.source)])))).tolist()
        for index, (s, e, x) in enumerate(self.source.chunks()):
            a, b = edges[index], edges[index + 1]
            if a == b:
                continue
            p = None if self.source_offset is None else self.source_offset[s:e]
            out[order[a:b]] = self._pairs_with(x, p, rs[a:b] - s, cs[a:b])
        return out

    def scan(self, dual: torch.Tensor, k: int, *, certificate: bool = False, direction: str | None = None):
        """Pricing / directional scans in the reference's output convention (gpu_resident/cost.py:104-161):

        * ``direction=None``: (row values - f, row idx, column values - g, column idx, metrics), values being the
          k best sigma_ij = f_i + g_j - c_ij per row / column; ``metrics`` (with ``certificate``) holds the
          relative l2 / linf dual feasibility, the max violation and the violation count;
        * ``direction="source"``: per source row the k best g_j - c_ij; ``"target"``: per target column the k
          best f_i - c_ij.
        """
        if direction not in (None, "source", "target") or (certificate and direction is not None):
            raise ValueError("direction must be source/target or None; certificates require both directions")
        n, m = self.shape
        f, g = dual[:n].contiguous(), dual[n:].contiguous()
        kr, kc = min(k, m), min(k, n)
        if direction == "source":
            f = torch.zeros_like(f)
        elif direction == "target":
            g = torch.zeros_like(g)
        rows = direction in (None, "source")
        cols = direction in (None, "target")
        if self.streamed:
            rv, ri, cv, ci, st = self._scan_streamed(f, g, k, rows, cols, certificate)
        elif self.kind == "l2^2":
            p, q = self.source_offset, self.target_offset
            rv, ri, cv, ci, st = pricing_l2sq(self.source, self.target, p, q, f - p, g - q, k, rows=rows, cols=cols,
                                              stats=certificate, linf=certificate)
        else:
            rv, ri, cv, ci, st = pricing_norm(self.source, self.target, f, g, k, NORM_KINDS[self.kind], rows=rows,
                                              cols=cols, stats=certificate, linf=certificate,
                                              precision=self.precision)
        if direction == "source":
            return rv[:, :kr], ri[:, :kr], None, None, None
        if direction == "target":
            return None, None, cv[:, :kc], ci[:, :kc], None
        metrics = None
        if certificate:
            num, den, count, mx, cmax = (float(v) for v in st.cpu())
            metrics = {"l2": num ** 0.5 / (1.0 + den ** 0.5), "linf": mx / (1.0 + cmax), "max": mx,
                       "count": int(round(count))}
        return rv[:, :kr] - f[:, None], ri[:, :kr], cv[:, :kc] - g[:, None], ci[:, :kc], metrics

    def _scan_streamed(self, f, g, k, rows, cols, certificate):
        """The scan with the source side streamed in chunks against the device-resident target side."""
        n, m = self.shape
        dev = self.target.device
        rv = torch.empty((n, k), dtype=torch.float64, device=dev) if rows else None
        ri = torch.empty((n, k), dtype=torch.int32, device=dev) if rows else None
        st = torch.zeros(5, dtype=torch.float64, device=dev) if certificate else None
        best = None
        l2sq = self.kind == "l2^2"
        side = ResidentSide(self.target) if l2sq else None   # the target's sweep copy, for this scan only
        chunk = None
        if l2sq:
            p, q = self.source_offset, self.target_offset
            db = g - q
            if cols and (rows or certificate):
                chunk = fused_chunk_rows(self.source.chunk, m, self.source.d, k, certificate, side.precision)
        for s, e, x in self.source.chunks(rows=chunk):
            if l2sq:
                # a columns-only scan runs the library's role-swapped pass per chunk (the target rows against the
                # chunk, reading the resident side's copy): as fast here as column lists fused into a row sweep,
                # and without the fused lists' partial-list buffer (up to 12 GiB). The k-th score of each running
                # column list is the chunk's floor: columns the chunk cannot change skip their exact re-evaluation.
                floor = best[0][:, k - 1].contiguous() if (cols and best is not None) else None
                out = pricing_l2sq(x, self.target, p[s:e], q, f[s:e] - p[s:e], db, k, rows=rows, cols=cols,
                                   stats=certificate, linf=certificate, resident=side, col_floor=floor)
            else:
                out = pricing_norm(x, self.target, f[s:e], g, k, NORM_KINDS[self.kind], rows=rows, cols=cols,
                                   stats=certificate, linf=certificate, precision=self.precision)
            if rows:
                rv[s:e], ri[s:e] = out[0], out[1]
            if cols:
                shifted = torch.where(out[3] >= 0, out[3] + s, out[3])
                best = merge_columns(best, (out[2], shifted), k)
            if certificate:
                st[:3] += out[4][:3]
                st[3:] = torch.maximum(st[3:], out[4][3:])
        cv, ci = best if cols else (None, None)
        return rv, ri, cv, ci, st


__all__ = ["Cost", "NORM_KINDS", "merge_columns", "offsets"]
