"""Point-cloud costs on the device and the scans HELLO runs on them.

The role of ``gpu_resident/cost.py:9-161`` in the reference: one object holding the (globally shuffled)
source / target features, the l2^2 offsets p = ||x||^2, q = ||y||^2, prefix slicing per hierarchy level,
pair costs on the active support and the pricing / directional scans. Every evaluation runs in the HIP
library (``hm_pricing_l2sq``, ``hm_pricing_norm``, ``hm_pair_costs_*``); nothing falls back to PyTorch math.
"""
from __future__ import annotations

from dataclasses import dataclass, replace

import torch

from ..costs.pairs import lowrank_pair_costs, norm_pair_costs
from ..kernels.generic_scan import pricing_l2sq, pricing_norm

NORM_KINDS = {"l1": 0, "linf": 1, "l2": 2}


def offsets(features: torch.Tensor) -> torch.Tensor:
    """fp64 squared row norms, in bounded chunks (gpu_resident/cost.py:91-101)."""
    out = torch.empty(len(features), device=features.device, dtype=torch.float64)
    block = max(1, (64 << 20) // (8 * features.shape[1]))
    for start in range(0, len(features), block):
        part = features[start:start + block].double()
        out[start:start + len(part)] = (part * part).sum(-1)
    return out


@dataclass
class Cost:
    source: torch.Tensor
    target: torch.Tensor
    kind: str
    source_offset: torch.Tensor | None = None
    target_offset: torch.Tensor | None = None
    precision: str = "fp32"   # cost arithmetic of the norm costs: "fp32" or "fp64" (l2^2 is fp64-exact in both)

    @classmethod
    def create(cls, source: torch.Tensor, target: torch.Tensor, kind: str) -> "Cost":
        if kind == "l2^2":
            return cls(source, target, kind, offsets(source), offsets(target))
        if kind not in NORM_KINDS:
            raise ValueError(f"unsupported cost type {kind!r}")
        return cls(source, target, kind)

    def sliced(self, n: int, m: int, precision: str = "fp32") -> "Cost":
        """The first n source and m target points: a hierarchy level after the global shuffle, with that level's
        cost precision (gpu_resident/cost.py:31-37)."""
        return replace(self, source=self.source[:n], target=self.target[:m],
                       source_offset=None if self.source_offset is None else self.source_offset[:n],
                       target_offset=None if self.target_offset is None else self.target_offset[:m],
                       precision=precision)

    @property
    def shape(self):
        return len(self.source), len(self.target)

    def pairs(self, rows: torch.Tensor, cols: torch.Tensor) -> torch.Tensor:
        """fp64 costs of (rows[e], cols[e]): exact p + q - 2<x, y> for l2^2; for the norms the pricing scan's fp32
        cost, or at fp64 precision the fp64 norm of the reference's pair-cost kernel (costs/metric.py:94-118)."""
        if self.kind == "l2^2":
            return lowrank_pair_costs(self.source, self.target, self.source_offset, self.target_offset, rows, cols)
        return norm_pair_costs(self.source, self.target, rows, cols, NORM_KINDS[self.kind], precision=self.precision)

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
        if self.kind == "l2^2":
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


__all__ = ["Cost", "NORM_KINDS", "offsets"]
