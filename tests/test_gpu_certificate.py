"""The l2^2 certificate of each sweep precision held to the error bound that sweep claims (GPU only).

The certificate (num = sum sigma+^2, den = sum c^2, count of sigma > 0, max sigma+, max |c|) is computed from the
sweep's own dot t of each pair, with an fp64 epilogue for the pairs whose fp32 score lies within the rounding slack
of zero: the reference's arithmetic (fp32 SGEMM dot, fp64 score; cost.cu:481-613, pricing_small.cu:241-257) on a
different dot. Against the exact fp64 scores sigma (an fp64 GEMM here), each pair's decision is therefore off by at
most E_ij = scale * b_ij + slack_i, where b_ij bounds |t - x.y| for the sweep at hand:

* fp32 MFMA: gamma(d + 2) sum_k |x_k y_k|, gamma(n) = n u' / (1 - n u') with u' = 2^-23 (twice the unit roundoff,
  which also covers truncating accumulation);
* split-bf16 (three bf16 products per feature, fp32 accumulation): (3 2^-16 (1 + 2^-7) + 3 2^-24
  + gamma(3.375 d + d / 128 + 2)) sum_k |x_k y_k|;
* int8 split (16-bit fixed point per 32-row block, scale s <= max|x| / 32639 over the side; two int8 limbs, the
  low-limb product dropped, exact int32 sums, one fp32 conversion): alpha_x beta_y + alpha_y beta_x + gamma_x
  gamma_y + 5 u rho_x rho_y + 2 u ||x|| ||y||, with alpha = 0.51 s, beta = ||x||_1 + 0.51 s d, gamma = 128 s sqrt(d)
  and rho = ||x||_2 + 257 s sqrt(d);

and slack_i = CERT_REL (wmax_i + |qb_i| + max|db|) (1 + 1e-3), wmax_i = 1.01 scale ||x_i|| max||y|| + max|db|,
CERT_REL = 2.5 fp32 units (the four fp32 roundings of the score). The sums accumulate in fp32 within a tile
(at most 256 terms) before fp64: a relative 1e-4 more. Hence

    count in [#{sigma > E}, #{sigma > -E}],  num in [sum (sigma - E)+^2, sum (sigma + E)+^2] (1 -+ 1e-4),
    den within sum (2|c| e + e^2) + 1e-4 den of the exact sum, e = E + 3u (|p| + |g| + |w|) + u |c|.

A dropped or mis-signed term, or a certificate taken from a coarser dot than the sweep claims, leaves the interval.
Two dual states per shape: a refinement-like one (hundreds of violated pairs per row, from a sampled c-transform) and
a near-converged one (exact c-transforms, then violations of 1e-7 of the cost scale), where every row has pairs at
zero and the count is decided by the dot's error.

The same cases also measure each sweep's certificate error next to the reference's own arithmetic (an fp32 GEMM of
the vendor library, fp64 epilogue), both against the exact sums, and print them.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from _shapes import gmm
from hello_ot_amd.kernels.generic_scan import pricing_l2sq

pytestmark = pytest.mark.gpu

U = 2.0 ** -24
CERT_REL = 1.4901161e-07
SCALE = 2.0


def _gamma(n):
    u2 = 2.0 * U
    return n * u2 / (1.0 - n * u2)


def _case(dev, m, n, d, state, seed):
    X = gmm(m, d, seed=seed, dev=dev, means_seed=seed + 100)
    Y = gmm(n, d, seed=seed + 1, dev=dev, means_seed=seed + 101)
    X64, Y64 = X.double(), Y.double()
    p, q = (X64 * X64).sum(1), (Y64 * Y64).sum(1)
    dots = X64 @ Y64.T
    cost = (p[:, None] + q[None, :]) - SCALE * dots
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    if state == "refine":
        sample = torch.randperm(n, generator=gen, device=dev)[: max(8, n // 64)]
        f = cost[:, sample].min(1).values
        g = torch.zeros(n, dtype=torch.float64, device=dev)
    else:
        f = cost.min(1).values
        g = (cost - f[:, None]).min(0).values
        scale = float(cost.abs().max())
        f = f + 1e-7 * scale * torch.rand(m, generator=gen, device=dev, dtype=torch.float64)
    return X, Y, p, q, f, g, dots, cost


def _bounds(X, Y, p, q, f, g, dots, cost, precision):
    """Per-pair decision error E of the sweep `precision`, and the certificate intervals it implies."""
    d = X.shape[1]
    Xa, Ya = X.double().abs(), Y.double().abs()
    xn, yn = X.double().norm(dim=1), Y.double().norm(dim=1)
    if precision == "fp32":
        b = _gamma(d + 2) * (Xa @ Ya.T)
    elif precision == "bf16x3":
        rel = 3 * 2.0 ** -16 * (1 + 2.0 ** -7) + 3 * 2.0 ** -24 + _gamma(3.375 * d + d / 128 + 2)
        b = rel * (Xa @ Ya.T)
    else:
        def terms(A, norm):
            s = float(A.abs().max()) / 32639.0
            alpha = 0.51 * s
            beta = A.double().abs().sum(1) + 0.51 * s * d
            gam = 128.0 * s * math.sqrt(d)
            rho = norm + 257.0 * s * math.sqrt(d)
            return alpha, beta, gam, rho
        ax, bx, gx, rx = terms(X, xn)
        ay, by, gy, ry = terms(Y, yn)
        b = (ax * by[None, :] + ay * bx[:, None] + gx * gy + 5 * U * rx[:, None] * ry[None, :]
             + 2 * U * xn[:, None] * yn[None, :])
    qb, db = f - p, g - q
    dmax = float(db.abs().max())
    wmax = 1.01 * SCALE * xn * float(yn.max()) + dmax
    slack = CERT_REL * (wmax + qb.abs() + dmax) * (1 + 1e-3)
    E = SCALE * b + slack[:, None]
    sigma = (SCALE * dots + qb[:, None]) + db[None, :]
    w = SCALE * dots + db[None, :]
    e = E + 3 * U * (p[:, None].abs() + g[None, :].abs() + w.abs()) + U * cost.abs()
    den = float((cost * cost).sum())
    return {
        "count": (int((sigma > E).sum()), int((sigma > -E).sum())),
        "num": (float(((sigma - E).clamp_min(0) ** 2).sum()) * (1 - 1e-4),
                float(((sigma + E).clamp_min(0) ** 2).sum()) * (1 + 1e-4)),
        "den": den, "den_slack": float((2 * cost.abs() * e + e * e).sum()) + 1e-4 * den,
        "max": max(float(sigma.max()), 0.0), "cmax": float(cost.abs().max()), "cmax_slack": float(e.max()),
        "exact": (float((sigma.clamp_min(0) ** 2).sum()), int((sigma > 0).sum())),
        "E_max": float(E.max()),
    }


def _reference_arithmetic(X, Y, p, q, f, g):
    """num and count from the vendor library's fp32 GEMM with an fp64 epilogue (the reference's arithmetic)."""
    dots32 = (X @ Y.T).double()
    sigma = (SCALE * dots32 + (f - p)[:, None]) + (g - q)[None, :]
    return float((sigma.clamp_min(0) ** 2).sum()), int((sigma > 0).sum())


@pytest.mark.parametrize("state", ["refine", "converged"])
@pytest.mark.parametrize("d", [64, 256, 1024, 8192])
def test_l2sq_certificate_within_each_sweeps_bound(cuda, capsys, d, state):
    torch.backends.cuda.matmul.allow_tf32 = False
    m, n = 1024, 2048
    X, Y, p, q, f, g, dots, cost = _case(cuda, m, n, d, state, seed=d + (0 if state == "refine" else 7))
    ref_num, ref_count = _reference_arithmetic(X, Y, p, q, f, g)
    lines = []
    for precision in ("fp32", "bf16x3", "int8x3"):
        bounds = _bounds(X, Y, p, q, f, g, dots, cost, precision)
        _, _, _, _, st = pricing_l2sq(X, Y, p, q, f - p, g - q, 2, linf=True, precision=precision)
        num, den, count, mx, cmax = (float(v) for v in st.cpu())
        exact_num, exact_count = bounds["exact"]
        lines.append(f"d={d:5d} {state:9s} {precision:6s}: num rel err {abs(num - exact_num) / exact_num:.2e} "
                     f"(fp32 GEMM {abs(ref_num - exact_num) / exact_num:.2e}), count {int(count)} vs exact "
                     f"{exact_count} (fp32 GEMM {ref_count}), den rel err {abs(den - bounds['den']) / bounds['den']:.1e}, "
                     f"E max {bounds['E_max']:.2e}")
        lo, hi = bounds["count"]
        assert lo <= count <= hi, (precision, count, bounds["count"])
        lo, hi = bounds["num"]
        assert lo <= num <= hi, (precision, num, bounds["num"])
        assert abs(den - bounds["den"]) <= bounds["den_slack"], (precision, den, bounds["den"])
        assert mx == pytest.approx(bounds["max"], rel=1e-12, abs=1e-12 * bounds["cmax"])
        assert abs(cmax - bounds["cmax"]) <= bounds["cmax_slack"]
    with capsys.disabled():
        print("\n[certificate] " + "\n[certificate] ".join(lines), flush=True)
