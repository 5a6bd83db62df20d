"""Input generators and large-shape checkers shared by the full-shape GPU tests.

The generators reproduce the BASELINE configurations (C3, C4, C5) on the device. The checkers verify a full-size
GPU result without materialising the full score matrix on the host:

* ``exact_row_topk`` / ``exact_col_topk`` stream one side through the CPU oracle (fixed-order fp64 dots) and keep
  the exact top-k with the lowest-index tie rule, for a sample of rows or columns;
* ``fp64_certificate`` recomputes the certificate sums of all pairs with an fp64 GEMM (rocBLAS through torch) in
  chunks -- an independent computation whose per-pair error (~1e-12 relative) is far below the tolerances used.
"""
from __future__ import annotations

import numpy as np
import torch

import oracle


def gmm(rows, d, seed, dev, means_seed, chunk=32768):
    """Rows of a 64-component Gaussian mixture (means ~ N(0, 4I), identity covariance, equal weights)."""
    g = torch.Generator(device=dev)
    g.manual_seed(means_seed)
    means = 2.0 * torch.randn(64, d, generator=g, device=dev)
    g.manual_seed(seed)
    out = torch.empty(rows, d, dtype=torch.float32, device=dev)
    for s in range(0, rows, chunk):
        e = min(rows, s + chunk)
        lab = torch.randint(0, 64, (e - s,), generator=g, device=dev)
        out[s:e] = torch.randn(e - s, d, generator=g, device=dev) + means[lab]
    return out


def sqnorms(x, chunk=65536):
    out = torch.empty(x.shape[0], dtype=torch.float64, device=x.device)
    for s in range(0, x.shape[0], chunk):
        out[s:s + chunk] = (x[s:s + chunk].double() ** 2).sum(1)
    return out


def sampled_c_transform(X, Y, p, q, seed=13, sample=4096):
    """f_i = min over `sample` random resident rows j of c_ij (g = 0): duals under which a few hundred pairs per row
    are violated, as in a refinement iteration."""
    gen = torch.Generator(device=X.device)
    gen.manual_seed(seed)
    idx = torch.randperm(Y.shape[0], device=X.device, generator=gen)[:sample]
    Ys, qs = Y[idx], q[idx]
    f = torch.empty(X.shape[0], dtype=torch.float64, device=X.device)
    for s in range(0, X.shape[0], 4096):
        dots = (X[s:s + 4096].double() @ Ys.double().T)
        f[s:s + 4096] = (p[s:s + 4096, None] + qs[None, :] - 2.0 * dots).min(1).values
    return f, torch.zeros(Y.shape[0], dtype=torch.float64, device=X.device)


def _merge_topk(vals, idx, k):
    """Best k of candidate (value, index) pairs per row: value descending, then index ascending."""
    out_v = np.full((vals.shape[0], k), -np.inf)
    out_i = np.full((vals.shape[0], k), -1, np.int32)
    for r in range(vals.shape[0]):
        ok = idx[r] >= 0
        v, i = vals[r][ok], idx[r][ok]
        order = np.lexsort((i, -v))[:k]
        out_v[r, :order.size] = v[order]
        out_i[r, :order.size] = i[order]
    return out_v, out_i


def exact_row_topk(X_rows, Y, p_rows, q, qb_rows, db, k, scale=2.0, chunk=65536):
    """Exact top-k of sigma_ij = (scale*dot64(x_i, y_j) + qb_i) + db_j over all j for the given host rows, with Y
    (a device tensor) streamed to the host in chunks and scored by the CPU oracle."""
    keep_v, keep_i = [], []
    q_h, db_h = q.cpu().numpy(), db.cpu().numpy()
    for s in range(0, Y.shape[0], chunk):
        e = min(Y.shape[0], s + chunk)
        sigma, _ = oracle.l2sq_matrices(X_rows, Y[s:e].cpu().numpy(), p_rows, q_h[s:e], qb_rows, db_h[s:e], scale)
        v, i = oracle.topk(sigma, k)
        keep_v.append(v)
        keep_i.append(np.where(i >= 0, i + s, -1))
    return _merge_topk(np.concatenate(keep_v, 1), np.concatenate(keep_i, 1), k)


def exact_col_topk(X, Y_cols, p, q_cols, qb, db_cols, k, scale=2.0):
    """Exact top-k over all rows i for the given host columns (X streamed from the device once)."""
    sigma, _ = oracle.l2sq_matrices(X.cpu().numpy(), Y_cols, p.cpu().numpy(), q_cols, qb.cpu().numpy(), db_cols,
                                    scale)
    return oracle.topk(sigma, k, transpose=True)


def fp64_certificate(X, Y, p, q, qb, db, scale=2.0, chunk=65536, envelope=2.0 ** -12):
    """Certificate of all pairs from fp64 GEMMs on the device: exact sums den, max sigma+, max|c|, and for the count,
    num and den the interval the sweep's fp32-grade scores and costs must fall in, from the per-pair envelope
    E_ij = envelope * scale * sum_k |x_ik y_jk| (see ``assert_l2sq_certificate`` in test_gpu_pricing)."""
    X64, Xa = X.double(), X.abs()
    num_lo = num_hi = den = den_slack = 0.0
    count_lo = count_hi = 0
    mx = cmax = env_max = 0.0
    for s in range(0, Y.shape[0], chunk):
        e = min(Y.shape[0], s + chunk)
        dots = scale * (X64 @ Y[s:e].double().T)
        sigma = (dots + qb[:, None]) + db[None, s:e]
        cost = (p[:, None] + q[None, s:e]) - dots
        del dots
        env = (envelope * scale * 1.001) * (Xa @ Y[s:e].abs().T).double()
        num_lo += float(((sigma - env).clamp_min(0.0) ** 2).sum())
        num_hi += float(((sigma + env).clamp_min(0.0) ** 2).sum())
        count_lo += int((sigma > env).sum())
        count_hi += int((sigma > -env).sum())
        env_max = max(env_max, float(env.max()))
        den += float((cost * cost).sum())
        den_slack += float((2.0 * cost.abs() * env + env * env).sum())
        mx = max(mx, float(sigma.max().clamp_min(0.0)))
        cmax = max(cmax, float(cost.abs().max()))
        del sigma, cost, env
    return {"count": (count_lo, count_hi), "num": (num_lo, num_hi), "den": den, "den_slack": den_slack, "max": mx,
            "cmax": cmax, "envelope": env_max}


def certified_lower_bounds(a, b, f, g, row_max, col_max):
    """Lower bounds on the optimal transport cost that weak duality certifies from duals (f, g) of any quality.

    With sigma_ij = f_i + g_j - c_ij and masses summing to 1 on each side:

    * ``row``: the c-transform f^c_i = min_j (c_ij - g_j) = f_i - max_j sigma_ij makes (f^c, g) dual feasible, so
      sum a_i (f_i - row_max_i) + sum b_j g_j <= OPT;
    * ``col``: the same with the roles swapped, sum a_i f_i + sum b_j (g_j - col_max_j);
    * ``uniform``: shifting every f_i by the largest violation, sum a f + sum b g - max(max sigma, 0).

    ``row_max`` / ``col_max`` are the exact maxima of sigma over each row / column (the scans' top-1 entries)."""
    dual_value = float(a @ f + b @ g)
    row = float(a @ (f - row_max) + b @ g)
    col = float(a @ f + b @ (g - col_max))
    uniform = dual_value - max(float(row_max.max()), 0.0)
    return {"dual_value": dual_value, "row": row, "col": col, "uniform": uniform, "best": max(row, col, uniform)}


def plan_residual(sol, a, b):
    """Marginal residual of a sparse plan (host arrays): A x - (a, b)."""
    n, m = a.size, b.size
    return np.concatenate((np.bincount(sol.rows, weights=sol.values, minlength=n) - a,
                           np.bincount(sol.cols, weights=sol.values, minlength=m) - b))


def random_csr(rng, m, n, per_row):
    """CSR with `per_row` distinct uniformly random columns per row, sorted within each row (the C3 support)."""
    cols = np.empty((m, per_row), np.int64)
    todo = np.arange(m)
    while todo.size:
        draw = np.sort(rng.integers(0, n, (todo.size, per_row + 8)), axis=1)
        dup = np.zeros_like(draw, bool)
        dup[:, 1:] = draw[:, 1:] == draw[:, :-1]
        ok = (~dup).sum(1) >= per_row
        prio = rng.random(draw.shape)
        prio[dup] = np.inf
        pick = np.argsort(prio, axis=1)[:, :per_row]
        chosen = np.sort(np.take_along_axis(draw, pick, axis=1), axis=1)
        cols[todo[ok]] = chosen[ok]
        todo = todo[~ok]
    rowptr = np.arange(0, m * per_row + 1, per_row, dtype=np.int32)
    return rowptr, cols.reshape(-1).astype(np.int32)


def norm_costs_fp32(x, Y, kind):
    """fp32 l1 / linf costs of one device row block x (r x d) against Y (n x d), features combined sequentially
    (one 32-feature chunk when d <= 32) exactly as the scan ranks them: every operation is one IEEE fp32 op."""
    acc = None
    for t in range(x.shape[1]):
        z = (x[:, None, t] - Y[None, :, t]).abs()
        if acc is None:
            acc = z
        elif kind == 0:
            acc = acc + z
        else:
            acc = torch.maximum(acc, z)
    return acc
