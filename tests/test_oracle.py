"""Pins of the CPU oracle (no GPU): reference known-answer tests, the reference's own CPU modules compiled
from /root/reference (oracle/_ref, when built), closed forms and brute force."""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle


def _lexsort_topk(sigma: np.ndarray, k: int):
    """Brute force: sort each row by (-sigma, index) and take k -- independent of the oracle's insertion."""
    m, n = sigma.shape
    idx = np.broadcast_to(np.arange(n), (m, n))
    order = np.lexsort((idx, -sigma), axis=1)[:, :k]
    vals = np.take_along_axis(sigma, order, axis=1)
    if k > n:
        pad = k - n
        order = np.concatenate([order, -np.ones((m, pad), np.int64)], axis=1)
        vals = np.concatenate([vals, -np.inf * np.ones((m, pad))], axis=1)
    return vals, order


# ----------------------------------------------------------------------------------------------------
# dot64
# ----------------------------------------------------------------------------------------------------

def test_dot64_integer_rows_are_exact():
    rng = np.random.default_rng(0)
    for d in (1, 7, 64, 65, 300):
        x = rng.integers(-1000, 1000, d).astype(np.float32)
        y = rng.integers(-1000, 1000, d).astype(np.float32)
        assert oracle.dot64(x, y) == float(np.dot(x.astype(np.int64), y.astype(np.int64)))


def test_dot64_lane_layout_is_pinned():
    # Case A: +2^53 in lane 0, -2^53 in lane 32 (they meet first, at stride 32), +1 in lane 1 -> 1.
    # A sequential sum would absorb the 1 into 2^53 and return 0.
    d = 128
    x = np.zeros(d, np.float32)
    y = np.zeros(d, np.float32)
    x[0], y[0] = 2.0**27, 2.0**26
    x[32], y[32] = -(2.0**27), 2.0**26
    x[1], y[1] = 1.0, 1.0
    assert oracle.dot64(x, y) == 1.0
    # Case B: the +1 moves to feature 64, i.e. lane 0's second step, and is absorbed there -> 0.
    x[1], y[1] = 0.0, 0.0
    x[64], y[64] = 1.0, 1.0
    assert oracle.dot64(x, y) == 0.0


def test_dot64_within_rounding_bound_of_exact_sum():
    rng = np.random.default_rng(1)
    for d in (3, 64, 257, 8192):
        x = rng.standard_normal(d).astype(np.float32)
        y = rng.standard_normal(d).astype(np.float32)
        prods = x.astype(np.float64) * y.astype(np.float64)
        exact = math.fsum(prods)
        bound = (d / 64 + 7) * 2.0**-53 * np.abs(prods).sum() * 1.01
        assert abs(oracle.dot64(x, y) - exact) <= bound


# ----------------------------------------------------------------------------------------------------
# l2^2 pricing semantics
# ----------------------------------------------------------------------------------------------------

def test_l2sq_directional_kat_matches_reference_test():
    # tests/torch_scan_test.py:26-59: 3 sources, 2 targets, target duals (0.2, -0.1)
    source = np.array([[0.0, 0.0], [1.0, 0.5], [2.0, -1.0]], np.float32)
    target = np.array([[0.25, 0.0], [1.5, 0.25]], np.float32)
    p = (source.astype(np.float64) ** 2).sum(1)
    q = (target.astype(np.float64) ** 2).sum(1)
    g = np.array([0.2, -0.1])
    f = np.zeros(3)
    sigma, cost = oracle.l2sq_matrices(source, target, p, q, f - p, g - q, 2.0)
    dense = ((source[:, None, :].astype(np.float64) - target[None, :, :]) ** 2).sum(2)
    np.testing.assert_allclose(cost, dense, atol=1e-12)
    vals, idx = oracle.topk(sigma, 1)
    np.testing.assert_array_equal(idx[:, 0], np.argmax(g[None, :] - dense, axis=1))
    # c-transform: min_j (c_ij - g_j) = -best sigma
    np.testing.assert_allclose(-vals[:, 0], np.min(dense - g[None, :], axis=1), atol=1e-12)


@pytest.mark.parametrize("k", [1, 3, 8])
def test_topk_matches_bruteforce_with_planted_ties(k):
    rng = np.random.default_rng(7)
    m, n, d = 40, 57, 5
    X = rng.standard_normal((m, d)).astype(np.float32)
    Y = rng.standard_normal((n, d)).astype(np.float32)
    Y[10] = Y[3]  # duplicate columns -> exact ties, lowest index must win
    Y[40] = Y[3]
    p = (X.astype(np.float64) ** 2).sum(1)
    q = (Y.astype(np.float64) ** 2).sum(1)
    f, g = rng.normal(0, 1, m), rng.normal(0, 1, n)
    g[10] = g[3]
    g[40] = g[3]
    sigma, _ = oracle.l2sq_matrices(X, Y, p, q, f - p, g - q, 2.0)
    v, i = oracle.topk(sigma, k)
    bv, bi = _lexsort_topk(sigma, k)
    np.testing.assert_array_equal(i, bi)
    np.testing.assert_array_equal(v, bv)
    cv, ci = oracle.topk(sigma, k, transpose=True)
    bcv, bci = _lexsort_topk(sigma.T.copy(), k)
    np.testing.assert_array_equal(ci, bci)
    # a row whose best is the duplicated column reports index 3, never 10 or 40
    assert not np.isin(i, [10, 40]).any() or np.isin(i, [3]).any()


def test_topk_missing_slots_are_sentinels():
    sigma = np.array([[1.0, 2.0]])
    v, i = oracle.topk(sigma, 4)
    np.testing.assert_array_equal(i[0], [1, 0, -1, -1])
    assert np.isneginf(v[0, 2:]).all()


def test_topk_negative_zero_ties_and_nan():
    sigma = np.array([[-0.0, 0.0, np.nan, -1.0]])
    v, i = oracle.topk(sigma, 3)
    np.testing.assert_array_equal(i[0], [0, 1, 3])  # -0 == +0 -> lower index first; NaN never enters


def test_stats_match_dense_certificate_formula():
    # tests/torch_scan_test.py:61-96 certificate: sqrt(sum sigma+^2) / (1 + ||C||_F), max sigma+
    rng = np.random.default_rng(3)
    X = rng.standard_normal((13, 4)).astype(np.float32)
    Y = rng.standard_normal((17, 4)).astype(np.float32)
    p = (X.astype(np.float64) ** 2).sum(1)
    q = (Y.astype(np.float64) ** 2).sum(1)
    f, g = rng.normal(2, 1, 13), rng.normal(2, 1, 17)
    sigma, cost = oracle.l2sq_matrices(X, Y, p, q, f - p, g - q, 2.0)
    st = oracle.stats(sigma, cost)
    pos = np.maximum(sigma, 0.0)
    assert st[0] == pytest.approx((pos**2).sum(), rel=1e-13)
    assert st[1] == pytest.approx((cost**2).sum(), rel=1e-13)
    assert st[2] == np.count_nonzero(sigma > 0)
    assert st[3] == pos.max()
    assert st[4] == np.abs(cost).max()


@pytest.mark.skipif(oracle.ref_scan() is None, reason="reference CPU scan not built (make -C oracle ref)")
@pytest.mark.parametrize("m,n,d,k", [(300, 257, 64, 8), (129, 500, 33, 2), (64, 64, 7, 1), (50, 40, 130, 16)])
def test_l2sq_oracle_matches_reference_cpu_epilogue(m, n, d, k):
    """Feed the reference's own _scan.dot_tile (scan.cpp:136-227) the oracle's fp64 dots."""
    sc = oracle.ref_scan()
    rng = np.random.default_rng(m * 31 + n)
    X = rng.standard_normal((m, d)).astype(np.float32)
    Y = rng.standard_normal((n, d)).astype(np.float32)
    p = (X.astype(np.float64) ** 2).sum(1)
    q = (Y.astype(np.float64) ** 2).sum(1)
    f, g = rng.normal(d, 2, m), rng.normal(d, 2, n)
    dots, _ = oracle.l2sq_matrices(X, Y, np.zeros(m), np.zeros(n), np.zeros(m), np.zeros(n), 1.0)
    rv = np.full((m, k), -np.inf)
    ri = np.full((m, k), -1, np.int64)
    cv = np.full((n, k), -np.inf)
    ci = np.full((n, k), -1, np.int64)
    ref_stats = sc.dot_tile(np.ascontiguousarray(dots), p, q, f, g, rv, ri, cv, ci, 2.0, 0, 0, 0, 4)
    orv, ori, ocv, oci, ost = oracle.l2sq_scan(X, Y, p, q, f - p, g - q, k, 2.0)
    np.testing.assert_array_equal(ri, ori)
    np.testing.assert_array_equal(ci, oci)
    np.testing.assert_allclose(rv, orv, rtol=1e-13, atol=1e-12)
    np.testing.assert_allclose(cv, ocv, rtol=1e-13, atol=1e-12)
    np.testing.assert_allclose([ref_stats[0], ref_stats[1], ref_stats[2], ref_stats[3], ref_stats[4]], ost,
                               rtol=1e-12)


# ----------------------------------------------------------------------------------------------------
# norm pricing semantics
# ----------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("kind,name", [(0, "l1"), (1, "linf"), (2, "l2")])
def test_norm_kat_matches_reference_test(kind, name):
    # tests/torch_scan_test.py:61-96 (values exactly representable in fp32)
    source = np.array([[0.0, 0.0], [1.0, 0.5], [2.0, -1.0]])
    target = np.array([[0.25, 0.0], [1.5, 0.25]])
    f = np.array([0.4, 0.1, -0.2])
    g = np.array([0.2, -0.1])
    diff = source[:, None, :] - target[None, :, :]
    dense = {"l1": np.abs(diff).sum(2), "linf": np.abs(diff).max(2), "l2": np.linalg.norm(diff, axis=2)}[name]
    sigma, cost = oracle.norm_matrices(source, target, f, g, kind)
    np.testing.assert_allclose(cost, dense, rtol=1e-7)
    score = f[:, None] + g[None, :] - dense
    st = oracle.stats(sigma, cost)
    num = np.linalg.norm(np.maximum(score, 0.0))
    den = np.linalg.norm(dense)
    assert math.sqrt(st[0]) / (1 + math.sqrt(st[1])) == pytest.approx(num / (1.0 + den), abs=1e-7)
    assert st[3] == pytest.approx(float(np.max(np.maximum(score, 0.0))), abs=1e-7)


def test_norm_chunked_fp32_accumulation_is_pinned():
    """33 features: the 33rd lands in a second 32-feature chunk; fp32 rounding differs from plain sequential."""
    x = np.zeros((1, 33), np.float32)
    y = np.zeros((1, 33), np.float32)
    x[0, 0] = 2.0**24
    x[0, 1:32] = 1.0   # 31 ones absorbed one at a time in fp32 after 2^24 -> each is lost
    x[0, 32] = 31.0
    _, c = oracle.norm_matrices(x, y, np.zeros(1), np.zeros(1), 0)
    # chunk 1: 2^24 + 1 + ... (each +1 rounds back to 2^24) = 2^24; chunk 2: 31; total 2^24 + 31 -> 2^24 + 32
    assert c[0, 0] == float(np.float32(2.0**24) + np.float32(31.0))
    assert c[0, 0] == 2.0**24 + 32


@pytest.mark.parametrize("kind,name", [(0, "l1"), (1, "linf"), (2, "l2")])
def test_norm_fp64_costs_kat_and_closed_forms(kind, name):
    """fp64 costs (compute_precision = 1): the reference KAT (tests/torch_scan_test.py:61-96), exact for l1 / linf
    (every difference and partial sum is exact there); and on random data linf exactly the numpy maximum (no rounding
    at all), l1 / l2 within 2 fp64 units per feature of the exactly rounded value (math.fsum)."""
    source = np.array([[0.0, 0.0], [1.0, 0.5], [2.0, -1.0]])
    target = np.array([[0.25, 0.0], [1.5, 0.25]])
    diff = source[:, None, :] - target[None, :, :]
    dense = {"l1": np.abs(diff).sum(2), "linf": np.abs(diff).max(2), "l2": np.linalg.norm(diff, axis=2)}[name]
    _, cost = oracle.norm_matrices(source, target, np.zeros(3), np.zeros(2), kind, precision=1)
    np.testing.assert_allclose(cost, dense, rtol=0 if kind < 2 else 1e-15, atol=0)
    rng = np.random.default_rng(70 + kind)
    X = rng.standard_normal((9, 37)).astype(np.float32)
    Y = rng.standard_normal((11, 37)).astype(np.float32)
    f, g = rng.standard_normal(9), rng.standard_normal(11)
    sigma, cost = oracle.norm_matrices(X, Y, f, g, kind, precision=1)
    z = X.astype(np.float64)[:, None, :] - Y.astype(np.float64)[None, :, :]
    if kind == 1:
        np.testing.assert_array_equal(cost, np.abs(z).max(2))
    else:
        terms = np.abs(z) if kind == 0 else z * z
        exact = np.array([[math.fsum(t) for t in row] for row in terms])
        exact = exact if kind == 0 else np.sqrt(exact)
        np.testing.assert_allclose(cost, exact, rtol=2 * 37 * 2.0**-53, atol=0)
    np.testing.assert_array_equal(sigma, (g[None, :] - cost) + f[:, None])


def test_norm_fp64_order_and_contraction_are_pinned():
    """The fp64 l1 cost is the left-to-right sum (a sequential prefix sum gives the same bits; fp32 or chunked sums
    do not), and the l2 cost accumulates fma(z, z, acc) with one rounding per feature (emulated exactly with
    rationals), which differs from a separate multiply and add on these inputs."""
    from fractions import Fraction

    rng = np.random.default_rng(11)
    X = rng.standard_normal((6, 45)).astype(np.float32)
    Y = rng.standard_normal((7, 45)).astype(np.float32)
    _, c1 = oracle.norm_matrices(X, Y, np.zeros(6), np.zeros(7), 0, precision=1)
    z = X.astype(np.float64)[:, None, :] - Y.astype(np.float64)[None, :, :]
    np.testing.assert_array_equal(c1, np.cumsum(np.abs(z), axis=2)[:, :, -1])
    # fp64 sums of fp32 differences are mostly exact; a huge first feature makes the order visible: left to right
    # every later 16 is absorbed by 2^60 (half its ulp is 128), while summing the 44 sixteens first keeps 704
    x = np.zeros((1, 45), np.float32)
    x[0, 0], x[0, 1:] = 2.0**60, 16.0
    _, c = oracle.norm_matrices(x, np.zeros((1, 45), np.float32), np.zeros(1), np.zeros(1), 0, precision=1)
    assert c[0, 0] == 2.0**60 != 2.0**60 + 768.0 == float(np.float64(2.0**60) + np.float64(704.0))
    _, c2 = oracle.norm_matrices(X, Y, np.zeros(6), np.zeros(7), 2, precision=1)
    fused = np.empty((6, 7))
    plain = np.empty((6, 7))
    for i in range(6):
        for j in range(7):
            acc = sep = 0.0
            for t in z[i, j]:
                acc = float(Fraction(acc) + Fraction(float(t)) * Fraction(float(t)))
                sep = sep + float(t) * float(t)
            fused[i, j], plain[i, j] = math.sqrt(acc), math.sqrt(sep)
    np.testing.assert_array_equal(c2, fused)
    assert (fused != plain).any()


# ----------------------------------------------------------------------------------------------------
# SDDMM and pair costs
# ----------------------------------------------------------------------------------------------------

def test_sddmm_closed_form_and_exact_integers():
    rng = np.random.default_rng(5)
    m, n, d = 50, 70, 96
    X = rng.standard_normal((m, d)).astype(np.float32)
    Y = rng.standard_normal((n, d)).astype(np.float32)
    p = (X.astype(np.float64) ** 2).sum(1)
    q = (Y.astype(np.float64) ** 2).sum(1)
    cols = [np.sort(rng.choice(n, 5, replace=False)) for _ in range(m)]
    rowptr = np.concatenate([[0], np.cumsum([len(c) for c in cols])]).astype(np.int32)
    col = np.concatenate(cols).astype(np.int32)
    out = oracle.sddmm_l2sq(X, Y, p, q, rowptr, col, 2.0)
    rows = np.repeat(np.arange(m), 5)
    dense = ((X[rows].astype(np.float64) - Y[col].astype(np.float64)) ** 2).sum(1)
    np.testing.assert_allclose(out, dense, rtol=1e-12, atol=1e-10)
    Xi = rng.integers(-50, 50, (m, d)).astype(np.float32)
    Yi = rng.integers(-50, 50, (n, d)).astype(np.float32)
    pi = (Xi.astype(np.float64) ** 2).sum(1)
    qi = (Yi.astype(np.float64) ** 2).sum(1)
    outi = oracle.sddmm_l2sq(Xi, Yi, pi, qi, rowptr, col, 2.0)
    exact = ((Xi[rows].astype(np.int64) - Yi[col].astype(np.int64)) ** 2).sum(1)
    np.testing.assert_array_equal(outi, exact.astype(np.float64))


@pytest.mark.parametrize("kind", [0, 1, 2])
def test_pair_costs_norm_match_numpy(kind):
    rng = np.random.default_rng(9)
    X = rng.random((30, 8)).astype(np.float32)
    Y = rng.random((40, 8)).astype(np.float32)
    rows = rng.integers(0, 30, 200)
    cols = rng.integers(0, 40, 200)
    out = oracle.pair_costs_norm(X, Y, rows, cols, kind)
    diff = X[rows].astype(np.float64) - Y[cols].astype(np.float64)
    ref = [np.abs(diff).sum(1), np.abs(diff).max(1), np.sqrt((diff**2).sum(1))][kind]
    np.testing.assert_allclose(out, ref, rtol=1e-14, atol=0)


# ----------------------------------------------------------------------------------------------------
# PDHG
# ----------------------------------------------------------------------------------------------------

def _small_problem():
    # tests/torch_restricted_ot_pdlp_test.py:16-23
    return dict(rows=np.array([0, 0, 1, 1]), cols=np.array([0, 1, 0, 1]),
                costs=np.array([0.0, 2.0, 1.0, 0.0]), source_mass=np.array([0.4, 0.6]),
                target_mass=np.array([0.5, 0.5]))


@pytest.mark.parametrize("warm", [False, True])
def test_pdhg_kat_small_problem(warm):
    # tests/torch_restricted_ot_pdlp_test.py:58-80: optimum 0.1 at x = (0.4, 0, 0.1, 0.5)
    kw = {}
    if warm:
        kw = dict(warm_start_primal=np.array([0.35, 0.05, 0.15, 0.45]), warm_start_dual=np.zeros(4))
    r = oracle.pdhg_solve(**_small_problem(), evaluation_frequency=20, iteration_limit=200_000, tolerance=1e-7, **kw)
    assert r["success"], r
    assert r["obj_val"] == pytest.approx(0.1, abs=2e-6)
    assert r["primal_feas"] < 1e-7 and r["dual_feas"] < 1e-7 and r["gap"] < 1e-7
    np.testing.assert_allclose(r["x"], [0.4, 0.0, 0.1, 0.5], atol=1e-5)


def test_pdhg_matches_linear_programming_optimum():
    scipy_opt = pytest.importorskip("scipy.optimize")
    rng = np.random.default_rng(3)
    ns, nt = 4, 5
    costs = rng.random((ns, nt))
    rows, cols = np.indices(costs.shape)
    a, b = np.full(ns, 1 / ns), np.full(nt, 1 / nt)
    r = oracle.pdhg_solve(rows.ravel(), cols.ravel(), costs.ravel(), a, b, tolerance=1e-8)
    A = np.zeros((ns + nt, ns * nt))
    for e, (i, j) in enumerate(zip(rows.ravel(), cols.ravel())):
        A[i, e] = 1
        A[ns + j, e] = 1
    lp = scipy_opt.linprog(costs.ravel(), A_eq=A, b_eq=np.concatenate([a, b]), bounds=(0, None), method="highs")
    assert r["success"]
    assert r["obj_val"] == pytest.approx(lp.fun, abs=2e-7)


@pytest.mark.skipif(oracle.ref_lp() is None, reason="reference CPU PDHG not built (make -C oracle ref)")
@pytest.mark.parametrize("freq,limit,tol", [(5, 40, 0.0), (20, 5000, 1e-7), (200, 100000, 1e-8)])
def test_pdhg_oracle_bit_identical_to_reference_solver(freq, limit, tol):
    """solver.cpp (reference, one thread) and the restatement produce the same bits."""
    lp = oracle.ref_lp()
    rng = np.random.default_rng(12)
    rows, cols = np.indices((7, 5))
    rows, cols = rows.ravel().astype(np.int64), cols.ravel().astype(np.int64)
    costs = rng.random(35)
    sm, tm = np.full(7, 1 / 7), np.full(5, 1 / 5)
    ref = lp.solve_once(rows, cols, costs, np.concatenate([sm, tm]), np.zeros(35), np.zeros(12), 7, 1, freq, 3600.0,
                        limit, tol, tol, tol, False, False)
    mine = oracle.pdhg_solve(rows, cols, costs, sm, tm, evaluation_frequency=freq, iteration_limit=limit,
                             tolerance=tol)
    assert ref["iterations"] == mine["iterations"]
    assert ref["termination_reason"] == mine["termination_reason"]
    assert ref["solver_diag"]["restart_count"] == mine["restart_count"]
    np.testing.assert_array_equal(ref["x"], mine["x"])
    np.testing.assert_array_equal(ref["y"], mine["y"])


@pytest.mark.skipif(oracle.ref_lp() is None, reason="reference CPU PDHG not built (make -C oracle ref)")
def test_pdhg_oracle_bit_identical_on_sparse_support_with_warm_start():
    lp = oracle.ref_lp()
    rng = np.random.default_rng(4)
    ns, nt = 30, 25
    rows = np.concatenate([np.arange(ns), rng.integers(0, ns, 120)]).astype(np.int64)
    cols = np.concatenate([rng.integers(0, nt, ns), rng.integers(0, nt, 120)]).astype(np.int64)
    rows = np.concatenate([rows, rng.integers(0, ns, nt)])
    cols = np.concatenate([cols, np.arange(nt)])
    costs = rng.random(rows.size)
    a = rng.random(ns)
    a /= a.sum()
    b = rng.random(nt)
    b /= b.sum()
    x0 = rng.random(rows.size) * 0.01
    y0 = rng.normal(0, 0.1, ns + nt)
    ref = lp.solve_once(rows, cols, costs, np.concatenate([a, b]), x0, y0, ns, 1, 50, 3600.0, 3000, 1e-9, 1e-9,
                        1e-9, False, False)
    mine = oracle.pdhg_solve(rows, cols, costs, a, b, warm_start_primal=x0, warm_start_dual=y0,
                             evaluation_frequency=50, iteration_limit=3000, tolerance=1e-9)
    np.testing.assert_array_equal(ref["x"], mine["x"])
    np.testing.assert_array_equal(ref["y"], mine["y"])
    assert ref["iterations"] == mine["iterations"]
