"""Parity of the MI355X pricing scans with the CPU oracle (GPU only)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from hello_ot_amd import _lib
from hello_ot_amd.kernels.generic_scan import ResidentSide, ScanExtension, pricing_l2sq, pricing_norm

pytestmark = pytest.mark.gpu


def _l2sq_case(m, n, d, seed, *, dual_mean=None, dup=False, integer=False):
    rng = np.random.default_rng(seed)
    if integer:
        X = rng.integers(-3, 4, (m, d)).astype(np.float32)
        Y = rng.integers(-3, 4, (n, d)).astype(np.float32)
    else:
        X = rng.standard_normal((m, d)).astype(np.float32)
        Y = rng.standard_normal((n, d)).astype(np.float32)
    if dup and n > 8:
        Y[n // 2] = Y[1]
        Y[n - 1] = Y[1]
    p = (X.astype(np.float64) ** 2).sum(1)
    q = (Y.astype(np.float64) ** 2).sum(1)
    mean = float(d) if dual_mean is None else dual_mean
    f = rng.normal(mean, 2.0, m)
    g = rng.normal(mean, 2.0, n)
    if dup and n > 8:
        g[n // 2] = g[1]
        g[n - 1] = g[1]
    if integer:
        f = np.round(f)
        g = np.round(g)
    return X, Y, p, q, f - p, g - q


def _to(dev, *arrays):
    return [torch.as_tensor(a).to(dev) for a in arrays]


# The l2^2 certificate is computed from the sweep's fp32 dots with an fp64 epilogue for every pair near zero (the
# reference's arithmetic: fp32 SGEMM dots, fp64 scores). Against the oracle's exact fp64 scores it is therefore
# pinned by intervals: with E_ij = 2^-12 * scale * sum_k |x_ik y_jk| (above the error of every sweep's dot for the
# data tested: fp32 and split-bf16 rounding, the int8 split's quantization), count lies in
# [#{sigma > E}, #{sigma > -E}], num in [sum max(sigma - E, 0)^2, sum max(sigma + E, 0)^2] and den within
# sum (2|c| E + E^2) (plus fp32 rounding, rtol 1e-5) of the exact sum; a dropped or mis-signed term moves them far
# outside. max|c| is within max E and fp32 rounding; the maximum violation is the exact fp64 maximum.
DOT_ENVELOPE = 2.0 ** -12


def l2sq_certificate_bounds(X, Y, p, q, qb, db, scale=2.0):
    sigma, cost = oracle.l2sq_matrices(X, Y, p, q, qb, db, scale)
    E = DOT_ENVELOPE * scale * (np.abs(X).astype(np.float64) @ np.abs(Y).astype(np.float64).T)
    return {
        "count": (np.count_nonzero(sigma > E), np.count_nonzero(sigma > -E)),
        "num": (float((np.maximum(sigma - E, 0.0) ** 2).sum()), float((np.maximum(sigma + E, 0.0) ** 2).sum())),
        "den": float((cost * cost).sum()), "den_slack": float((2.0 * np.abs(cost) * E + E * E).sum()),
        "max": float(max(sigma.max(), 0.0)), "cmax": float(np.abs(cost).max()), "envelope": float(E.max()),
    }


def assert_l2sq_certificate(st, bounds, linf=True):
    got = st.cpu().numpy()
    lo, hi = bounds["num"]
    assert lo * (1 - 1e-9) <= got[0] <= hi * (1 + 1e-9), (got[0], bounds["num"])
    assert abs(got[1] - bounds["den"]) <= bounds["den_slack"] + 1e-5 * bounds["den"], (got[1], bounds["den"])
    lo, hi = bounds["count"]
    assert lo <= got[2] <= hi, (got[2], bounds["count"])
    assert got[3] == bounds["max"]
    if linf:
        # max|c| comes from the sweep's fp32 costs: within the dot envelope and fp32 rounding of the exact maximum
        assert abs(got[4] - bounds["cmax"]) <= bounds["envelope"] + 1e-6 * bounds["cmax"], (got[4], bounds["cmax"])


def _assert_stats(gpu, ref, rtol=1e-12):
    """Norm certificates: every cost and score is exact, so count and the maximum are exact; the sums accumulate
    fp32 squares per tile (scores near zero in fp64), so they agree to fp32 rounding (rtol 1e-6)."""
    gpu = gpu.cpu().numpy()
    np.testing.assert_allclose(gpu[0], ref[0], rtol=1e-6)
    np.testing.assert_allclose(gpu[1], ref[1], rtol=1e-6)
    assert gpu[2] == ref[2]
    assert gpu[3] == ref[3]


@pytest.mark.parametrize("m,n,d,k,scale", [
    (257, 300, 64, 8, 2.0),     # ragged rows/cols, C2 dimension
    (130, 129, 3, 1, 2.0),      # tiny d, one candidate
    (64, 1000, 33, 2, 1.0),     # dot_scale 1, d not a multiple of 4
    (100, 200, 7, 17, 2.0),     # irregular k (reference tests k in {1,3,8,17,32})
    (50, 40, 100, 32, 2.0),     # k close to n
    (300, 500, 300, 3, 2.0),    # two-level fp32 accumulation (d > 256)
    (300, 700, 200, 17, 2.0),   # split sweep with 256-row panels and 40-entry partial lists
    (520, 3000, 640, 4, 1.0),   # 256-row panels (the last ragged), 20 chunks per tile, 24 tiles per row
    (1, 1, 1, 1, 2.0),          # smallest problem
    (5, 3, 16, 8, 2.0),         # k > n: sentinel slots
])
@pytest.mark.parametrize("precision", ["fp32", "bf16x3", "int8x3"])
def test_l2sq_bidirectional_matches_oracle(cuda, m, n, d, k, scale, precision):
    X, Y, p, q, qb, db = _l2sq_case(m, n, d, seed=m + 7 * n + d)
    orv, ori, ocv, oci, ost = oracle.l2sq_scan(X, Y, p, q, qb, db, k, scale)
    tX, tY, tp, tq, tqb, tdb = _to(cuda, X, Y, p, q, qb, db)
    rv, ri, cv, ci, st = pricing_l2sq(tX, tY, tp, tq, tqb, tdb, k, dot_scale=scale, rows=True, cols=True,
                                      stats=True, linf=True, precision=precision)
    np.testing.assert_array_equal(ri.cpu().numpy(), ori)
    np.testing.assert_array_equal(ci.cpu().numpy(), oci)
    np.testing.assert_array_equal(rv.cpu().numpy(), orv)   # exact fp64 re-evaluation: same bits
    np.testing.assert_array_equal(cv.cpu().numpy(), ocv)
    assert_l2sq_certificate(st, l2sq_certificate_bounds(X, Y, p, q, qb, db, scale))


@pytest.mark.parametrize("precision", ["fp32", "bf16x3", "int8x3"])
def test_l2sq_ties_and_duplicates_lowest_index_wins(cuda, precision):
    X, Y, p, q, qb, db = _l2sq_case(200, 301, 8, seed=5, dup=True, integer=True)
    for k in (1, 4, 16):
        orv, ori, ocv, oci, _ = oracle.l2sq_scan(X, Y, p, q, qb, db, k, 2.0)
        rv, ri, cv, ci, _ = pricing_l2sq(*_to(cuda, X, Y, p, q, qb, db), k, stats=False, precision=precision)
        np.testing.assert_array_equal(ri.cpu().numpy(), ori)
        np.testing.assert_array_equal(ci.cpu().numpy(), oci)
        np.testing.assert_array_equal(rv.cpu().numpy(), orv)


@pytest.mark.parametrize("m,n,d,k,integer", [
    (65536 + 300, 97, 256, 2, True),    # columns fused into the row sweep, merged across two query chunks
    (65536 + 300, 97, 256, 8, False),
    (2 * 65536 + 300, 97, 256, 4, False),  # three query chunks: later chunks' lists start at the running floors
    (65536 + 300, 97, 12, 8, True),     # columns by a second, role-swapped sweep; query side in two chunks
    (97, 65536 + 300, 12, 3, True),     # role-swapped sweep over two resident-side chunks
])
@pytest.mark.parametrize("precision", ["fp32", "bf16x3", "int8x3"])
def test_l2sq_chunked_sides_and_ties(cuda, m, n, d, k, integer, precision):
    """Shapes with more than 65536 rows on one side: the kernel processes that side in internal chunks (and,
    with fused columns, merges the exact column lists across query chunks). With integer data every score is
    exact and ties abound; duplicated rows placed in different chunks must resolve to the lower index."""
    X, Y, p, q, qb, db = _l2sq_case(m, n, d, seed=31 + k + d, integer=integer)
    big, side = (X, "x") if m > n else (Y, "y")
    for src, dst in ((3, 65536 + 7), (40, 65536 + 250), (5000, 65536 + 1)):
        big[dst] = big[src]
        if side == "x":
            p[dst], qb[dst] = p[src], qb[src]
        else:
            q[dst], db[dst] = q[src], db[src]
    orv, ori, ocv, oci, ost = oracle.l2sq_scan(X, Y, p, q, qb, db, k, 2.0)
    rv, ri, cv, ci, st = pricing_l2sq(*_to(cuda, X, Y, p, q, qb, db), k, linf=True, precision=precision)
    np.testing.assert_array_equal(ci.cpu().numpy(), oci)
    np.testing.assert_array_equal(cv.cpu().numpy(), ocv)
    np.testing.assert_array_equal(ri.cpu().numpy(), ori)
    np.testing.assert_array_equal(rv.cpu().numpy(), orv)
    assert_l2sq_certificate(st, l2sq_certificate_bounds(X, Y, p, q, qb, db))


@pytest.mark.parametrize("precision", ["fp32", "bf16x3", "int8x3"])
@pytest.mark.parametrize("copies", [400, 1500])
def test_l2sq_dense_near_ties_resolved_exactly(cuda, precision, copies):
    # `copies` target rows sit within 1e-4 of one point the queries also sit near: every query row has hundreds
    # of candidates inside twice the sweep's error bound. 400 are resolved by the wide pass (under its 512-candidate
    # capacity), 1500 overflow it into the exact full rescan; both must give the oracle's exact lists.
    rng = np.random.default_rng(copies)
    m, n, d, k = 40, 2000, 300, 8
    base = rng.standard_normal(d).astype(np.float32)
    X = (base + 1e-3 * rng.standard_normal((m, d))).astype(np.float32)
    Y = (3.0 * rng.standard_normal((n, d))).astype(np.float32)
    Y[:copies] = (base + 1e-4 * rng.standard_normal((copies, d))).astype(np.float32)
    p = (X.astype(np.float64) ** 2).sum(1)
    q = (Y.astype(np.float64) ** 2).sum(1)
    qb, db = -p, -q
    orv, ori, ocv, oci, ost = oracle.l2sq_scan(X, Y, p, q, qb, db, k, 2.0)
    rv, ri, cv, ci, st = pricing_l2sq(*_to(cuda, X, Y, p, q, qb, db), k, linf=True, precision=precision)
    np.testing.assert_array_equal(ri.cpu().numpy(), ori)
    np.testing.assert_array_equal(rv.cpu().numpy(), orv)
    np.testing.assert_array_equal(ci.cpu().numpy(), oci)
    np.testing.assert_array_equal(cv.cpu().numpy(), ocv)
    # every pair's sigma lies within the dot's rounding of 0 here: the certificate must stay inside its interval
    assert_l2sq_certificate(st, l2sq_certificate_bounds(X, Y, p, q, qb, db))


@pytest.mark.parametrize("d,precision", [(300, "fp32"), (300, "bf16x3"), (300, "int8x3"), (64, "fp32"),
                                         (64, "bf16x3")])
def test_l2sq_scattered_near_ties_resolved_from_lists(cuda, d, precision):
    # 40 query rows and 40 candidates sit within 1e-3 of one point, scattered over both sides: each such row (and
    # column) has 40 candidates inside twice the sweep's error bound, more than its merged list keeps, but spread
    # over its partial lists so that none holds KL of them. The finalize then resolves it from the lists it
    # already has (queue 1, no new sweep); the lists must still be the oracle's exact ones.
    rng = np.random.default_rng(d)
    m, n, k = 2048, 2000, 8
    base = rng.standard_normal(d).astype(np.float32)
    X = (3.0 * rng.standard_normal((m, d))).astype(np.float32)
    Y = (3.0 * rng.standard_normal((n, d))).astype(np.float32)
    xs = rng.choice(m, 40, replace=False)
    ys = rng.choice(n, 40, replace=False)
    X[xs] = (base + 1e-3 * rng.standard_normal((40, d))).astype(np.float32)
    Y[ys] = (base + 1e-3 * rng.standard_normal((40, d))).astype(np.float32)
    p = (X.astype(np.float64) ** 2).sum(1)
    q = (Y.astype(np.float64) ** 2).sum(1)
    qb, db = -p, -q
    orv, ori, ocv, oci, ost = oracle.l2sq_scan(X, Y, p, q, qb, db, k, 2.0)
    _lib.profile_reset()
    _lib.profile_enable(True)
    try:
        rv, ri, cv, ci, st = pricing_l2sq(*_to(cuda, X, Y, p, q, qb, db), k, linf=True, precision=precision)
        torch.cuda.synchronize()
        from_lists = _lib.profile_query("l2sq_list_rows")[1], _lib.profile_query("l2sq_list_columns")[1]
    finally:
        _lib.profile_enable(False)
    np.testing.assert_array_equal(ri.cpu().numpy(), ori)
    np.testing.assert_array_equal(rv.cpu().numpy(), orv)
    np.testing.assert_array_equal(ci.cpu().numpy(), oci)
    np.testing.assert_array_equal(cv.cpu().numpy(), ocv)
    assert from_lists[0] > 0 and from_lists[1] > 0, from_lists


@pytest.mark.parametrize("m,d,precision", [(70, 4, "fp32"), (300, 256, "bf16x3"), (300, 256, "int8x3")])
def test_l2sq_all_equal_scores_take_lowest_indices(cuda, m, d, precision):
    # every pair ties exactly: integer-valued identical points -> every row's top-k is columns 0..k-1 and every
    # column's is rows 0..k-1 (at d = 256 through the 256-row split sweep's fused column lists)
    n, k = 500, 8
    X = np.ones((m, d), np.float32)
    Y = np.ones((n, d), np.float32)
    p = (X.astype(np.float64) ** 2).sum(1)
    q = (Y.astype(np.float64) ** 2).sum(1)
    qb, db = -p, -q
    rv, ri, cv, ci, st = pricing_l2sq(*_to(cuda, X, Y, p, q, qb, db), k, precision=precision)
    assert (ri.cpu().numpy() == np.arange(k)[None, :]).all()
    assert (ci.cpu().numpy() == np.arange(k)[None, :]).all()
    assert (rv.cpu().numpy() == 0.0).all()


@pytest.mark.parametrize("precision", ["fp32", "bf16x3", "int8x3"])
def test_l2sq_c2_shape_properties_and_sampled_rows(cuda, precision):
    """C2 (131072 x 131072, d=64, k=8): full-size run, every row sorted with valid indices, and 96 random
    rows plus 96 random columns re-derived by the oracle."""
    m = n = 131072
    d, k = 64, 8
    g = torch.Generator(device="cpu").manual_seed(42)
    X = torch.randn(m, d, generator=g, dtype=torch.float32)
    Y = torch.randn(n, d, generator=g, dtype=torch.float32)
    f = 64.0 + 2.0 * torch.randn(m, generator=g, dtype=torch.float64)
    gg = 64.0 + 2.0 * torch.randn(n, generator=g, dtype=torch.float64)
    p = (X.double() ** 2).sum(1)
    q = (Y.double() ** 2).sum(1)
    rv, ri, cv, ci, st = pricing_l2sq(*[t.to(cuda) for t in (X, Y, p, q, f - p, gg - q)], k, precision=precision)
    rv, ri, cv, ci = rv.cpu().numpy(), ri.cpu().numpy(), cv.cpu().numpy(), ci.cpu().numpy()
    assert (np.diff(rv, axis=1) <= 0).all() and (np.diff(cv, axis=1) <= 0).all()
    assert ri.min() >= 0 and ri.max() < n and ci.min() >= 0 and ci.max() < m
    rng = np.random.default_rng(0)
    Xn, Yn, pn, qn = X.numpy(), Y.numpy(), p.numpy(), q.numpy()
    qbn, dbn = (f - p).numpy(), (gg - q).numpy()
    rows = rng.choice(m, 96, replace=False)
    orv, ori = oracle.topk(oracle.l2sq_matrices(Xn[rows], Yn, pn[rows], qn, qbn[rows], dbn, 2.0)[0], k)
    np.testing.assert_array_equal(ri[rows], ori)
    np.testing.assert_array_equal(rv[rows], orv)
    cols = rng.choice(n, 96, replace=False)
    sig_c = oracle.l2sq_matrices(Xn, Yn[cols], pn, qn[cols], qbn, dbn[cols], 2.0)[0]
    ocv, oci = oracle.topk(sig_c, k, transpose=True)
    np.testing.assert_array_equal(ci[cols], oci)
    np.testing.assert_array_equal(cv[cols], ocv)


@pytest.mark.parametrize("kind", [0, 1, 2])
@pytest.mark.parametrize("m,n,d,k", [(300, 257, 8, 2), (129, 700, 3, 8), (64, 64, 40, 1), (20, 30, 100, 5)])
def test_norm_bidirectional_matches_oracle(cuda, kind, m, n, d, k):
    rng = np.random.default_rng(m + n + d + kind)
    X = rng.random((m, d)).astype(np.float32)
    Y = rng.random((n, d)).astype(np.float32)
    f = rng.normal(0.3, 0.2, m)
    g = rng.normal(0.3, 0.2, n)
    orv, ori, ocv, oci, ost = oracle.norm_scan(X, Y, f, g, k, kind)
    rv, ri, cv, ci, st = pricing_norm(*_to(cuda, X, Y, f, g), k, kind)
    np.testing.assert_array_equal(ri.cpu().numpy(), ori)
    np.testing.assert_array_equal(ci.cpu().numpy(), oci)
    np.testing.assert_array_equal(rv.cpu().numpy(), orv)
    np.testing.assert_array_equal(cv.cpu().numpy(), ocv)
    _assert_stats(st, ost)
    np.testing.assert_allclose(st[4].item(), ost[4], rtol=1e-7)


@pytest.mark.parametrize("kind", [0, 1, 2])
@pytest.mark.parametrize("m,n,d,k", [(300, 257, 8, 2), (129, 700, 3, 8), (64, 64, 40, 1), (20, 30, 100, 5),
                                     (257, 300, 64, 32), (40, 600, 130, 2)])
def test_norm_fp64_bidirectional_matches_oracle(cuda, kind, m, n, d, k):
    """fp64 costs (HM_FP64, the reference's compute_precision = 1): lists bit-exact against the oracle's fp64 costs,
    count and maximum exact, the fp64 sums to 1e-12 (their order is not fixed)."""
    rng = np.random.default_rng(7 * m + n + d + kind)
    X = rng.random((m, d)).astype(np.float32)
    Y = rng.random((n, d)).astype(np.float32)
    f = rng.normal(0.3, 0.2, m) * d ** 0.5
    g = rng.normal(0.3, 0.2, n) * d ** 0.5
    orv, ori, ocv, oci, ost = oracle.norm_scan(X, Y, f, g, k, kind, precision=1)
    rv, ri, cv, ci, st = pricing_norm(*_to(cuda, X, Y, f, g), k, kind, precision="fp64")
    np.testing.assert_array_equal(ri.cpu().numpy(), ori)
    np.testing.assert_array_equal(ci.cpu().numpy(), oci)
    np.testing.assert_array_equal(rv.cpu().numpy(), orv)
    np.testing.assert_array_equal(cv.cpu().numpy(), ocv)
    got = st.cpu().numpy()
    np.testing.assert_allclose(got[[0, 1]], ost[[0, 1]], rtol=1e-12)
    assert got[2] == ost[2] and got[3] == ost[3] and got[4] == ost[4]
    # the fp64 and fp32 costs rank differently somewhere (the flag reaches the kernel)
    _, _, _, _, ost32 = oracle.norm_scan(X, Y, f, g, k, kind)
    assert ost32[0] != ost[0] or ost32[1] != ost[1]


def test_norm_fp64_scan_extension_and_solve(cuda):
    """ScanExtension's compute_precision = 1 reaches the fp64 sweep, and an l1 solve at cost_precision='fp64'
    (fp64 scans and fp64 pair costs on every level) lands on the exact LP optimum of the fp64 costs."""
    from scipy.optimize import linprog

    from hello_ot_amd import SolverOptions, solve

    rng = np.random.default_rng(64)
    X = rng.random((90, 5)).astype(np.float32)
    Y = rng.random((110, 5)).astype(np.float32)
    f, g = rng.normal(0.5, 0.1, 90), rng.normal(0.5, 0.1, 110)
    ext = ScanExtension()
    out = ext.fused_gcost_bidir_certificate(*_to(cuda, X, Y, f, g), 2, 0, compute_precision=1)
    orv, ori, ocv, oci, ost = oracle.norm_scan(X, Y, f, g, 2, 0, precision=1)
    np.testing.assert_array_equal(out[0].cpu().numpy(), orv)
    np.testing.assert_array_equal(out[3].cpu().numpy(), oci)
    assert int(out[8]) == ost[2]
    a, b = np.full(90, 1 / 90), np.full(110, 1 / 110)
    r = solve(X, Y, source_mass=a, target_mass=b, cost="l1",
              options=SolverOptions(cost_precision="fp64", coarsest_size_threshold=30, verbose="off"))
    assert all(l.solve.summary.converged for l in r.solve_stage.levels if l.kind == "refined")
    _, C = oracle.norm_matrices(X, Y, np.zeros(90), np.zeros(110), 0, precision=1)
    A = np.zeros((200, 90 * 110))
    for i in range(90):
        A[i, i * 110:(i + 1) * 110] = 1.0
    for j in range(110):
        A[90 + j, j::110] = 1.0
    exact = linprog(C.reshape(-1), A_eq=A, b_eq=np.concatenate((a, b)), bounds=(0, None), method="highs").fun
    assert abs(r.objective - exact) <= 5e-6 * exact
    assert r.metadata["cost_precision"] == "fp64"


def test_norm_ties_on_a_grid(cuda):
    # integer grid points: many exactly equal l1 distances
    rng = np.random.default_rng(2)
    X = rng.integers(0, 4, (100, 2)).astype(np.float32)
    Y = rng.integers(0, 4, (150, 2)).astype(np.float32)
    f = np.zeros(100)
    g = np.zeros(150)
    for kind in (0, 1):
        orv, ori, ocv, oci, _ = oracle.norm_scan(X, Y, f, g, 4, kind)
        rv, ri, cv, ci, _ = pricing_norm(*_to(cuda, X, Y, f, g), 4, kind, stats=False)
        np.testing.assert_array_equal(ri.cpu().numpy(), ori)
        np.testing.assert_array_equal(ci.cpu().numpy(), oci)


def test_scan_extension_reference_layouts(cuda):
    ext = ScanExtension()
    X, Y, p, q, qb, db = _l2sq_case(90, 110, 16, seed=3)
    out = ext.fused_bidir_topk_stats_raw(*_to(cuda, X, Y, p, q, qb, db), 4096, 4096, 256, 2, True, True, False, 2, 2.0)
    assert out[0].shape == (90, 2) and out[0].dtype == torch.float64
    assert out[1].dtype == torch.int32 and out[3].dtype == torch.int32
    assert out[4].shape == (4,) and out[5].device.type == "cpu"
    _, _, _, _, ost = oracle.l2sq_scan(X, Y, p, q, qb, db, 2, 2.0)
    np.testing.assert_allclose(out[4].cpu().numpy(), [ost[0], ost[1], ost[2], ost[4]], rtol=2e-5)
    with pytest.raises(ValueError, match="power-of-two bucket"):
        ext.fused_bidir_topk_stats_raw(*_to(cuda, X, Y, p, q, qb, db), 1, 1, 256, 3, True, True, False, 0, 2.0)
    with pytest.raises(ValueError, match="invalid raw pricing tile"):
        ext.fused_bidir_topk_stats_raw(*_to(cuda, X, Y, p, q, qb, db), 1, 1, 256, 2, True, True, False, 2, 3.0)
    f = np.random.default_rng(1).random(90)
    g = np.random.default_rng(2).random(110)
    norm = ext.fused_gcost_bidir_certificate(*_to(cuda, X, Y, f, g), 4, 0)
    assert len(norm) == 9 and norm[1].dtype == torch.int64 and norm[8].dtype == torch.int64


@pytest.mark.parametrize("precision", ["fp32", "bf16x3", "int8x3"])
@pytest.mark.parametrize("m,n,k", [(300, 3000, 2), (70, 1000, 16)])
def test_l2sq_c5_feature_count_matches_oracle(cuda, precision, m, n, k):
    """d = 8192 (the C5 feature count): the long-accumulation path of both sweeps (staggered 128-feature block
    restarts, 64-chunk error-bound terms) against the oracle's exact lists."""
    d = 8192
    rng = np.random.default_rng(m + n + k)
    means = 2.0 * rng.standard_normal((8, d))
    X = (means[rng.integers(0, 8, m)] + rng.standard_normal((m, d))).astype(np.float32)
    Y = (means[rng.integers(0, 8, n)] + rng.standard_normal((n, d))).astype(np.float32)
    p = (X.astype(np.float64) ** 2).sum(1)
    q = (Y.astype(np.float64) ** 2).sum(1)
    sigma0, cost0 = oracle.l2sq_matrices(X, Y, p, q, -p, -q, 2.0)
    f = (cost0.min(1) + rng.normal(0.0, 40.0, m))         # near a c-transform: a few violated pairs per row
    g = np.zeros(n)
    orv, ori, ocv, oci, ost = oracle.l2sq_scan(X, Y, p, q, f - p, g - q, k, 2.0)
    rv, ri, cv, ci, st = pricing_l2sq(*_to(cuda, X, Y, p, q, f - p, g - q), k, linf=True, precision=precision)
    np.testing.assert_array_equal(ri.cpu().numpy(), ori)
    np.testing.assert_array_equal(rv.cpu().numpy(), orv)
    np.testing.assert_array_equal(ci.cpu().numpy(), oci)
    np.testing.assert_array_equal(cv.cpu().numpy(), ocv)
    assert_l2sq_certificate(st, l2sq_certificate_bounds(X, Y, p, q, f - p, g - q))


@pytest.mark.parametrize("precision", ["fp32", "bf16x3", "int8x3"])
@pytest.mark.parametrize("d", [40, 300])
def test_l2sq_stats_only_matches_oracle(cuda, precision, d):
    """Certificate-only calls (ScanExtension.raw_lowrank_stats_only, generic_scan.py:502-510): the five sums
    without candidate lists; the maximum violation is the exact fp64 maximum."""
    X, Y, p, q, qb, db = _l2sq_case(333, 517, d, seed=d)
    f, g = qb + p, db + q
    bounds = l2sq_certificate_bounds(X, Y, p, q, qb, db)
    st = pricing_l2sq(*_to(cuda, X, Y, p, q, qb, db), 1, rows=False, cols=False, stats=True, linf=True,
                      precision=precision)[4]
    assert_l2sq_certificate(st, bounds)
    # the reference's entry point (default sweep precision for this d)
    assert_l2sq_certificate(ScanExtension().raw_lowrank_stats_only(*_to(cuda, X, Y, p, q, f, g), 4096, 4096, 2.0),
                            bounds)


@pytest.mark.parametrize("precision", ["fp32", "bf16x3", "int8x3"])
@pytest.mark.parametrize("d", [24, 300])
def test_l2sq_directional_top16_with_one_zero_side(cuda, precision, d):
    """The initialization's directional scans (initialization/state.py:493-689, initial.cu:33-100): rows only with
    f = 0 (per source row the 16 best g_j - c_ij) and columns only with g = 0, as the host loop calls them."""
    X, Y, p, q, qb, db = _l2sq_case(410, 390, d, seed=7 * d)
    f0, g0 = np.zeros(len(X)), np.zeros(len(Y))
    g, f = db + q, qb + p
    orv, ori, _, _, _ = oracle.l2sq_scan(X, Y, p, q, f0 - p, g - q, 16, 2.0)
    rv, ri, cv, ci, st = pricing_l2sq(*_to(cuda, X, Y, p, q, f0 - p, g - q), 16, rows=True, cols=False,
                                      stats=False, precision=precision)
    assert cv is None and ci is None and st is None
    np.testing.assert_array_equal(ri.cpu().numpy(), ori)
    np.testing.assert_array_equal(rv.cpu().numpy(), orv)
    _, _, ocv, oci, _ = oracle.l2sq_scan(X, Y, p, q, f - p, g0 - q, 16, 2.0)
    rv, ri, cv, ci, _ = pricing_l2sq(*_to(cuda, X, Y, p, q, f - p, g0 - q), 16, rows=False, cols=True,
                                     stats=False, precision=precision)
    assert rv is None and ri is None
    np.testing.assert_array_equal(ci.cpu().numpy(), oci)
    np.testing.assert_array_equal(cv.cpu().numpy(), ocv)


@pytest.mark.parametrize("kind", [0, 1, 2])
def test_norm_directional_top16_with_one_zero_side(cuda, kind):
    rng = np.random.default_rng(40 + kind)
    X = rng.random((260, 8)).astype(np.float32)
    Y = rng.random((300, 8)).astype(np.float32)
    f, g = rng.normal(0.3, 0.2, 260), rng.normal(0.3, 0.2, 300)
    orv, ori, _, _, _ = oracle.norm_scan(X, Y, np.zeros(260), g, 16, kind)
    rv, ri, _, _, _ = pricing_norm(*_to(cuda, X, Y, np.zeros(260), g), 16, kind, rows=True, cols=False, stats=False)
    np.testing.assert_array_equal(ri.cpu().numpy(), ori)
    np.testing.assert_array_equal(rv.cpu().numpy(), orv)
    _, _, ocv, oci, _ = oracle.norm_scan(X, Y, f, np.zeros(300), 16, kind)
    _, _, cv, ci, _ = pricing_norm(*_to(cuda, X, Y, f, np.zeros(300)), 16, kind, rows=False, cols=True, stats=False)
    np.testing.assert_array_equal(ci.cpu().numpy(), oci)
    np.testing.assert_array_equal(cv.cpu().numpy(), ocv)


def _norm_call(dev, X, Y, f, g, k, kind, ws_bytes, flags):
    lib = _lib.load()
    m, n, d = X.shape[0], Y.shape[0], X.shape[1]
    out = (torch.full((m, k), 7.0, dtype=torch.float64, device=dev), torch.full((m, k), 7, dtype=torch.int32, device=dev),
           torch.full((n, k), 7.0, dtype=torch.float64, device=dev), torch.full((n, k), 7, dtype=torch.int32, device=dev),
           torch.full((5,), 7.0, dtype=torch.float64, device=dev))
    ws = torch.full((ws_bytes,), 0xAB, dtype=torch.uint8, device=dev)    # stale bytes: nothing may be read unwritten
    rc = lib.hm_pricing_norm(_lib.stream_handle(dev), *map(_lib.ptr, (X, Y, f, g)), m, n, d, k, kind, flags,
                             *map(_lib.ptr, out), _lib.ptr(ws), ws.numel())
    return rc, out


@pytest.mark.parametrize("kind", [0, 1, 2])
@pytest.mark.parametrize("m,n,d,k", [(300, 257, 100, 2), (130, 400, 65, 1), (257, 129, 9, 2)])
def test_norm_fused_sweep_ragged_rows_and_wide_features(cuda, kind, m, n, d, k):
    """The fused sweep (k <= 2, rows and columns) with a partial last workgroup of rows, features past the register
    width (d > 64: streamed from memory) and ragged column tiles, against the oracle."""
    rng = np.random.default_rng(m + 3 * n + d + kind)
    X = rng.random((m, d)).astype(np.float32)
    Y = rng.random((n, d)).astype(np.float32)
    f, g = rng.normal(0.3, 0.2, m), rng.normal(0.3, 0.2, n)
    orv, ori, ocv, oci, ost = oracle.norm_scan(X, Y, f, g, k, kind)
    rv, ri, cv, ci, st = pricing_norm(*_to(cuda, X, Y, f, g), k, kind)
    np.testing.assert_array_equal(ri.cpu().numpy(), ori)
    np.testing.assert_array_equal(rv.cpu().numpy(), orv)
    np.testing.assert_array_equal(ci.cpu().numpy(), oci)
    np.testing.assert_array_equal(cv.cpu().numpy(), ocv)
    _assert_stats(st, ost)


@pytest.mark.parametrize("kind", [0, 1, 2])
@pytest.mark.parametrize("k,grid", [(2, False), (1, False), (2, True)])
def test_norm_fused_columns_overflow_and_two_sweep_paths_agree(cuda, kind, k, grid):
    """k <= 2 bidirectional calls evaluate each pair once and collect the column lists through the candidate buffer.
    The workspace size picks the path: the full buffer, a buffer of about 100 candidates (it overflows, so the
    role-swapped sweep supplies the columns) and the smallest accepted workspace (two sweeps). All three equal the
    oracle. The grid case makes most scores tie exactly (integer features, zero duals)."""
    rng = np.random.default_rng(70 + kind + 3 * k + 10 * grid)
    m, n, d = 3000, 2100, 6
    if grid:
        X = rng.integers(0, 3, (m, d)).astype(np.float32)
        Y = rng.integers(0, 3, (n, d)).astype(np.float32)
        f, g = np.zeros(m), np.zeros(n)
    else:
        X = rng.random((m, d)).astype(np.float32)
        Y = rng.random((n, d)).astype(np.float32)
        f, g = rng.normal(0.3, 0.2, m), rng.normal(0.3, 0.2, n)
    orv, ori, ocv, oci, ost = oracle.norm_scan(X, Y, f, g, k, kind)
    tX, tY, tf, tg = _to(cuda, X, Y, f, g)
    flags = _lib.HM_ROWS | _lib.HM_COLS | _lib.HM_STATS | _lib.HM_LINF
    lib = _lib.load()
    full = int(lib.hm_pricing_norm_workspace_bytes(m, n, d, k, flags))
    # the library's full capacity is 16 n k + 65536 candidates of 20 bytes (16 in the buffer, 4 in the grouping)
    small = full - 20 * (16 * n * k + 65536 - 100)
    rc, _ = _norm_call(cuda, tX, tY, tf, tg, k, kind, 1024, flags)
    assert rc == _lib.HM_ENOSPC and "too small" in _lib.last_error()
    least = int(_lib.last_error().split("<")[1].split()[0])         # the two-sweep minimum the error names
    assert least < small < full
    for ws in (full, small, least):
        rc, (rv, ri, cv, ci, st) = _norm_call(cuda, tX, tY, tf, tg, k, kind, ws, flags)
        _lib.check(rc, "hm_pricing_norm")
        np.testing.assert_array_equal(ri.cpu().numpy(), ori)
        np.testing.assert_array_equal(rv.cpu().numpy(), orv)
        np.testing.assert_array_equal(ci.cpu().numpy(), oci)
        np.testing.assert_array_equal(cv.cpu().numpy(), ocv)
        _assert_stats(st, ost)


@pytest.mark.parametrize("k", [1, 2])
def test_reference_module_names_raw_entry_points(cuda, k):
    """hello_ot_native.hierot_generic_{pricing_small,cost}_ext under the reference's module names: raw_scan_tiled's
    lists and stats, raw_initial's rows-only top-k and raw_certificate_tiled in both stat layouts, against the
    oracle on raw scores (scale * <x, y> + qb) + dbb and costs (nx + ny) - scale * <x, y>."""
    import importlib

    small = importlib.import_module("hello_ot_native.hierot_generic_pricing_small_ext")
    cost = importlib.import_module("hello_ot_native.hierot_generic_cost_ext")
    X, Y, p, q, qb, db = _l2sq_case(170, 230, 40, seed=50 + k)
    tX, tY, tp, tq, tqb, tdb = _to(cuda, X, Y, p, q, qb, db)
    orv, ori, ocv, oci, ost = oracle.l2sq_scan(X, Y, p, q, qb, db, k, 2.0)
    rv, ri, cv, ci, st, timing = small.raw_scan_tiled(tX, tY, tp, tq, tqb, tdb, k, 2.0, True, True, 64, 64)
    np.testing.assert_array_equal(ri.cpu().numpy(), ori)
    np.testing.assert_array_equal(rv.cpu().numpy(), orv)
    np.testing.assert_array_equal(ci.cpu().numpy(), oci)
    np.testing.assert_array_equal(cv.cpu().numpy(), ocv)
    assert ri.dtype == torch.int32 and timing.device.type == "cpu" and st.shape == (4,)
    b, got = l2sq_certificate_bounds(X, Y, p, q, qb, db), st.cpu().numpy()     # (num, den, count, max|cost|)
    assert b["num"][0] * (1 - 1e-9) <= got[0] <= b["num"][1] * (1 + 1e-9)
    assert abs(got[1] - b["den"]) <= b["den_slack"] + 1e-5 * b["den"]
    assert b["count"][0] <= got[2] <= b["count"][1]
    assert abs(got[3] - b["cmax"]) <= b["envelope"] + 1e-6 * b["cmax"]
    vals, idx = cost.raw_initial(tX, tY, tqb, tdb, 8, 64, 64, 2.0)
    zr, zc = np.zeros(len(X)), np.zeros(len(Y))
    dv, di, _, _, _ = oracle.l2sq_scan(X, Y, zr, zc, qb, db, 8, 2.0)     # raw scores do not involve the costs
    np.testing.assert_array_equal(idx.cpu().numpy(), di)
    np.testing.assert_array_equal(vals.cpu().numpy(), dv)
    f, g = qb + p, db + q                                   # duals; the entry point forms f - nx and g - ny
    tf, tg = _to(cuda, f, g)
    caller = cost.raw_certificate_tiled(tX, tY, tp, tq, tf, tg, 64, 64, 2.0, True, False, True)
    kernel = cost.raw_certificate_tiled(tX, tY, tp, tq, tf, tg, 64, 64, 2.0, True, False, False)
    np.testing.assert_array_equal(kernel.cpu().numpy(), caller.cpu().numpy()[[0, 1, 3, 4, 2]])
    assert_l2sq_certificate(caller, l2sq_certificate_bounds(X, Y, p, q, f - p, g - q))
    # squared norms: fp64 sums of exact squares, equal up to the summation order
    np.testing.assert_allclose(cost.norms(tX).cpu().numpy(), (X.astype(np.float64) ** 2).sum(1), rtol=1e-14)


@pytest.mark.parametrize("kind", [0, 1, 2])
def test_scan_extension_norm_directional_and_certificate(cuda, kind):
    """ScanExtension.fused_gcost_topk (ascending cost - dual, int64 ids) and fused_gcost_certificate (num, den, max,
    costmax, count), against the oracle's fp32 costs and exact scores."""
    rng = np.random.default_rng(60 + kind)
    X = rng.random((210, 6)).astype(np.float32)
    Y = rng.random((190, 6)).astype(np.float32)
    f, g = rng.normal(0.3, 0.2, 210), rng.normal(0.3, 0.2, 190)
    ext = ScanExtension()
    tX, tY, tf, tg = _to(cuda, X, Y, f, g)
    vals, ids = ext.fused_gcost_topk(tX, tY, tg, 4, kind)
    orv, ori, _, _, _ = oracle.norm_scan(X, Y, np.zeros(210), g, 4, kind)
    assert ids.dtype == torch.int64
    np.testing.assert_array_equal(ids.cpu().numpy(), ori)
    np.testing.assert_array_equal(vals.cpu().numpy(), -orv)
    assert (np.diff(vals.cpu().numpy(), axis=1) >= 0).all()
    num, den, mx, cmax, count = ext.fused_gcost_certificate(tX, tY, tf, tg, kind)
    _, _, _, _, ost = oracle.norm_scan(X, Y, f, g, 1, kind)
    _assert_stats(torch.stack((num, den, count.double(), mx, cmax)), ost)
    np.testing.assert_allclose(cmax.item(), ost[4], rtol=1e-7)
    assert count.dtype == torch.int64
    _, den0, _, _, _ = ext.fused_gcost_certificate(tX, tY, tf, tg, kind, 0)    # six-argument form, no denominator
    assert den0.item() == 0.0


@pytest.mark.parametrize("precision", ["fp32", "bf16x3", "int8x3"])
@pytest.mark.parametrize("k,rows", [(4, False), (2, True)])
def test_l2sq_column_floor_keeps_every_entry_above_it(cuda, precision, k, rows):
    """hm_pricing_l2sq_resident_floor: with a floor per column the column lists keep, in place, every entry of the
    full lists that scores at least the floor (ties at the floor included), and whatever follows scores below it or
    is padding; merged into the lists the floors came from they give exactly the full lists' merge. Columns-only
    calls take the role-swapped pass, rows + columns with k <= 2 the fused column lists."""
    from hello_ot_amd.resident.cost import merge_columns

    X, Y, p, q, qb, db = _l2sq_case(600, 3000, 300, seed=37)
    tX, tY, tp, tq, tqb, tdb = _to(cuda, X, Y, p, q, qb, db)
    side = ResidentSide(tY, precision)
    first = pricing_l2sq(tX[:256], tY, tp[:256], tq, tqb[:256], tdb, k, rows=rows, stats=False, resident=side)
    full = pricing_l2sq(tX[256:], tY, tp[256:], tq, tqb[256:], tdb, k, rows=rows, stats=False, resident=side)
    fv, fi = full[2].cpu().numpy(), full[3].cpu().numpy()
    # floors: the first chunk's k-th scores, then some columns without one, some set to an entry of the full list
    # (a tie at the floor) and some above every score
    floor = first[2][:, k - 1].clone()
    floor[::7] = -float("inf")
    floor[3::11] = full[2][3::11, 0]
    floor[5::13] = full[2][5::13, k - 1]
    floor[9::17] = 1e300
    got = pricing_l2sq(tX[256:], tY, tp[256:], tq, tqb[256:], tdb, k, rows=rows, stats=False, resident=side,
                       col_floor=floor)
    if rows:
        assert torch.equal(got[0], full[0]) and torch.equal(got[1], full[1])
    gv, gi = got[2].cpu().numpy(), got[3].cpu().numpy()
    fl = floor.cpu().numpy()[:, None]
    above = fv >= fl                                     # lists are sorted: a prefix of each row
    np.testing.assert_array_equal(np.where(above, gv, 0.0), np.where(above, fv, 0.0))
    np.testing.assert_array_equal(np.where(above, gi, 0), np.where(above, fi, 0))
    rest = ~above
    assert (gv[rest] < fl.repeat(k, axis=1)[rest]).all()
    assert ((gi[rest] == -1) == np.isneginf(gv[rest])).all()
    skipped = int(np.isneginf(gv).sum() - np.isneginf(fv).sum())
    assert skipped > 0                                   # columns the chunk cannot change were left out
    # the streamed scan's use: the floors of the first chunk's lists, then the merge
    base = first[2][:, k - 1].contiguous()
    got = pricing_l2sq(tX[256:], tY, tp[256:], tq, tqb[256:], tdb, k, rows=rows, stats=False, resident=side,
                       col_floor=base)
    shift = lambda out: (out[2], torch.where(out[3] >= 0, out[3] + 256, out[3]))
    ref_v, ref_i = merge_columns((first[2], first[3]), shift(full), k)
    mv, mi = merge_columns((first[2], first[3]), shift(got), k)
    assert torch.equal(mv, ref_v) and torch.equal(mi, ref_i)
    with pytest.raises(ValueError, match="col_floor"):
        pricing_l2sq(tX, tY, tp, tq, tqb, tdb, k, col_floor=base)


@pytest.mark.parametrize("precision", ["fp32", "bf16x3", "int8x3"])
def test_l2sq_resident_side_gives_the_same_outputs(cuda, precision):
    """Query chunks priced against a resident Y side (prepared once) give exactly the ordinary call's outputs,
    chunk after chunk; the first chunk also equals the oracle. A side prepared for another precision, or another
    tensor, is rejected."""
    X, Y, p, q, qb, db = _l2sq_case(600, 3000, 300, seed=31)
    tX, tY, tp, tq, tqb, tdb = _to(cuda, X, Y, p, q, qb, db)
    side = ResidentSide(tY, precision)
    for s, e in ((0, 256), (256, 600), (0, 256)):
        args = (tX[s:e], tY, tp[s:e], tq, tqb[s:e], tdb, 4)
        ref = pricing_l2sq(*args, linf=True, precision=precision)
        got = pricing_l2sq(*args, linf=True, resident=side)
        for a, b in zip(ref, got):
            assert torch.equal(a, b)
    orv, ori, ocv, oci, _ = oracle.l2sq_scan(X[:256], Y, p[:256], q, qb[:256], db, 4, 2.0)
    rv, ri, cv, ci, _ = pricing_l2sq(tX[:256], tY, tp[:256], tq, tqb[:256], tdb, 4, resident=side)
    np.testing.assert_array_equal(ri.cpu().numpy(), ori)
    np.testing.assert_array_equal(rv.cpu().numpy(), orv)
    np.testing.assert_array_equal(ci.cpu().numpy(), oci)
    other = "fp32" if precision != "fp32" else "bf16x3"
    with pytest.raises(ValueError, match="prepared for precision"):
        pricing_l2sq(tX, tY, tp, tq, tqb, tdb, 4, precision=other, resident=side)
    with pytest.raises(ValueError, match="tensor it was prepared from"):
        pricing_l2sq(tX, tY.clone(), tp, tq, tqb, tdb, 4, resident=side)
    # the library's own check of the precision bits (the Python mirror is bypassed here)
    lib = _lib.load()
    flags = 7 | (_lib.HM_BF16X3 if other == "bf16x3" else 0)
    ws = torch.empty(lib.hm_pricing_l2sq_resident_workspace_bytes(600, 3000, 300, 4, flags), dtype=torch.uint8,
                     device=cuda)
    out = [torch.empty((600, 4), dtype=torch.float64, device=cuda), torch.empty((600, 4), dtype=torch.int32, device=cuda),
           torch.empty((3000, 4), dtype=torch.float64, device=cuda), torch.empty((3000, 4), dtype=torch.int32, device=cuda),
           torch.empty(5, dtype=torch.float64, device=cuda)]
    rc = lib.hm_pricing_l2sq_resident(_lib.stream_handle(cuda), *(_lib.ptr(t) for t in (tX, tY, tp, tq, tqb, tdb)), 600,
                                      3000, 300, 4, 2.0, flags, *(_lib.ptr(t) for t in out), _lib.ptr(side.buffer),
                                      side.buffer.numel(), _lib.ptr(ws), ws.numel())
    assert rc == _lib.HM_EINVAL and "another sweep precision" in _lib.last_error()
