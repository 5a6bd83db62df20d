"""The BASELINE configurations at their full shapes on the MI355X path (GPU only).

* C5 pricing step: 8192 query rows x 1,280,000 resident rows, d = 8192, k = 2 (the bench's headline step);
* C4: l1 / linf bidirectional scans at 524288 x 524288, d = 8, and the full HELLO solves of both costs;
* C3: SDDMM on the 262144 x 262144 CSR support (16 columns per row, d = 256) and 1000 PDHG iterations on it.

Candidate lists are checked bit-exactly against the CPU oracle on sampled rows and columns (the full lists are
checked for order and index range); certificate totals against an independent fp64 recomputation over all
pairs. The reference's own GPU test pins its scan the same way, on smaller shapes
(tests/hello_gpu_resident_test.py:26-67).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from _shapes import (certified_lower_bounds, exact_col_topk, exact_row_topk, fp64_certificate, gmm, norm_costs_fp32,
                     random_csr, sampled_c_transform, sqnorms)
from hello_ot_amd import SolverOptions, solve
from hello_ot_amd.costs.pairs import lowrank_csr_costs
from hello_ot_amd.kernels.generic_scan import pricing_l2sq, pricing_norm
from hello_ot_amd.lp import NativeRestrictedOTPDLP
from test_gpu_pricing import assert_l2sq_certificate

pytestmark = pytest.mark.gpu

# Certified optimality gap of the full solves at the default tolerance 1e-6: objective minus the best weak-duality
# lower bound of the returned duals, relative to the objective.
CERTIFIED_GAP = 1e-5


def _say(msg):
    print(f"[full-shape] {msg}", flush=True)


def _assert_sorted_valid(vals, idx, bound):
    vals, idx = vals.cpu().numpy(), idx.cpu().numpy()
    assert (np.diff(vals, axis=1) <= 0).all()
    assert idx.min() >= 0 and idx.max() < bound


def test_c5_pricing_step_full_shape(cuda):
    """C5 step: the three sweeps give identical exact lists; 16 rows and 16 columns equal the oracle's exact top-2;
    the certificate totals (int8 and split-bf16 sweeps) agree with an fp64 GEMM over all 1.05e10 pairs."""
    m, n, d, k = 8192, 1_280_000, 8192, 2
    _say("C5: generating 1,280,000 x 8192 resident rows")
    Y = gmm(n, d, seed=2, dev=cuda, means_seed=12)
    X = gmm(m, d, seed=1, dev=cuda, means_seed=11)
    p, q = sqnorms(X), sqnorms(Y)
    f, g = sampled_c_transform(X, Y, p, q)
    qb, db = f - p, g - q
    outs = {}
    for precision in ("int8x3", "bf16x3", "fp32"):
        _say(f"C5: {precision} sweep")
        outs[precision] = pricing_l2sq(X, Y, p, q, qb, db, k, linf=True, precision=precision)
        torch.cuda.synchronize()
    rv, ri, cv, ci, st = outs["int8x3"]
    for other in ("bf16x3", "fp32"):
        for a, b in zip(outs["int8x3"][:4], outs[other][:4]):
            assert torch.equal(a, b), other
    _assert_sorted_valid(rv, ri, n)
    _assert_sorted_valid(cv, ci, m)
    rng = np.random.default_rng(5)
    rows = np.sort(rng.choice(m, 16, replace=False))
    cols = np.sort(rng.choice(n, 16, replace=False))
    _say("C5: oracle rows (Y streamed to the host)")
    rows_t = torch.as_tensor(rows, device=cuda)
    orv, ori = exact_row_topk(X[rows_t].cpu().numpy(), Y, p[rows_t].cpu().numpy(), q, qb[rows_t].cpu().numpy(),
                              db, k)
    np.testing.assert_array_equal(ri[rows_t].cpu().numpy(), ori)
    np.testing.assert_array_equal(rv[rows_t].cpu().numpy(), orv)
    _say("C5: oracle columns")
    cols_t = torch.as_tensor(cols, device=cuda)
    ocv, oci = exact_col_topk(X, Y[cols_t].cpu().numpy(), p, q[cols_t].cpu().numpy(), qb, db[cols_t].cpu().numpy(), k)
    np.testing.assert_array_equal(ci[cols_t].cpu().numpy(), oci)
    np.testing.assert_array_equal(cv[cols_t].cpu().numpy(), ocv)
    _say("C5: fp64 certificate over all pairs")
    bounds = fp64_certificate(X, Y, p, q, qb, db)
    _say(f"C5: certificate {st.cpu().numpy().tolist()} bounds {bounds}")
    assert bounds["count"][0] > 1e5          # a refinement-like state: many violated pairs
    # the maximum from the GEMM checker is within its own rounding (~1e-12 relative) of the exact fp64 maximum
    got = st.cpu().numpy()
    np.testing.assert_allclose(got[3], bounds["max"], rtol=1e-10)
    bounds["max"] = float(got[3])
    assert_l2sq_certificate(st, bounds)
    assert_l2sq_certificate(outs["bf16x3"][4], bounds)


def _c4_inputs(dev, seed=4):
    m = 524288
    rng = np.random.default_rng(seed)
    X = torch.as_tensor(rng.random((m, 8)).astype(np.float32)).to(dev)
    Y = torch.as_tensor(rng.random((m, 8)).astype(np.float32)).to(dev)
    return rng, X, Y


def _norm_certificate(X, Y, f, g, kind, block=2048, extrema=False):
    """(num, den, count, max sigma+, max|c|) of the fp32 norm costs over all pairs, on the device; with ``extrema``
    also the maximum of sigma over each row and over each column (fp64 tensors)."""
    num = den = 0.0
    count = 0
    mx = cmax = 0.0
    row_max = torch.empty(X.shape[0], dtype=torch.float64, device=X.device)
    col_max = torch.full((Y.shape[0],), -torch.inf, dtype=torch.float64, device=X.device)
    for s in range(0, X.shape[0], block):
        c = norm_costs_fp32(X[s:s + block], Y, kind).double()
        sigma = (g[None, :] - c) + f[s:s + block, None]
        if extrema:
            row_max[s:s + block] = sigma.max(1).values
            torch.maximum(col_max, sigma.max(0).values, out=col_max)
        pos = sigma.clamp_min(0.0)
        num += float((pos * pos).sum())
        den += float((c * c).sum())
        count += int((sigma > 0).sum())
        mx = max(mx, float(pos.max()))
        cmax = max(cmax, float(c.max()))
        del c, sigma, pos
    cert = np.array([num, den, float(count), mx, cmax])
    return (cert, row_max, col_max) if extrema else cert


@pytest.mark.parametrize("kind", [0, 1])
def test_c4_norm_scan_full_shape(cuda, kind):
    """C4 scan (l1 / linf, 524288^2, d = 8): sampled rows and columns bit-exact against the oracle, the certificate
    against the same fp32 costs summed over all 2.7e11 pairs."""
    rng, X, Y = _c4_inputs(cuda)
    m = n = X.shape[0]
    f = torch.as_tensor(rng.normal(1.2, 0.1, m)).to(cuda)
    g = torch.as_tensor(rng.normal(1.2, 0.1, n)).to(cuda)
    _say(f"C4 kind={kind}: scan")
    rv, ri, cv, ci, st = pricing_norm(X, Y, f, g, 2, kind)
    _assert_sorted_valid(rv, ri, n)
    _assert_sorted_valid(cv, ci, m)
    rows = np.sort(rng.choice(m, 32, replace=False))
    cols = np.sort(rng.choice(n, 32, replace=False))
    Xh, Yh, fh, gh = X.cpu().numpy(), Y.cpu().numpy(), f.cpu().numpy(), g.cpu().numpy()
    orv, ori, _, _, _ = oracle.norm_scan(Xh[rows], Yh, fh[rows], gh, 2, kind)
    np.testing.assert_array_equal(ri.cpu().numpy()[rows], ori)
    np.testing.assert_array_equal(rv.cpu().numpy()[rows], orv)
    _, _, ocv, oci, _ = oracle.norm_scan(Xh, Yh[cols], fh, gh[cols], 2, kind)
    np.testing.assert_array_equal(ci.cpu().numpy()[cols], oci)
    np.testing.assert_array_equal(cv.cpu().numpy()[cols], ocv)
    _say(f"C4 kind={kind}: certificate over all pairs")
    ref = _norm_certificate(X, Y, f, g, kind)
    got = st.cpu().numpy()
    np.testing.assert_allclose(got[[0, 1, 4]], ref[[0, 1, 4]], rtol=1e-9)
    assert got[2] == ref[2] and got[3] == ref[3]       # exact scores: exact count and maximum


@pytest.mark.parametrize("kind", ["l1", "linf"])
def test_c4_full_solve(cuda, capsys, kind):
    """C4 solve (524288^2, d = 8, U(0.5, 1.5) masses) against an independent recomputation of HELLO's stopping rule
    over all 2.7e11 pairs: the relative l2 dual infeasibility sqrt(sum sigma+^2) / (1 + sqrt(sum c^2)) of the
    returned duals at most the 1e-6 tolerance (gpu_resident/solver.py:_refine stops on exactly this quantity),
    the last LP's primal residual and duality gap within 1e-6, and the solver's own certificate equal to the
    recomputed one.

    Objective: weak duality certifies OPT >= LB for the c-transform of the returned duals (each f_i lowered by its
    row's largest violation; the best of the row, column and uniform bounds, ``certified_lower_bounds``), computed
    from the exact maxima over all pairs. The objective of the returned plan must lie within CERTIFIED_GAP of that
    bound, relative to the objective, so it is within CERTIFIED_GAP of the optimum whatever the reference returns
    at the same tolerance."""
    rng, X, Y = _c4_inputs(cuda)
    m = X.shape[0]
    a, b = rng.uniform(0.5, 1.5, m), rng.uniform(0.5, 1.5, m)
    a, b = a / a.sum(), b / b.sum()
    _say(f"C4 solve {kind}")
    r = solve(X, Y, source_mass=a, target_mass=b, cost=kind, options=SolverOptions(verbose="off"))
    finest = r.solve_stage.levels[-1].solve
    last = finest.iterations[-1]
    assert finest.summary.converged and last.convergence.dual_feasibility <= 1e-6
    sol = r.solution.to_cpu()
    # the last LP's relative primal residual bound: ||A x - (a, b)|| <= 1e-6 (1 + ||(a, b)||)
    residual = np.concatenate((np.bincount(sol.rows, weights=sol.values, minlength=m) - a,
                               np.bincount(sol.cols, weights=sol.values, minlength=m) - b))
    assert np.linalg.norm(residual) <= 1e-6 * (1.0 + np.sqrt(a @ a + b @ b))
    assert np.abs(residual).max() <= 1e-2 / m         # no entry off by more than 1% of a mean mass
    f, g = r.solution.source_dual, r.solution.target_dual
    code = {"l1": 0, "linf": 1}[kind]
    _say(f"C4 solve {kind}: certificate of the returned duals over all pairs")
    cert, row_max, col_max = _norm_certificate(X, Y, f, g, code, extrema=True)
    infeasibility = np.sqrt(cert[0]) / (1.0 + np.sqrt(cert[1]))
    at, bt = torch.as_tensor(a, device=cuda), torch.as_tensor(b, device=cuda)
    lb = certified_lower_bounds(at, bt, f, g, row_max, col_max)
    dual_value = lb["dual_value"]
    gap = abs(r.objective - dual_value) / (1.0 + abs(r.objective) + abs(dual_value))
    certified = (r.objective - lb["best"]) / abs(r.objective)
    with capsys.disabled():
        _say(f"C4 solve {kind}: objective {r.objective!r} dual value {dual_value!r} infeasibility {infeasibility:.3e} "
             f"violated pairs {int(cert[2])} max violation {cert[3]:.3e} lower bounds row {lb['row']!r} col "
             f"{lb['col']!r} uniform {lb['uniform']!r} certified relative gap {certified:.3e}")
    assert infeasibility <= 1e-6
    np.testing.assert_allclose(infeasibility, last.convergence.dual_feasibility, rtol=1e-6)
    assert last.dual_violation.violations_found == int(cert[2])
    assert last.convergence.max_dual_violation == cert[3]
    assert max(float(row_max.max()), 0.0) == cert[3] == max(float(col_max.max()), 0.0)
    assert gap <= 1e-6
    # the plan is feasible only to the LP's 1e-6 residual, so its objective may sit that far below the optimum
    assert -1e-6 <= certified <= CERTIFIED_GAP


def test_c3_sddmm_and_pdhg_full_shape(cuda):
    """C3 (m = n = 262144, d = 256, 16 sorted random columns per row): SDDMM bit-exact against the oracle, then
    1000 PDHG iterations (uniform marginals, zero warm start) against the oracle's iterates at 1e-8."""
    m = n = 262144
    d, per = 256, 16
    rng = np.random.default_rng(3)
    X = rng.standard_normal((m, d)).astype(np.float32)
    Y = rng.standard_normal((n, d)).astype(np.float32)
    rowptr, col = random_csr(rng, m, n, per)
    p = (X.astype(np.float64) ** 2).sum(1)
    q = (Y.astype(np.float64) ** 2).sum(1)
    _say("C3: SDDMM")
    t = [torch.as_tensor(v).to(cuda) for v in (X, Y, p, q, rowptr, col)]
    costs = lowrank_csr_costs(*t)
    ref = oracle.sddmm_l2sq(X, Y, p, q, rowptr, col, 2.0)
    np.testing.assert_array_equal(costs.cpu().numpy(), ref)
    _say("C3: 1000 PDHG iterations")
    rows = np.repeat(np.arange(m), per)
    a = np.full(m, 1.0 / m)
    b = np.full(n, 1.0 / n)
    r = NativeRestrictedOTPDLP(device=cuda, evaluation_frequency=200, iteration_limit=1000).solve_restricted(
        rows=rows, cols=col, costs=costs, source_mass=a, target_mass=b, tolerance=0.0)
    want = oracle.pdhg_solve(rows, col, ref, a, b, evaluation_frequency=200, iteration_limit=1000, tolerance=0.0)
    assert r.iterations == want["iterations"] == 1000
    assert r.solver_diag["restart_count"] == want["restart_count"]
    np.testing.assert_allclose(r.x.cpu().numpy(), want["x"], rtol=1e-8, atol=1e-8 * np.abs(want["x"]).max())
    np.testing.assert_allclose(r.y.cpu().numpy(), want["y"], rtol=1e-8, atol=1e-9 * np.abs(want["y"]).max())
    assert r.obj_val == pytest.approx(want["obj_val"], rel=1e-9)
