"""End-to-end HELLO solves on the MI355X path against exact LP optima (GPU only).

The reference pins its solver end to end against POT's exact ``emd2`` (tests/cpp_backend_test.py:38-69,
tests/hello_gpu_resident_test.py:73-104: objective rel 5e-5 / 1e-5, marginals 3e-6 / 4e-6); POT is absent here, so
the exact optimum comes from scipy's HiGHS LP on the dense problem, and C1 is checked against its analytic
Brenier plan (examples/quickstart.py:83-94)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from hello_ot_amd import SolverOptions, solve

pytestmark = pytest.mark.gpu


def _cost_matrix(X, Y, kind):
    if kind == "l2^2":
        X64, Y64 = X.astype(np.float64), Y.astype(np.float64)
        return (X64 ** 2).sum(1)[:, None] + (Y64 ** 2).sum(1)[None, :] - 2.0 * X64 @ Y64.T
    code = {"l1": 0, "linf": 1, "l2": 2}[kind]
    _, cost = oracle.norm_matrices(X, Y, np.zeros(len(X)), np.zeros(len(Y)), code)
    return cost


def _exact(C, a, b):
    from scipy.optimize import linprog

    n, m = C.shape
    A = np.zeros((n + m, n * m))
    for i in range(n):
        A[i, i * m:(i + 1) * m] = 1.0
    for j in range(m):
        A[n + j, j::m] = 1.0
    res = linprog(C.reshape(-1), A_eq=A, b_eq=np.concatenate((a, b)), bounds=(0, None), method="highs")
    assert res.status == 0
    return res.fun


@pytest.mark.parametrize("kind,n,m,d,uniform", [
    ("l2^2", 240, 240, 5, True),
    ("l2^2", 130, 170, 300, False),   # d >= 256: fused-column pricing path
    ("l1", 200, 150, 4, False),
    ("linf", 160, 190, 3, False),
    ("l2", 150, 150, 6, True),
])
def test_solve_matches_exact_lp(cuda, kind, n, m, d, uniform):
    rng = np.random.default_rng(n + m + d)
    X = rng.random((n, d)).astype(np.float32)
    Y = (rng.random((m, d)) + 0.2).astype(np.float32)
    if uniform:
        a, b = np.full(n, 1.0 / n), np.full(m, 1.0 / m)
    else:
        a, b = rng.uniform(0.5, 1.5, n), rng.uniform(0.5, 1.5, m)
        a, b = a / a.sum(), b / b.sum()
    opts = SolverOptions(coarsest_size_threshold=40, verbose="off", cost_perturbation="off")
    r = solve(X, Y, source_mass=a, target_mass=b, cost=kind, options=opts)
    assert len(r.solve_stage.levels) >= 3
    assert all(l.solve.summary.converged for l in r.solve_stage.levels if l.kind == "refined")
    exact = _exact(_cost_matrix(X, Y, kind), a, b)
    print(f"[solve-vs-highs] {kind} {n}x{m} d={d} rel={abs(r.objective - exact) / abs(exact):.3e}", flush=True)
    # at the default 1e-6 KKT tolerance the objective lands within a few 1e-6 of the exact optimum
    assert abs(r.objective - exact) <= 5e-6 * abs(exact)
    coarsest, refined = r.solve_stage.levels[0], [l for l in r.solve_stage.levels if l.kind == "refined"]
    assert coarsest.kind == "coarsest" and r.metadata["coarsest_solver"] == "mi355x_network_simplex"
    k = opts.assignment_topk
    for level in refined:   # the reference's initialization record (gpu_resident/solver.py:60-63)
        init = level.initialization
        assert init.support_after_forward == level.n_source * min(level.n_target, k)
        assert init.initial_active_support_size == init.support_after_reverse + init.northwest_edges_added
        assert init.support_after_reverse <= level.n_source * k + level.n_target * k
    sol = r.solution.to_cpu()
    rows = np.bincount(sol.rows, weights=sol.values, minlength=n)
    cols = np.bincount(sol.cols, weights=sol.values, minlength=m)
    np.testing.assert_allclose(rows, a, atol=5e-6)
    np.testing.assert_allclose(cols, b, atol=5e-6)


@pytest.mark.parametrize("kind,n,m,d,tol", [("l2^2", 240, 200, 5, 5e-8), ("l1", 200, 150, 4, 1e-9)])
def test_tight_tolerance_solve_matches_the_exact_optimum_to_1e7(cuda, kind, n, m, d, tol):
    """At a tight KKT tolerance the objective is within 1e-7 of HiGHS's exact optimum. The l2^2 certificate is
    computed from fp32-grade dots (as the reference's, from fp32 SGEMM tiles), whose rounding on the support's
    near-zero scores bounds the tolerance it can certify from below (about 1e-8 here); the norm certificate is exact."""
    rng = np.random.default_rng(n * m + d)
    X = rng.random((n, d)).astype(np.float32)
    Y = (rng.random((m, d)) + 0.2).astype(np.float32)
    a, b = rng.uniform(0.5, 1.5, n), rng.uniform(0.5, 1.5, m)
    a, b = a / a.sum(), b / b.sum()
    opts = SolverOptions(coarsest_size_threshold=40, verbose="off", cost_perturbation="off", tolerance=tol)
    r = solve(X, Y, source_mass=a, target_mass=b, cost=kind, options=opts)
    exact = _exact(_cost_matrix(X, Y, kind), a, b)
    print(f"[solve-vs-highs tight] {kind} rel={abs(r.objective - exact) / abs(exact):.3e}", flush=True)
    assert abs(r.objective - exact) <= 1e-7 * abs(exact)


@pytest.mark.parametrize("precision", ["fp64", "finest_fp64"])
def test_fp64_cost_precision_runs_the_exact_l2sq_path(cuda, precision):
    """cost_precision='fp64' / 'finest_fp64' on l2^2: the path already ranks by fp64 scores and evaluates pair
    costs in fp64, so the solve lands on the same optimum as the default (HiGHS to 5e-6, the fp32 run to 1e-9) and
    records the option."""
    rng = np.random.default_rng(77)
    n, m, d = 200, 180, 6
    X = rng.random((n, d)).astype(np.float32)
    Y = (rng.random((m, d)) + 0.2).astype(np.float32)
    base = SolverOptions(coarsest_size_threshold=40, verbose="off", cost_perturbation="off")
    r32 = solve(X, Y, cost="l2^2", options=base)
    r64 = solve(X, Y, cost="l2^2", options=SolverOptions(coarsest_size_threshold=40, verbose="off",
                                                         cost_perturbation="off", cost_precision=precision))
    exact = _exact(_cost_matrix(X, Y, "l2^2"), np.full(n, 1.0 / n), np.full(m, 1.0 / m))
    assert r64.metadata["cost_precision"] == precision
    assert abs(r64.objective - exact) <= 5e-6 * abs(exact)
    assert r64.objective == pytest.approx(r32.objective, rel=1e-9)


def test_coarsest_only_problem_is_solved_exactly(cuda):
    """A problem that fits the coarsest threshold is one network-simplex solve: HiGHS's optimum to 1e-12 and a
    vertex (at most n + m - 1 positive flows)."""
    rng = np.random.default_rng(5)
    n, m = 90, 70
    X = rng.random((n, 3)).astype(np.float32)
    Y = rng.random((m, 3)).astype(np.float32)
    r = solve(X, Y, cost="l2^2", options=SolverOptions(verbose="off"))
    assert len(r.solve_stage.levels) == 1 and r.solve_stage.levels[0].kind == "coarsest"
    exact = _exact(_cost_matrix(X, Y, "l2^2"), np.full(n, 1.0 / n), np.full(m, 1.0 / m))
    assert abs(r.objective - exact) <= 1e-12 * abs(exact)
    sol = r.solution.to_cpu()
    assert (sol.values > 0).sum() <= n + m - 1


def test_brenier_c1_recovers_the_analytic_plan(cuda):
    """C1: x ~ N(0, I) (2048 x 32, seed 42), y = x + 2 tanh(x) rows permuted; the optimal plan is the permutation
    (examples/quickstart.py:83-94) and the objective is mean ||x - T(x)||^2."""
    n, dim, seed = 2048, 32, 42
    rng = np.random.default_rng(seed)
    source = rng.normal(size=(n, dim)).astype(np.float32)
    mapped = source + np.float32(2.0) * np.tanh(source)
    perm = rng.permutation(n)
    target = mapped[perm]
    disp = source.astype(np.float64) - mapped.astype(np.float64)
    truth = float(np.mean(np.sum(disp * disp, axis=1)))
    r = solve(source, target, options=SolverOptions(verbose="off"))
    assert abs(r.objective - truth) <= 1e-7 * truth
    sol = r.solution.to_cpu()
    inverse = np.argsort(perm)          # target index of source i's image
    big = sol.values > 0.5 / n
    assert big.sum() == n
    np.testing.assert_array_equal(sol.cols[big], inverse[sol.rows[big]])


def test_solve_with_the_smallest_support_budget_sparsifies(cuda):
    """beta = gamma + 2 (the smallest budget HELLO accepts) caps an LP's positive edges at m + n + 1, below what
    PDHG leaves on these supports: the refinement must sparsify by cycle cancelling
    (gpu_resident/support.py:124-137) and still reach the exact optimum."""
    n = m = 200
    rng = np.random.default_rng(11)
    X = rng.random((n, 4)).astype(np.float32)
    Y = rng.random((m, 4)).astype(np.float32)
    a, b = rng.uniform(0.5, 1.5, n), rng.uniform(0.5, 1.5, m)
    a, b = a / a.sum(), b / b.sum()
    opts = SolverOptions(coarsest_size_threshold=60, support_budget_factor=4.0, verbose="off",
                         cost_perturbation="off")
    r = solve(X, Y, source_mass=a, target_mass=b, cost="l1", options=opts)
    events = r.metadata["support_sparsification"]
    assert events["events"] >= 1 and events["removed_edges"] > 0
    assert all(l.solve.summary.converged for l in r.solve_stage.levels if l.kind == "refined")
    exact = _exact(_cost_matrix(X, Y, "l1"), a, b)
    assert abs(r.objective - exact) <= 2e-5 * abs(exact)
    sol = r.solution.to_cpu()
    np.testing.assert_allclose(np.bincount(sol.rows, weights=sol.values, minlength=n), a, atol=5e-6)
    np.testing.assert_allclose(np.bincount(sol.cols, weights=sol.values, minlength=m), b, atol=5e-6)


def test_consumed_inputs_come_back_in_the_callers_order(cuda, monkeypatch):
    """consume_input_features reorders device inputs in place for the solve and puts them back when it ends, also
    when it fails (the reference's in-place reorder, gpu_resident/storage.py:74-120, and its tests
    hello_gpu_resident_test.py:234-249); inputs sharing storage are refused."""
    import hello_ot_amd.api as api

    rng = np.random.default_rng(19)
    X = torch.as_tensor(rng.random((230, 5)).astype(np.float32)).to(cuda)
    Y = torch.as_tensor((rng.random((190, 5)) + 0.2).astype(np.float32)).to(cuda)
    Xc, Yc = X.clone(), Y.clone()
    opts = dict(coarsest_size_threshold=40, verbose="off", cost_perturbation="off")
    r = solve(X, Y, options=SolverOptions(consume_input_features=True, **opts))
    assert torch.equal(X, Xc) and torch.equal(Y, Yc)
    ref = solve(Xc, Yc, options=SolverOptions(**opts))
    assert r.objective == pytest.approx(ref.objective, rel=1e-12)
    assert torch.equal(r.solution.rows, ref.solution.rows) and torch.equal(r.solution.cols, ref.solution.cols)

    def fail(*args, **kwargs):
        raise RuntimeError("injected coarsest failure")

    monkeypatch.setattr(api, "solve_coarsest", fail)
    with pytest.raises(RuntimeError, match="injected coarsest failure"):
        solve(X, Y, options=SolverOptions(consume_input_features=True, **opts))
    assert torch.equal(X, Xc) and torch.equal(Y, Yc)
    with pytest.raises(ValueError, match="disjoint storage"):
        solve(X, X[:100], options=SolverOptions(consume_input_features=True, **opts))


def test_gpu_resident_input_validation(cuda):
    """hello_gpu_resident_test.py:267-276: the GPU-resident entry wants both sides as contiguous fp32 tensors on one
    device, with disjoint storage when consumed."""
    x = torch.randn(5, 3, device=cuda)
    options = SolverOptions(gpu_resident=True, consume_input_features=True, verbose="off")
    with pytest.raises(ValueError, match="disjoint storage"):
        solve(x, x, options=options)
    with pytest.raises(ValueError, match="contiguous FP32"):
        solve(x.double(), x.clone(), options=options)
    with pytest.raises(ValueError, match="same device"):
        solve(x, x.cpu(), options=options)
    with pytest.raises(ValueError, match="same device"):
        solve(x.cpu().numpy(), x.clone(), options=options)


@pytest.mark.parametrize("cost", ["l2^2", "l1", "l2", "linf"])
@pytest.mark.parametrize("precision", ["fp32", "fp64", "finest_fp64"])
def test_solution_contract_against_the_dense_lp(cuda, cost, precision):
    """The reference's end-to-end check of the GPU-resident solve (hello_gpu_resident_test.py:73-104, without the
    perturbed stage): consumed inputs unchanged afterwards, the plan on the device, marginals to 4e-6, the
    objective against the exact dense LP (abs 4e-5, rel 1e-5; HiGHS here, POT's emd2 there), one "original" cost
    stage, the returned duals' relative l2 violation over all pairs at most 1.1e-6, host export and warm start."""
    rng = np.random.default_rng(910)
    x = torch.tensor(rng.normal(size=(37, 7)), device=cuda, dtype=torch.float32)
    y = torch.tensor(rng.normal(size=(43, 7)), device=cuda, dtype=torch.float32)
    before_x, before_y = x.clone(), y.clone()
    a, b = rng.uniform(0.1, 2, 37), rng.uniform(0.1, 2, 43)
    a, b = a / a.sum(), b / b.sum()
    result = solve(x, y, source_mass=torch.tensor(a, device=cuda), target_mass=b, cost=cost,
                   options=SolverOptions(gpu_resident=True, consume_input_features=True, coarsest_size_threshold=8,
                                         assignment_topk=2, pricing_topk=2, support_budget_factor=4,
                                         cost_perturbation="off", cost_precision=precision, verbose="off"))
    assert torch.equal(x, before_x) and torch.equal(y, before_y)
    solution = result.solution
    assert all(getattr(solution, k).is_cuda for k in ("rows", "cols", "values", "source_dual", "target_dual"))
    dense = solution.to_sparse_matrix().to_dense()
    torch.testing.assert_close(dense.sum(1), torch.tensor(a, device=cuda), atol=4e-6, rtol=0)
    torch.testing.assert_close(dense.sum(0), torch.tensor(b, device=cuda), atol=4e-6, rtol=0)
    delta = x.double()[:, None] - y.double()[None]
    costs = {"l2^2": lambda: delta.square().sum(-1), "l1": lambda: delta.abs().sum(-1),
             "l2": lambda: delta.square().sum(-1).sqrt(), "linf": lambda: delta.abs().amax(-1)}[cost]()
    expected = _exact(costs.cpu().numpy(), a, b)
    assert result.objective == pytest.approx(expected, abs=4e-5, rel=1e-5)
    assert [stage.name for stage in result.cost_stages] == ["original"]
    assert result.perturbed_cost_stage is None and result.original_cost_stage is result.solve_stage
    violation = (solution.source_dual[:, None] + solution.target_dual[None] - costs).clamp_min(0)
    assert float(violation.norm() / (1 + costs.norm())) <= 1.1e-6
    assert isinstance(solution.to_cpu().values, np.ndarray)
    state = solution.to_warm_start_state()
    assert state.x_prev.is_cuda and state.dual_uv.numel() == 80 and (state.n_source, state.n_target) == (37, 43)


def test_finest_linf_stops_the_finest_level_on_the_linf_violation(cuda):
    """stopping_norm="finest_linf" (gpu_resident/solver.py:86-100): the finest level stops when the certificate's
    linf metric max sigma+ / (1 + max|c|) is at most the tolerance, the other levels on l2; l2^2 only."""
    rng = np.random.default_rng(31)
    n, m, d = 220, 190, 5
    X = rng.random((n, d)).astype(np.float32)
    Y = (rng.random((m, d)) + 0.2).astype(np.float32)
    opts = dict(coarsest_size_threshold=40, verbose="off", cost_perturbation="off")
    r = solve(X, Y, options=SolverOptions(stopping_norm="finest_linf", **opts))
    finest = r.solve_stage.levels[-1].solve
    last = finest.iterations[-1].convergence
    assert finest.summary.converged and last.norm == "linf"
    assert last.dual_feasibility == last.relative_linf_dual_feasibility <= 1e-6
    assert all(it.convergence.norm == "l2" for level in r.solve_stage.levels[1:-1] for it in level.solve.iterations)
    # the dense check of the returned duals in linf
    C = _cost_matrix(X, Y, "l2^2")
    f, g = r.solution.source_dual.cpu().numpy(), r.solution.target_dual.cpu().numpy()
    assert np.clip(f[:, None] + g[None, :] - C, 0, None).max() / (1.0 + np.abs(C).max()) <= 1.1e-6
    exact = _exact(C, np.full(n, 1.0 / n), np.full(m, 1.0 / m))
    assert abs(r.objective - exact) <= 5e-6 * abs(exact)
    with pytest.raises(ValueError, match="finest_linf currently requires l2"):
        solve(X, Y, cost="l1", options=SolverOptions(stopping_norm="finest_linf", **opts))
