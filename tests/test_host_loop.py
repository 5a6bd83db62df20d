"""Host-side HELLO logic that needs no GPU: options, hierarchy, northwest basis, support bookkeeping."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from hello_ot_amd import Problem, SolverOptions
from hello_ot_amd.resident.leaf import transport_simplex
from hello_ot_amd.resident.solver import candidate_keys, derive_hierarchy_seeds, level_sizes, shuffle_once_permutation
from hello_ot_amd.resident.support import ActiveSet, balanced_masses, staircase


def test_options_defaults_and_validation_match_the_reference():
    o = SolverOptions()
    assert (o.split_count, o.coarsest_size_threshold, o.assignment_topk, o.pricing_topk) == (4, 1024, 16, 2)
    assert (o.support_budget_factor, o.tolerance, o.backend, o.cost_perturbation) == (10.0, 1e-6, "native", "auto")
    with pytest.raises(ValueError, match="split_count must be one of: 2, 4, 8"):
        SolverOptions(split_count=3)
    with pytest.raises(ValueError, match="support_budget_factor >= pricing_topk"):
        SolverOptions(pricing_topk=9, support_budget_factor=10.0)
    with pytest.raises(ValueError, match="tolerance must be finite"):
        SolverOptions(tolerance=0.0)
    with pytest.raises(ValueError, match="verbose must be one of"):
        SolverOptions(verbose=True)
    with pytest.raises(NotImplementedError, match="backend='native'"):
        SolverOptions(backend="cpp").check_supported()
    with pytest.raises(NotImplementedError, match="cost_perturbation='on'"):
        SolverOptions(cost_perturbation="on").check_supported()
    for precision in ("fp32", "fp64", "finest_fp64"):   # the l2^2 path ranks by fp64 scores for all three
        SolverOptions(cost_precision=precision).check_supported()


def test_stopping_norm_per_level_follows_the_reference():
    """test_hello_ot_public_api.py:114-130: finest_linf stops the finest level on linf, every other level on l2."""
    from hello_ot_amd.config import finest_stopping_norm, level_stopping_norm

    assert SolverOptions().stopping_norm == "l2"
    assert SolverOptions(stopping_norm="finest_linf").stopping_norm == "finest_linf"
    for bad in ("linf", "other"):
        with pytest.raises(ValueError, match="stopping_norm"):
            SolverOptions(stopping_norm=bad)
    assert level_stopping_norm("l2", level_index=0) == "l2" and level_stopping_norm("l2", level_index=3) == "l2"
    assert level_stopping_norm("finest_linf", level_index=0) == "linf"
    assert level_stopping_norm("finest_linf", level_index=1) == "l2"
    assert finest_stopping_norm("finest_linf") == "linf"


def test_cost_precision_per_level_follows_the_reference():
    """config.py:23-28: fp64 everywhere, or only at the finest level (index 0) for finest_fp64."""
    from hello_ot_amd.config import level_precision

    assert [level_precision("fp32", i) for i in range(3)] == ["fp32"] * 3
    assert [level_precision("fp64", i) for i in range(3)] == ["fp64"] * 3
    assert [level_precision("finest_fp64", i) for i in range(3)] == ["fp64", "fp32", "fp32"]
    with pytest.raises(ValueError, match="cost_precision must be one of"):
        level_precision("fp16", 0)


def test_problem_validation():
    with pytest.raises(ValueError, match="same feature dimension"):
        Problem(np.zeros((3, 2)), np.zeros((3, 3)), "l2^2")
    with pytest.raises(ValueError, match="cost_type must be one of"):
        Problem(np.zeros((3, 2)), np.zeros((3, 2)), "l3")
    with pytest.raises(ValueError, match="strictly positive"):
        Problem(np.zeros((3, 2)), np.zeros((3, 2)), "l1", source_mass=[1.0, 0.0, 1.0])
    p = Problem(np.ones((4, 2)), np.ones((5, 2)), " L2^2 ")
    assert p.shape == (4, 5) and p.cost_type == "l2^2" and p.source_points.dtype == np.float32
    # test_hello_ot_public_api.py:35-62, 80-85: uniform masses by default; zero, negative, NaN and inf refused
    np.testing.assert_array_equal(p.source_mass, np.full(4, 0.25))
    np.testing.assert_array_equal(p.target_mass, np.full(5, 0.2))
    for mass in ([0.0, 1.0], [-0.1, 1.1], [np.nan, 1.0], [np.inf, 1.0]):
        with pytest.raises(ValueError, match="strictly positive"):
            Problem(np.zeros((2, 1)), np.zeros((2, 1)), "l2^2", source_mass=np.asarray(mass))
        with pytest.raises(ValueError, match="strictly positive"):
            Problem(np.zeros((2, 1)), np.zeros((2, 1)), "l2^2", target_mass=np.asarray(mass))
    with pytest.raises(ValueError, match="2D array"):
        Problem(np.zeros(3), np.zeros((3, 1)), "l2^2")
    with pytest.raises(ValueError, match="non-empty"):
        Problem(np.zeros((0, 2)), np.zeros((3, 2)), "l2^2")


def test_hierarchy_chain_and_global_shuffle():
    # the larger side shrinks by split_count until both fit the threshold (hierarchy/construction.py:111-138)
    assert level_sizes(2048, 2048, 1024, 4) == [(2048, 2048), (512, 2048), (512, 512)]
    assert level_sizes(10, 7, 1024, 4) == [(10, 7)]
    sizes = level_sizes(1_280_000, 1_280_000, 1024, 4)
    assert sizes[-1] == (313, 313) and len(sizes) == 13  # six divisions by 4 per side
    src, tgt, children = derive_hierarchy_seeds(42, 4)
    rng = np.random.default_rng(42)
    assert (src, tgt) == (int(rng.integers(0, 2**31 - 1)), int(rng.integers(0, 2**31 - 1))) and len(children) == 4
    ps, pt = shuffle_once_permutation(100, 80, 42, 4)
    assert np.array_equal(np.sort(ps), np.arange(100)) and np.array_equal(np.sort(pt), np.arange(80))
    ps2, _ = shuffle_once_permutation(100, 80, 42, 4)
    assert np.array_equal(ps, ps2)


@pytest.mark.parametrize("n,m,seed", [(5, 3, 0), (40, 55, 1), (1, 7, 2), (9, 1, 3)])
def test_staircase_basis_is_a_feasible_spanning_tree(n, m, seed):
    rng = np.random.default_rng(seed)
    a, b = balanced_masses(torch.as_tensor(rng.uniform(0.5, 1.5, n)), torch.as_tensor(rng.uniform(0.5, 1.5, m)))
    assert abs(float(a.sum() - b.sum())) <= 1e-15
    keys, flows = staircase(a, b)
    assert len(keys) == n + m - 1 and bool((flows >= 0).all())
    rows, cols = keys // m, keys % m
    # staircase: rows and cols never decrease and each step moves exactly one of them
    dr, dc = np.diff(rows.numpy()), np.diff(cols.numpy())
    assert ((dr + dc) == 1).all()
    np.testing.assert_allclose(torch.zeros(n, dtype=torch.float64).index_add_(0, rows, flows).numpy(), a.numpy(),
                               atol=1e-15)
    np.testing.assert_allclose(torch.zeros(m, dtype=torch.float64).index_add_(0, cols, flows).numpy(), b.numpy(),
                               atol=1e-15)


def _northwest_rule(a, b):
    """Textbook northwest-corner rule on exact (dyadic) masses: allocate min(residual supply, residual demand),
    then advance the row when its supply is used up -- first, when both are (the degenerate zero edge follows)."""
    i = j = 0
    ra, rb = a[0], b[0]
    edges = []
    while True:
        x = min(ra, rb)
        edges.append((i, j, x))
        ra -= x
        rb -= x
        if i == len(a) - 1 and j == len(b) - 1:
            return edges
        if ra == 0 and i < len(a) - 1:
            i += 1
            ra = a[i]
        else:
            j += 1
            rb = b[j]


@pytest.mark.parametrize("seed", range(6))
def test_staircase_matches_the_northwest_corner_rule_on_exact_masses(seed):
    # integer multiples of 2^-10: every cumulative sum is exact, so ties (degenerate edges) are genuine
    rng = np.random.default_rng(seed)
    n, m = rng.integers(1, 30, 2)
    a = rng.integers(1, 9, n).astype(np.float64)
    b = rng.integers(1, 9, m).astype(np.float64)
    b[-1] += a.sum() - b.sum()
    if b[-1] <= 0:
        a[-1] += 1 - b[-1]
        b[-1] = 1.0
    a, b = a / 1024.0, b / 1024.0
    keys, flows = staircase(torch.as_tensor(a), torch.as_tensor(b))
    want = _northwest_rule(list(a), list(b))
    assert (keys // m).tolist() == [e[0] for e in want]
    assert (keys % m).tolist() == [e[1] for e in want]
    assert flows.tolist() == [e[2] for e in want]


class _TableCost:
    def __init__(self, table):
        self.table = torch.as_tensor(table, dtype=torch.float64)

    def pairs(self, rows, cols):
        return self.table[rows, cols]


def test_active_set_absorb_and_trim():
    n, m = 4, 5
    a = torch.full((n,), 0.25, dtype=torch.float64)
    b = torch.full((m,), 0.2, dtype=torch.float64)
    s = ActiveSet.seeded(torch.tensor([3, 17], dtype=torch.int64), a, b)
    assert int(s.pinned.sum()) == n + m - 1 and bool((torch.diff(s.keys) > 0).all())
    assert float(s.flow.sum()) == pytest.approx(1.0)
    before = set(s.keys.tolist())
    new = s.absorb(torch.tensor([0, 6, 12, 19], dtype=torch.int64), born=0)
    assert set(new.tolist()) == {0, 6, 12, 19} - before
    assert bool((torch.diff(s.keys) > 0).all()) and set(s.keys.tolist()) == before | {0, 6, 12, 19}
    fresh = s.born == 0
    assert set(s.keys[fresh].tolist()) == set(new.tolist()) and float(s.flow[fresh].abs().sum()) == 0.0
    table = np.arange(n * m, dtype=np.float64).reshape(n, m)
    dual = torch.zeros(n + m, dtype=torch.float64)
    size = len(s)
    # cost(r, c) = key and zero duals: the reduced cost of an edge is its key, so trimming one edge removes the
    # largest key that is neither pinned nor added in this iteration
    expected = int(s.keys[(~s.pinned) & (~fresh)].max())
    removed = s.trim(_TableCost(table), dual, size - 1, iteration=0)
    assert removed.tolist() == [expected] and len(s) == size - 1 and expected not in s.keys.tolist()
    with pytest.raises(RuntimeError, match="insufficient old zero-flow edges"):
        s.trim(_TableCost(table), dual, 1, iteration=1)


@pytest.mark.parametrize("seed", range(5))
def test_trim_selects_as_a_stable_descending_sort(seed):
    """Pruning removes the `excess` largest reduced costs among the eligible edges, equal values in key order
    (refinement/budgeted_pruning.py:27-58: a stable descending argsort); many exact ties here."""
    rng = np.random.default_rng(seed)
    n, m = 30, 40
    keys = np.sort(rng.choice(n * m, 500, replace=False))
    flow = np.where(rng.random(500) < 0.2, rng.random(500), 0.0)
    pinned = rng.random(500) < 0.1
    born = np.where(rng.random(500) < 0.1, 3, -1).astype(np.int32)
    table = rng.integers(0, 12, (n, m)).astype(np.float64)        # few distinct values: ties everywhere
    dual = rng.integers(-2, 3, n + m).astype(np.float64)
    s = ActiveSet(torch.as_tensor(keys), torch.as_tensor(flow), torch.as_tensor(pinned), torch.as_tensor(born), n, m)
    budget = 420
    removed = s.trim(_TableCost(table), torch.as_tensor(dual), budget, iteration=3)
    rows, cols = keys // m, keys % m
    eligible = np.nonzero((~pinned) & (born < 3) & (np.abs(flow) <= 1e-15))[0]
    reduced = table[rows[eligible], cols[eligible]] - dual[rows[eligible]] - dual[n + cols[eligible]]
    order = np.argsort(-reduced, kind="stable")[: 500 - budget]
    assert removed.tolist() == sorted(keys[eligible[order]].tolist())
    assert len(s) == budget and not set(removed.tolist()) & set(s.keys.tolist())


def _highs(C, a, b):
    import scipy.sparse as sp
    from scipy.optimize import linprog

    n, m = C.shape
    rows, cols = np.repeat(np.arange(n), m), np.tile(np.arange(m), n)
    A = sp.vstack([sp.csr_matrix((np.ones(n * m), (rows, np.arange(n * m))), shape=(n, n * m)),
                   sp.csr_matrix((np.ones(n * m), (cols, np.arange(n * m))), shape=(m, n * m))])
    res = linprog(C.ravel(), A_eq=A, b_eq=np.concatenate((a, b)), bounds=(0, None), method="highs")
    assert res.status == 0
    return res.fun


@pytest.mark.parametrize("n,m,uniform,kind", [(1, 1, True, "r"), (1, 6, False, "r"), (7, 1, True, "r"),
                                              (12, 17, False, "r"), (60, 60, True, "l2"), (80, 130, False, "l1"),
                                              (150, 150, True, "grid")])
def test_transport_simplex_is_exact(n, m, uniform, kind):
    """The coarsest level's exact solver: HiGHS's optimum (1e-12), a feasible basic plan (at most n + m - 1 arcs,
    marginals to 1e-15), duals tight on the basis and feasible on every pair (strong duality to 1e-12). Uniform
    masses with n = m (an assignment problem, highly degenerate) and integer grid costs (massive ties) exercise the
    anti-cycling rule."""
    rng = np.random.default_rng(n * 1000 + m)
    if kind == "r":
        C = rng.random((n, m))
    elif kind == "grid":
        P, Q = rng.integers(0, 5, (n, 2)), rng.integers(0, 5, (m, 2))
        C = np.abs(P[:, None, :] - Q[None, :, :]).sum(-1).astype(np.float64)
    else:
        X, Y = rng.random((n, 3)), rng.random((m, 3))
        D = X[:, None, :] - Y[None, :, :]
        C = (D ** 2).sum(-1) if kind == "l2" else np.abs(D).sum(-1)
    if uniform:
        a, b = np.full(n, 1.0 / n), np.full(m, 1.0 / m)
    else:
        a, b = rng.uniform(0.5, 1.5, n), rng.uniform(0.5, 1.5, m)
        a, b = a / a.sum(), b / b.sum()
    r, c, x, u, v, _ = transport_simplex(C, a, b)
    assert len(x) <= n + m - 1 and (x >= 0).all()
    np.testing.assert_allclose(np.bincount(r, weights=x, minlength=n), a, rtol=0, atol=1e-15)
    np.testing.assert_allclose(np.bincount(c, weights=x, minlength=m), b, rtol=0, atol=1e-15)
    primal = float(C[r, c] @ x)
    scale = np.abs(C).max() + 1.0
    assert abs(primal - _highs(C, a, b)) <= 1e-12 * scale
    assert np.abs(C[r, c] - u[r] - v[c]).max() <= 1e-12 * scale
    assert (C - u[:, None] - v[None, :]).min() >= -1e-12 * scale
    assert abs(primal - (a @ u + b @ v)) <= 1e-12 * scale


def _assert_exact_vertex(C, a, b, r, c, x, u, v, optimum):
    n, m = C.shape
    scale = np.abs(C).max() + 1.0
    assert len(x) <= n + m - 1 and (x >= 0).all()
    np.testing.assert_allclose(np.bincount(r, weights=x, minlength=n), a, rtol=0, atol=1e-15)
    np.testing.assert_allclose(np.bincount(c, weights=x, minlength=m), b, rtol=0, atol=1e-15)
    primal = float(C[r, c] @ x)
    assert abs(primal - optimum) <= 1e-12 * scale
    assert np.abs(C[r, c] - u[r] - v[c]).max() <= 1e-12 * scale
    assert (C - u[:, None] - v[None, :]).min() >= -1e-12 * scale
    assert abs(primal - (a @ u + b @ v)) <= 1e-12 * scale


@pytest.mark.parametrize("kind", ["l2", "grid"])
def test_transport_simplex_at_the_default_coarsest_size(kind):
    """1024 x 1024 with uniform masses, the largest level the default coarsest_size_threshold hands to the simplex:
    an assignment problem, so its optimum is the Hungarian method's (scipy linear_sum_assignment) divided by n.
    Integer grid costs make almost every pivot degenerate (ties everywhere)."""
    from scipy.optimize import linear_sum_assignment

    n = 1024
    rng = np.random.default_rng(1024 if kind == "l2" else 2048)
    if kind == "l2":
        X, Y = rng.normal(size=(n, 8)), rng.normal(size=(n, 8))
        C = ((X[:, None, :] - Y[None, :, :]) ** 2).sum(-1)
    else:
        P, Q = rng.integers(0, 12, (n, 2)), rng.integers(0, 12, (n, 2))
        C = np.abs(P[:, None, :] - Q[None, :, :]).sum(-1).astype(np.float64)
    a = b = np.full(n, 1.0 / n)
    r, c, x, u, v, pivots = transport_simplex(C, a, b)
    ri, ci = linear_sum_assignment(C)
    _assert_exact_vertex(C, a, b, r, c, x, u, v, float(C[ri, ci].sum()) / n)
    assert pivots > n


def test_transport_simplex_with_zero_masses():
    """Points with zero mass (their rows / columns carry no flow, and their duals must still be feasible)."""
    rng = np.random.default_rng(17)
    n, m = 50, 64
    C = rng.random((n, m))
    a, b = rng.uniform(0.5, 1.5, n), rng.uniform(0.5, 1.5, m)
    a[rng.choice(n, 9, replace=False)] = 0.0
    b[rng.choice(m, 13, replace=False)] = 0.0
    a, b = a / a.sum(), b / b.sum()
    r, c, x, u, v, _ = transport_simplex(C, a, b)
    _assert_exact_vertex(C, a, b, r, c, x, u, v, _highs(C, a, b))
    assert np.all(x[a[r] == 0.0] == 0.0) and np.all(x[b[c] == 0.0] == 0.0)


def test_transport_simplex_rejects_bad_input():
    with pytest.raises(ValueError, match="unbalanced"):
        transport_simplex(np.ones((2, 2)), np.array([0.5, 0.5]), np.array([0.2, 0.2]))
    with pytest.raises(ValueError, match="finite"):
        transport_simplex(np.array([[1.0, np.nan]]), np.array([1.0]), np.array([0.5, 0.5]))
    with pytest.raises(ValueError, match="match"):
        transport_simplex(np.ones((2, 3)), np.array([1.0]), np.array([0.5, 0.5]))


def test_candidate_keys_filter_and_dedupe():
    dual = torch.tensor([0.5, -1.0, 0.0, 0.0, 0.0], dtype=torch.float64)  # n = 2, m = 3
    xv = torch.tensor([[-0.2, -0.7], [2.0, -3.0]], dtype=torch.float64)
    xi = torch.tensor([[1, 2], [0, -1]], dtype=torch.int32)
    yv = torch.tensor([[0.1], [-0.1], [-5.0]], dtype=torch.float64)
    yi = torch.tensor([[1], [0], [0]], dtype=torch.int32)
    all_keys = candidate_keys(xv, xi, yv, yi, dual, 2, 3)
    assert all_keys.tolist() == sorted({1, 2, 3, 3, 1, 2})
    pos = candidate_keys(xv, xi, yv, yi, dual, 2, 3, positive=True)
    # rows: 0.5-0.2 > 0 -> (0,1); 0.5-0.7 < 0; -1+2 > 0 -> (1,0); columns: 0+0.1 > 0 -> (1,0)
    assert pos.tolist() == [1, 3]


def test_primal_support_cap_reserves_basis_and_violations():
    from hello_ot_amd.config import active_support_budget, primal_support_cap

    # refinement/support_budget.py:56-67: budget - (V - 1) - gamma * V
    assert primal_support_cap(10.0, 2, 300, 500) == active_support_budget(10.0, 300, 500) - 799 - 1600
    assert primal_support_cap(4.0, 2, 200, 200) == 401


@pytest.mark.parametrize("n", [1, 2, 17, 1000])
@pytest.mark.parametrize("block", [1, 3, 64, 5000])
def test_inplace_row_permutation_walks_cycles(n, block):
    """The bounded in-place row permutation on the host: value[perm] for random permutations and their inverses,
    the identity, a reversal, a single n-cycle and adjacent swaps, with blocks shorter than, equal to and longer
    than the cycles (cycles crossing block boundaries read their saved first rows)."""
    from hello_ot_amd.resident.host import permute_rows_inplace

    g = torch.Generator().manual_seed(n * 131 + block)
    ar = torch.arange(n)
    rand = torch.randperm(n, generator=g)
    inverse = torch.empty_like(rand)
    inverse[rand] = ar
    swaps = ar.clone()
    swaps[: n - n % 2] = ar[: n - n % 2].view(-1, 2).flip(1).reshape(-1)
    for perm in (rand, inverse, ar, ar.flip(0), torch.roll(ar, 1), swaps):
        value = torch.randn((n, 3), generator=g)
        want = value[perm].clone()
        assert permute_rows_inplace(value, perm, block) is value
        assert torch.equal(value, want)


def test_streamed_rows_in_shuffle_order_without_a_copy():
    """HostRows with an order reads the caller's host rows in that order (prefixes too) and keeps no copy; the solve
    streams a contiguous fp32 host source this way and copies anything else once in shuffle order."""
    from hello_ot_amd.api import _streamed_side
    from hello_ot_amd.resident.host import HostRows

    g = torch.Generator().manual_seed(5)
    host = torch.randn((50, 4), generator=g)
    perm = torch.randperm(50, generator=g)
    rows = _streamed_side(host, perm, "cpu")
    assert rows.host is host and len(rows) == 50 and rows.shape == (50, 4)
    assert torch.equal(rows.to_device(), host[perm])
    assert torch.equal(rows.prefix(20).to_device(), host[perm[:20]])
    out = torch.empty((7, 4))
    rows._read(3, 10, out)
    assert torch.equal(out, host[perm[3:10]])
    as_numpy = _streamed_side(host.numpy(), perm, "cpu")
    assert as_numpy.host.data_ptr() == host.data_ptr()
    copied = _streamed_side(host.double(), perm, "cpu")
    assert copied.order is None and torch.equal(copied.host, host[perm])
    with pytest.raises(ValueError, match="vector"):
        HostRows(host, "cpu", order=perm.view(5, 10))


def test_column_list_merge_against_a_sort():
    """merge_columns on the CPU: the best k of two sorted lists per column, equal values taking the running list's
    entries first (their rows are the lower ones), -inf sentinels included, against a stable sort of the union."""
    from hello_ot_amd.resident.cost import merge_columns

    rng = np.random.default_rng(12)
    for _ in range(300):
        rows, k = int(rng.integers(1, 12)), int(rng.integers(1, 6))
        kb = int(rng.integers(1, k + 1))
        lists = []
        for width, base in ((k, 0), (kb, 1000)):
            v = rng.integers(0, 4, (rows, width)).astype(np.float64)
            v[rng.random((rows, width)) < 0.2] = -np.inf
            lists.append((-np.sort(-v, axis=1), base + np.tile(np.arange(width), (rows, 1))))
        (av, ai), (bv, bi) = lists
        gv, gi = merge_columns((torch.tensor(av), torch.tensor(ai)), (torch.tensor(bv), torch.tensor(bi)), k)
        for r in range(rows):
            union = [(-av[r, j], 0, j, ai[r, j], av[r, j]) for j in range(k)]
            union += [(-bv[r, j], 1, j, bi[r, j], bv[r, j]) for j in range(kb)]
            union.sort()
            assert gv[r].tolist() == [u[4] for u in union[:k]]
            assert gi[r].tolist() == [u[3] for u in union[:k]]
