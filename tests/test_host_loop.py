"""Host-side HELLO logic that needs no GPU: options, hierarchy, northwest basis, support bookkeeping."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from hello_ot_amd import Problem, SolverOptions
from hello_ot_amd.resident.solver import candidate_keys, derive_hierarchy_seeds, level_sizes, shuffle_once_permutation
from hello_ot_amd.resident.support import Support, normalize_masses, northwest


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


def test_problem_validation():
    with pytest.raises(ValueError, match="same feature dimension"):
        Problem(np.zeros((3, 2)), np.zeros((3, 3)), "l2^2")
    with pytest.raises(ValueError, match="cost_type must be one of"):
        Problem(np.zeros((3, 2)), np.zeros((3, 2)), "l3")
    with pytest.raises(ValueError, match="strictly positive"):
        Problem(np.zeros((3, 2)), np.zeros((3, 2)), "l1", source_mass=[1.0, 0.0, 1.0])
    p = Problem(np.ones((4, 2)), np.ones((5, 2)), " L2^2 ")
    assert p.shape == (4, 5) and p.cost_type == "l2^2" and p.source_points.dtype == np.float32


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
def test_northwest_basis_is_a_feasible_spanning_tree(n, m, seed):
    rng = np.random.default_rng(seed)
    a, b = normalize_masses(torch.as_tensor(rng.uniform(0.5, 1.5, n)), torch.as_tensor(rng.uniform(0.5, 1.5, m)))
    assert abs(float(a.sum() - b.sum())) <= 1e-15
    keys, flows = northwest(a, b)
    assert len(keys) == n + m - 1 and bool((flows >= 0).all())
    rows, cols = keys // m, keys % m
    # staircase: rows and cols never decrease and each step moves exactly one of them
    dr, dc = np.diff(rows.numpy()), np.diff(cols.numpy())
    assert ((dr + dc) == 1).all()
    np.testing.assert_allclose(torch.zeros(n, dtype=torch.float64).index_add_(0, rows, flows).numpy(), a.numpy(),
                               atol=1e-15)
    np.testing.assert_allclose(torch.zeros(m, dtype=torch.float64).index_add_(0, cols, flows).numpy(), b.numpy(),
                               atol=1e-15)


class _TableCost:
    def __init__(self, table):
        self.table = torch.as_tensor(table, dtype=torch.float64)

    def pairs(self, rows, cols):
        return self.table[rows, cols]


def test_support_extend_and_budgeted_pruning():
    n, m = 4, 5
    a = torch.full((n,), 0.25, dtype=torch.float64)
    b = torch.full((m,), 0.2, dtype=torch.float64)
    s = Support.initial(torch.tensor([3, 17], dtype=torch.int64), a, b)
    assert int(s.structural.sum()) == n + m - 1 and bool((torch.diff(s.keys) > 0).all())
    fresh = s.extend(torch.tensor([0, 19, 12, 6], dtype=torch.int64))
    assert set(s.keys[fresh].tolist()) == {19, 12, 6} - set(s.keys[~fresh].tolist())
    table = np.arange(n * m, dtype=np.float64).reshape(n, m)
    dual = torch.zeros(n + m, dtype=torch.float64)
    size = len(s.keys)
    # cost(r, c) = r * m + c = key and zero duals: the reduced cost of an edge is its key, so pruning one edge
    # removes the largest non-structural (zero-flow) key
    expected = int(s.keys[~s.structural].max())
    removed = s.prune(_TableCost(table), dual, torch.zeros(size, dtype=torch.bool), size - 1)
    assert removed.tolist() == [expected] and len(s.keys) == size - 1 and expected not in s.keys.tolist()
    with pytest.raises(RuntimeError, match="insufficient old zero-flow edges"):
        s.prune(_TableCost(table), dual, torch.zeros(len(s.keys), dtype=torch.bool), 1)


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
