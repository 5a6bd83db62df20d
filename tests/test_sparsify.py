"""Support sparsification (hm_sparsify_support, host code in the native library) against the reference's own
sparsifier compiled into oracle/_ref (support_sparsifier_lct.cpp) and the plain-Python restatement in the oracle:
identical cycle, exchange and output counts and zero patterns, flows to 1e-12. CPU only: the routine touches no
device memory."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from hello_ot_amd.resident.sparsify import sparsify_transport_support


def _support(seed, ns, nt, edges, zero_fraction=0.2):
    rng = np.random.default_rng(seed)
    key = np.unique(rng.integers(0, ns, edges) * nt + rng.integers(0, nt, edges))
    rows, cols = key // nt, key % nt
    values = rng.random(len(key))
    values[rng.random(len(key)) < zero_fraction] = 0.0
    costs = rng.random(len(key))
    return rows, cols, values, costs


def _sums(rows, cols, values, ns, nt):
    return np.bincount(rows, weights=values, minlength=ns), np.bincount(cols, weights=values, minlength=nt)


CASES = [(0, 40, 50, 700, 0), (1, 41, 50, 700, 10), (2, 30, 30, 400, 5), (3, 60, 20, 900, 0), (4, 5, 7, 35, 1)]


@pytest.mark.parametrize("seed,ns,nt,edges,extra", CASES)
def test_matches_the_reference_sparsifier(seed, ns, nt, edges, extra):
    ref = oracle.ref_sparsify()
    if ref is None:
        pytest.skip("reference sparsifier not built (make -C oracle ref needs /root/reference)")
    rows, cols, values, costs = _support(seed, ns, nt, edges)
    target = ns + nt - 1 + extra
    r = ref.sparsify_transport_support(ns, nt, rows, cols, values, costs, target, 1e-15)
    mine = sparsify_transport_support(rows, cols, values, costs, n_source=ns, n_target=nt, target_nnz=target)
    # the same cycles, choices and zero pattern; flows to rounding (the reference rounds sums of pending additions,
    # this implementation rounds each addition as it is made)
    np.testing.assert_array_equal(mine.values > 0, r["values"] > 0)
    np.testing.assert_allclose(mine.values, r["values"], rtol=1e-12, atol=1e-14)
    assert (mine.output_nnz, mine.cycle_updates, mine.tree_operations) == \
        (r["output_nnz"], r["cycle_updates"], r["tree_operations"])


@pytest.mark.parametrize("seed,ns,nt,edges,extra", CASES)
def test_matches_the_oracle_and_keeps_the_invariants(seed, ns, nt, edges, extra):
    rows, cols, values, costs = _support(seed, ns, nt, edges)
    target = ns + nt - 1 + extra
    mine = sparsify_transport_support(rows, cols, values, costs, n_source=ns, n_target=nt, target_nnz=target)
    ov, onnz, ocycles = oracle.sparsify_support(rows, cols, values, costs, ns, nt, target)
    np.testing.assert_allclose(mine.values, ov, rtol=0, atol=1e-12)
    assert (mine.output_nnz, mine.cycle_updates) == (onnz, ocycles)
    # invariants: marginals kept, cost not increased, flows >= 0, at most the target positive
    r0, c0 = _sums(rows, cols, values, ns, nt)
    r1, c1 = _sums(rows, cols, mine.values, ns, nt)
    np.testing.assert_allclose(r1, r0, atol=1e-12)
    np.testing.assert_allclose(c1, c0, atol=1e-12)
    assert costs @ mine.values <= costs @ values + 1e-12
    assert (mine.values >= 0).all() and mine.output_nnz <= target
    assert mine.output_nnz == np.count_nonzero(mine.values)


def test_oracle_restatement_matches_the_reference():
    ref = oracle.ref_sparsify()
    if ref is None:
        pytest.skip("reference sparsifier not built")
    for seed in range(6):
        rows, cols, values, costs = _support(100 + seed, 25, 35, 500)
        target = 25 + 35 - 1 + 3 * seed
        r = ref.sparsify_transport_support(25, 35, rows, cols, values, costs, target, 1e-15)
        ov, onnz, ocycles = oracle.sparsify_support(rows, cols, values, costs, 25, 35, target)
        np.testing.assert_allclose(ov, r["values"], rtol=0, atol=1e-12)
        assert (onnz, ocycles) == (r["output_nnz"], r["cycle_updates"])


def test_already_sparse_support_is_returned_unchanged():
    rows, cols, values, costs = _support(7, 20, 20, 150)
    out = sparsify_transport_support(rows, cols, values, costs, n_source=20, n_target=20, target_nnz=len(rows))
    np.testing.assert_array_equal(out.values, values)
    assert out.cycle_updates == 0 and out.output_nnz == np.count_nonzero(values)


def test_two_by_two_cycle_goes_the_cheaper_way():
    # flows 0.25 everywhere on a 2x2 support; the diagonal is cheaper, so the whole cycle moves onto it
    rows, cols = np.array([0, 0, 1, 1]), np.array([0, 1, 0, 1])
    values = np.full(4, 0.25)
    costs = np.array([0.0, 1.0, 1.0, 0.0])
    out = sparsify_transport_support(rows, cols, values, costs, n_source=2, n_target=2, target_nnz=3)
    np.testing.assert_allclose(out.values, [0.5, 0.0, 0.0, 0.5])
    assert out.output_nnz == 2 and out.cycle_updates == 1


def test_larger_support_runs_fast_and_keeps_the_invariants():
    ns, nt = 3000, 4000
    rows, cols, values, costs = _support(9, ns, nt, 60000, zero_fraction=0.0)
    target = ns + nt - 1 + 1000
    out = sparsify_transport_support(rows, cols, values, costs, n_source=ns, n_target=nt, target_nnz=target)
    assert out.output_nnz <= target and out.wall_time < 5.0
    r0, c0 = _sums(rows, cols, values, ns, nt)
    r1, c1 = _sums(rows, cols, out.values, ns, nt)
    np.testing.assert_allclose(r1, r0, atol=1e-11)
    np.testing.assert_allclose(c1, c0, atol=1e-11)
    assert costs @ out.values <= costs @ values + 1e-9


@pytest.mark.parametrize("kwargs,match", [
    (dict(n_source=0), "n_source and n_target must be positive"),
    (dict(target_nnz=2), "target_nnz must be at least"),
    (dict(values=np.array([-1.0, 0.5])), "values must be finite and nonnegative"),
    (dict(rows=np.array([0, 3])), "rows contain an out-of-range source index"),
])
def test_validation_messages(kwargs, match):
    args = dict(rows=np.array([0, 1]), cols=np.array([0, 1]), values=np.array([0.5, 0.5]),
                costs=np.array([1.0, 1.0]), n_source=2, n_target=2, target_nnz=3)
    args.update(kwargs)
    with pytest.raises(ValueError, match=match):
        sparsify_transport_support(args.pop("rows"), args.pop("cols"), args.pop("values"), args.pop("costs"), **args)


@pytest.mark.parametrize("seed", range(8))
def test_exact_ties_follow_path_order(seed):
    """Dyadic flows and integer costs: exact ties between candidate leaving edges everywhere. The leaving edge is the
    first tied edge along the path from the entering edge's source (the oracle's rule), which makes the result a
    function of the input alone; the reference's link-cut tree picks among exactly tied minima by its own splay
    history, so only this restatement is compared bit for bit here."""
    rng = np.random.default_rng(1000 + seed)
    ns, nt = rng.integers(5, 80, 2)
    key = np.unique(rng.integers(0, ns, 8 * (ns + nt)) * nt + rng.integers(0, nt, 8 * (ns + nt)))
    rows, cols = key // nt, key % nt
    values = rng.integers(0, 4, len(key)).astype(np.float64) / 8.0
    costs = rng.integers(0, 5, len(key)).astype(np.float64)
    target = int(ns + nt - 1 + rng.integers(0, 10))
    mine = sparsify_transport_support(rows, cols, values, costs, n_source=ns, n_target=nt, target_nnz=target)
    ov, onnz, ocycles = oracle.sparsify_support(rows, cols, values, costs, ns, nt, target)
    np.testing.assert_array_equal(mine.values, ov)
    assert (mine.output_nnz, mine.cycle_updates) == (onnz, ocycles)
    r0, c0 = _sums(rows, cols, values, ns, nt)
    r1, c1 = _sums(rows, cols, mine.values, ns, nt)
    np.testing.assert_array_equal(r1, r0)       # dyadic flows: every sum is exact
    np.testing.assert_array_equal(c1, c0)
    assert costs @ mine.values <= costs @ values and mine.output_nnz <= target
