"""Parity of the MI355X SDDMM and Halpern-PDHG kernels with the CPU oracle (GPU only)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from hello_ot_amd.costs.pairs import lowrank_csr_costs, lowrank_pair_costs, norm_pair_costs
from hello_ot_amd.lp import NativeRestrictedOTPDLP

pytestmark = pytest.mark.gpu


def _csr(rng, m, n, per_row):
    cols = [np.sort(rng.choice(n, per_row, replace=False)) for _ in range(m)]
    rowptr = np.concatenate([[0], np.cumsum([len(c) for c in cols])]).astype(np.int32)
    return rowptr, np.concatenate(cols).astype(np.int32)


@pytest.mark.parametrize("m,n,d,per_row", [(300, 400, 256, 16), (100, 90, 7, 5), (64, 64, 600, 3), (33, 50, 64, 50),
                                            (200, 300, 8192, 16), (64, 80, 8194, 5)])   # C5's d, and d + 2
def test_sddmm_csr_bit_exact(cuda, m, n, d, per_row):
    rng = np.random.default_rng(m + d)
    X = rng.standard_normal((m, d)).astype(np.float32)
    Y = rng.standard_normal((n, d)).astype(np.float32)
    p = (X.astype(np.float64) ** 2).sum(1)
    q = (Y.astype(np.float64) ** 2).sum(1)
    rowptr, col = _csr(rng, m, n, per_row)
    ref = oracle.sddmm_l2sq(X, Y, p, q, rowptr, col, 2.0)
    t = [torch.as_tensor(a).to(cuda) for a in (X, Y, p, q, rowptr, col)]
    out = lowrank_csr_costs(t[0], t[1], t[2], t[3], t[4], t[5], dot_scale=2.0)
    np.testing.assert_array_equal(out.cpu().numpy(), ref)


def test_sddmm_csr_empty_rows_and_validation(cuda):
    rng = np.random.default_rng(1)
    X = rng.standard_normal((6, 8)).astype(np.float32)
    Y = rng.standard_normal((5, 8)).astype(np.float32)
    p = (X.astype(np.float64) ** 2).sum(1)
    q = (Y.astype(np.float64) ** 2).sum(1)
    rowptr = np.array([0, 0, 2, 2, 3, 3, 3], np.int32)
    col = np.array([4, 1, 0], np.int32)
    ref = oracle.sddmm_l2sq(X, Y, p, q, rowptr, col, 2.0)
    t = [torch.as_tensor(a).to(cuda) for a in (X, Y, p, q, rowptr, col)]
    np.testing.assert_array_equal(lowrank_csr_costs(*t).cpu().numpy(), ref)
    bad = torch.as_tensor(np.array([4, 1, 5], np.int32)).to(cuda)
    with pytest.raises(ValueError, match="out of bounds"):
        lowrank_csr_costs(t[0], t[1], t[2], t[3], t[4], bad)


@pytest.mark.parametrize("d", [1, 8, 20, 64, 130, 8192])
def test_pair_costs_l2sq_and_norms_bit_exact(cuda, d):
    rng = np.random.default_rng(d)
    X = rng.random((40, d)).astype(np.float32)
    Y = rng.random((50, d)).astype(np.float32)
    p = (X.astype(np.float64) ** 2).sum(1)
    q = (Y.astype(np.float64) ** 2).sum(1)
    rows = rng.integers(0, 40, 777)
    cols = rng.integers(0, 50, 777)
    order = np.lexsort((cols, rows))
    rows_s, cols_s = rows[order], cols[order]
    rowptr = np.searchsorted(rows_s, np.arange(41)).astype(np.int32)
    ref = oracle.sddmm_l2sq(X, Y, p, q, rowptr, cols_s.astype(np.int32), 2.0)
    tX, tY, tp, tq = (torch.as_tensor(a).to(cuda) for a in (X, Y, p, q))
    out = lowrank_pair_costs(tX, tY, tp, tq, torch.as_tensor(rows_s).to(cuda), torch.as_tensor(cols_s).to(cuda))
    np.testing.assert_array_equal(out.cpu().numpy(), ref)
    for kind in (0, 1, 2):
        refn = oracle.pair_costs_norm(X, Y, rows, cols, kind)
        outn = norm_pair_costs(tX, tY, torch.as_tensor(rows).to(cuda), torch.as_tensor(cols).to(cuda), kind)
        np.testing.assert_array_equal(outn.cpu().numpy(), refn)


@pytest.mark.parametrize("d", [3, 8, 33, 100])
def test_norm_pair_costs_fp32_match_the_pricing_cost(cuda, d):
    """fp32 pair costs equal, bit for bit, the fp32 chunked cost the norm pricing scan ranks with (the oracle's
    cost matrix), so restricted LPs and pricing see the same c_ij."""
    rng = np.random.default_rng(100 + d)
    X = rng.random((30, d)).astype(np.float32)
    Y = rng.random((45, d)).astype(np.float32)
    rows = rng.integers(0, 30, 500)
    cols = rng.integers(0, 45, 500)
    tX, tY = torch.as_tensor(X).to(cuda), torch.as_tensor(Y).to(cuda)
    for kind in (0, 1, 2):
        _, cost = oracle.norm_matrices(X, Y, np.zeros(30), np.zeros(45), kind)
        out = norm_pair_costs(tX, tY, torch.as_tensor(rows).to(cuda), torch.as_tensor(cols).to(cuda), kind,
                              precision="fp32")
        np.testing.assert_array_equal(out.cpu().numpy(), cost[rows, cols])


def _small_problem():
    return dict(rows=np.array([0, 0, 1, 1]), cols=np.array([0, 1, 0, 1]), costs=np.array([0.0, 2.0, 1.0, 0.0]),
                source_mass=np.array([0.4, 0.6]), target_mass=np.array([0.5, 0.5]))


@pytest.mark.parametrize("warm", [False, True])
def test_pdhg_kat_small_problem(cuda, warm):
    # tests/torch_restricted_ot_pdlp_test.py:58-80
    kw = {}
    if warm:
        kw = dict(warm_start_primal=np.array([0.35, 0.05, 0.15, 0.45]), warm_start_dual=np.zeros(4))
    r = NativeRestrictedOTPDLP(device=cuda, evaluation_frequency=20, iteration_limit=200_000).solve_restricted(
        **_small_problem(), tolerance=1e-7, **kw)
    assert r.success, r.solver_diag
    assert r.x.dtype == torch.float64 and r.y.dtype == torch.float64
    assert r.obj_val == pytest.approx(0.1, abs=2e-6)
    assert r.primal_feas < 1e-7 and r.dual_feas < 1e-7 and r.gap < 1e-7


def test_pdhg_rejects_unbalanced_mass(cuda):
    problem = _small_problem()
    problem["target_mass"] = np.array([0.4, 0.5])
    with pytest.raises(ValueError, match="equal source and target total mass"):
        NativeRestrictedOTPDLP(device=cuda).solve_restricted(**problem)


def _sparse_lp(seed, ns, nt, extra):
    rng = np.random.default_rng(seed)
    rows = np.concatenate([np.arange(ns), rng.integers(0, ns, extra), rng.integers(0, ns, nt)])
    cols = np.concatenate([rng.integers(0, nt, ns), rng.integers(0, nt, extra), np.arange(nt)])
    perm = rng.permutation(rows.size)  # arbitrary edge order
    rows, cols = rows[perm], cols[perm]
    costs = rng.random(rows.size)
    a = rng.random(ns)
    a /= a.sum()
    b = rng.random(nt)
    b /= b.sum()
    return rows.astype(np.int64), cols.astype(np.int64), costs, a, b


@pytest.mark.parametrize("freq,limit,tol", [(5, 40, 0.0), (50, 3000, 1e-9), (200, 100000, 1e-7)])
def test_pdhg_matches_oracle_iterates(cuda, freq, limit, tol):
    rows, cols, costs, a, b = _sparse_lp(4, 60, 45, 400)
    ref = oracle.pdhg_solve(rows, cols, costs, a, b, evaluation_frequency=freq, iteration_limit=limit, tolerance=tol)
    r = NativeRestrictedOTPDLP(device=cuda, evaluation_frequency=freq, iteration_limit=limit).solve_restricted(
        rows=rows, cols=cols, costs=costs, source_mass=a, target_mass=b, tolerance=tol)
    assert r.iterations == ref["iterations"]
    assert r.termination_reason == ref["termination_reason"]
    assert r.solver_diag["restart_count"] == ref["restart_count"]
    np.testing.assert_allclose(r.x.cpu().numpy(), ref["x"], rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(r.y.cpu().numpy(), ref["y"], rtol=1e-9, atol=1e-12)
    assert r.obj_val == pytest.approx(ref["obj_val"], rel=1e-10)


def test_pdhg_warm_start_matches_oracle(cuda):
    rows, cols, costs, a, b = _sparse_lp(9, 30, 25, 120)
    rng = np.random.default_rng(0)
    x0 = rng.random(rows.size) * 0.01
    y0 = rng.normal(0, 0.1, a.size + b.size)
    ref = oracle.pdhg_solve(rows, cols, costs, a, b, warm_start_primal=x0, warm_start_dual=y0,
                            evaluation_frequency=50, iteration_limit=3000, tolerance=1e-9)
    r = NativeRestrictedOTPDLP(device=cuda, evaluation_frequency=50, iteration_limit=3000).solve_restricted(
        rows=rows, cols=cols, costs=costs, source_mass=a, target_mass=b, warm_start_primal=x0,
        warm_start_dual=y0, tolerance=1e-9)
    assert r.iterations == ref["iterations"]
    np.testing.assert_allclose(r.x.cpu().numpy(), ref["x"], rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(r.y.cpu().numpy(), ref["y"], rtol=1e-9, atol=1e-12)


def test_pdhg_node_blocks_with_hub_nodes_match_oracle(cuda):
    """Degrees far above the lane-group chunk on both sides, so both passes run as node blocks: source 0 reaches
    all 2600 targets (two 2048-edge rounds in its workgroup, its running sum carried across them), target 0 all
    40 sources, the other nodes a handful of edges."""
    ns, nt = 40, 2600
    rng = np.random.default_rng(21)
    rows = np.concatenate([np.zeros(nt, np.int64), np.arange(1, ns), rng.integers(1, ns, 200)])
    cols = np.concatenate([np.arange(nt), np.zeros(ns - 1, np.int64), rng.integers(1, nt, 200)])
    perm = rng.permutation(rows.size)
    rows, cols = rows[perm], cols[perm]
    costs = rng.random(rows.size)
    a = rng.random(ns)
    a /= a.sum()
    b = rng.random(nt)
    b /= b.sum()
    ref = oracle.pdhg_solve(rows, cols, costs, a, b, evaluation_frequency=50, iteration_limit=600, tolerance=0.0)
    r = NativeRestrictedOTPDLP(device=cuda, evaluation_frequency=50, iteration_limit=600).solve_restricted(
        rows=rows, cols=cols, costs=costs, source_mass=a, target_mass=b, tolerance=0.0)
    assert r.iterations == ref["iterations"] == 600
    assert r.solver_diag["restart_count"] == ref["restart_count"]
    np.testing.assert_allclose(r.x.cpu().numpy(), ref["x"], rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(r.y.cpu().numpy(), ref["y"], rtol=1e-9, atol=1e-12)


def test_pdhg_node_blocks_of_several_nodes_across_rounds_match_oracle(cuda):
    """Node blocks holding several nodes each (16384 sources: four per workgroup) whose edges exceed one 2048-edge
    round, so a node's edges straddle a round boundary and its running sum is carried across rounds inside a
    workgroup with other nodes: blocks of degrees (300, 900, 1400, 200) put the third node across the boundary,
    blocks of (10, 4500, 30, 5) stretch the second over three rounds; the other sources have 4 edges. The C5
    finest level runs this shape on its source side (256 nodes and about 3300 edges per workgroup)."""
    ns, nt = 16384, 5000
    rng = np.random.default_rng(33)
    degree = np.full(ns, 4)
    degree[: 32 * 4] = np.tile([300, 900, 1400, 200], 32)
    degree[32 * 4: 48 * 4] = np.tile([10, 4500, 30, 5], 16)
    rows = np.repeat(np.arange(ns), degree)
    cols = np.concatenate([rng.choice(nt, k, replace=False) for k in degree])
    missing = np.setdiff1d(np.arange(nt), cols)         # every target gets at least one edge
    rows = np.concatenate((rows, rng.integers(0, ns, missing.size)))
    cols = np.concatenate((cols, missing))
    perm = rng.permutation(rows.size)
    rows, cols = rows[perm].astype(np.int64), cols[perm].astype(np.int64)
    costs = rng.random(rows.size)
    a = rng.random(ns)
    a /= a.sum()
    b = rng.random(nt)
    b /= b.sum()
    ref = oracle.pdhg_solve(rows, cols, costs, a, b, evaluation_frequency=50, iteration_limit=400, tolerance=0.0)
    r = NativeRestrictedOTPDLP(device=cuda, evaluation_frequency=50, iteration_limit=400).solve_restricted(
        rows=rows, cols=cols, costs=costs, source_mass=a, target_mass=b, tolerance=0.0)
    assert r.iterations == ref["iterations"] == 400
    assert r.solver_diag["restart_count"] == ref["restart_count"]
    np.testing.assert_allclose(r.x.cpu().numpy(), ref["x"], rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(r.y.cpu().numpy(), ref["y"], rtol=1e-9, atol=1e-12)


def _nodes_per_block(nodes):
    """The node-block pass's nodes per workgroup: about 2048 workgroups, at most 256 nodes each."""
    npb = 1
    while npb < 256 and npb * 2 * 2048 <= nodes:
        npb *= 2
    return npb


def _gather_kinds(node, other, nodes):
    """How each node block of a side reads its edges' other-side node numbers: as 16-bit offsets from the smallest
    when they span fewer than 65536 nodes ("offsets"), else as 4-byte numbers ("numbers")."""
    npb = _nodes_per_block(nodes)
    blk = node // npb
    order = np.argsort(blk, kind="stable")
    blk, g = blk[order], other[order]
    starts = np.searchsorted(blk, np.arange((nodes + npb - 1) // npb + 1))
    kinds = []
    for b in range(starts.size - 1):
        e = g[starts[b]:starts[b + 1]]
        kinds.append("offsets" if e.size and e.max() - e.min() < 65536 else "numbers")
    return np.array(kinds)


def test_pdhg_node_blocks_with_16_bit_gather_offsets_match_oracle(cuda, monkeypatch):
    """131072 nodes a side, node blocks on both (hub nodes of degree 26-30 against a mean of 6.3), each source
    joined to the next 6 targets (wrapping round), and far edges 65536 nodes away from the blocks they start in (3
    from every eighth block, 80 from every eighth block shifted by two, each group landing in one or two blocks of
    the other side). Both ways of reading a block's gathered node numbers then run on both sides, each in at least
    100 blocks (checked on the host first): 16-bit offsets from the block's smallest, and 4-byte numbers."""
    ns = nt = 131072
    rng = np.random.default_rng(5)
    rs = [np.repeat(np.arange(ns), 6)]
    cs = [(np.repeat(np.arange(ns), 6) + np.tile(np.arange(6), ns)) % nt]
    hub_s, hub_t = np.arange(7, ns, 4096), np.arange(100, nt, 4096)
    rs.append(np.repeat(hub_s, 24))
    cs.append((np.repeat(hub_s, 24) + 6 + np.tile(np.arange(24), hub_s.size)) % nt)
    cs.append(np.repeat(hub_t, 20))
    rs.append((np.repeat(hub_t, 20) - 6 - np.tile(np.arange(20), hub_t.size)) % ns)
    for own_side, far_side, nodes, other_nodes in ((rs, cs, ns, nt), (cs, rs, nt, ns)):
        npb = _nodes_per_block(nodes)
        for blk in range(nodes // npb):
            if blk % 8 in (3, 5):
                cnt = 3 if blk % 8 == 3 else 80
                own_side.append(rng.integers(blk * npb, (blk + 1) * npb, cnt))
                far_side.append((blk * npb + 65536 + rng.integers(-32, 33, cnt)) % other_nodes)
    key = np.unique(np.concatenate(rs).astype(np.int64) * nt + np.concatenate(cs).astype(np.int64))
    perm = rng.permutation(key.size)
    rows, cols = key[perm] // nt, key[perm] % nt
    assert max(np.bincount(rows).max(), np.bincount(cols).max()) > 8 >= rows.size / ns   # node blocks, both sides
    for node, other, nodes in ((rows, cols, ns), (cols, rows, nt)):
        kinds = _gather_kinds(node, other, nodes)
        assert all(np.count_nonzero(kinds == kind) >= 100 for kind in ("offsets", "numbers"))
    costs = rng.random(rows.size)
    a, b = rng.random(ns), rng.random(nt)
    a, b = a / a.sum(), b / b.sum()
    monkeypatch.setenv("HELLOOT_PDHG_REORDER", "off")   # the caller's numbers, whose blocks are checked above
    ref = oracle.pdhg_solve(rows, cols, costs, a, b, evaluation_frequency=50, iteration_limit=300, tolerance=0.0)
    r = NativeRestrictedOTPDLP(device=cuda, evaluation_frequency=50, iteration_limit=300).solve_restricted(
        rows=rows, cols=cols, costs=costs, source_mass=a, target_mass=b, tolerance=0.0)
    assert r.iterations == ref["iterations"] == 300
    assert r.solver_diag["restart_count"] == ref["restart_count"]
    np.testing.assert_allclose(r.x.cpu().numpy(), ref["x"], rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(r.y.cpu().numpy(), ref["y"], rtol=1e-9, atol=1e-12)


def test_pdhg_c3_shape_1000_iterations_against_oracle(cuda):
    """C3 structure (16 sorted uniform columns per row, uniform marginals, SDDMM costs), 1000 iterations,
    at m = n = 8192 where the CPU oracle finishes in seconds."""
    m = n = 8192
    d = 256
    rng = np.random.default_rng(3)
    X = rng.standard_normal((m, d)).astype(np.float32)
    Y = rng.standard_normal((n, d)).astype(np.float32)
    rowptr, col = _csr(rng, m, n, 16)
    p = (X.astype(np.float64) ** 2).sum(1)
    q = (Y.astype(np.float64) ** 2).sum(1)
    costs = oracle.sddmm_l2sq(X, Y, p, q, rowptr, col, 2.0)
    rows = np.repeat(np.arange(m), 16)
    a = np.full(m, 1.0 / m)
    b = np.full(n, 1.0 / n)
    ref = oracle.pdhg_solve(rows, col, costs, a, b, evaluation_frequency=200, iteration_limit=1000, tolerance=0.0)
    r = NativeRestrictedOTPDLP(device=cuda, evaluation_frequency=200, iteration_limit=1000).solve_restricted(
        rows=rows, cols=col, costs=costs, source_mass=a, target_mass=b, tolerance=0.0)
    assert r.iterations == ref["iterations"] == 1000
    assert r.solver_diag["restart_count"] == ref["restart_count"]
    np.testing.assert_allclose(r.x.cpu().numpy(), ref["x"], rtol=1e-8, atol=1e-14)
    np.testing.assert_allclose(r.y.cpu().numpy(), ref["y"], rtol=1e-8, atol=1e-10)
    assert r.obj_val == pytest.approx(ref["obj_val"], rel=1e-9)


def _renumber_case(name):
    """LPs of the tests above, for the solve with internal node numbers."""
    rng = np.random.default_rng(0)
    if name == "sparse":
        rows, cols, costs, a, b = _sparse_lp(4, 60, 45, 400)
        return rows, cols, costs, a, b, 50, 3000, 1e-9, None, None
    if name == "warm":
        rows, cols, costs, a, b = _sparse_lp(9, 30, 25, 120)
        return rows, cols, costs, a, b, 50, 3000, 1e-9, rng.random(rows.size) * 0.01, rng.normal(0, 0.1, 55)
    if name == "hubs":
        ns, nt = 40, 2600
        rng = np.random.default_rng(21)
        rows = np.concatenate([np.zeros(nt, np.int64), np.arange(1, ns), rng.integers(1, ns, 200)])
        cols = np.concatenate([np.arange(nt), np.zeros(ns - 1, np.int64), rng.integers(1, nt, 200)])
        perm = rng.permutation(rows.size)
        a, b = rng.random(ns), rng.random(nt)
        return rows[perm], cols[perm], rng.random(rows.size), a / a.sum(), b / b.sum(), 50, 600, 0.0, None, None
    # clustered: 8 clusters of about 500 sources and 400 targets under shuffled numbers, each cluster's mass 1/8
    # and its support 6 random targets per source plus a north-west-corner staircase (so the LP is feasible), and
    # 200 edges across clusters
    ns, nt, k = 4000, 3200, 8
    cs, ct = rng.integers(0, k, ns), rng.integers(0, k, nt)
    a, b = rng.random(ns) + 0.1, rng.random(nt) + 0.1
    rows, cols = [], []
    for c in range(k):
        si, ti = np.flatnonzero(cs == c), np.flatnonzero(ct == c)
        a[si] /= a[si].sum() * k
        b[ti] /= b[ti].sum() * k
        rows.append(np.repeat(si, 6))
        cols.append(rng.choice(ti, 6 * si.size))
        u = v = 0
        left_a, left_b = a[si[0]], b[ti[0]]
        while u < si.size and v < ti.size:              # north-west corner rule on the cluster's masses
            rows.append(si[u:u + 1])
            cols.append(ti[v:v + 1])
            if left_a <= left_b:
                left_b -= left_a
                u += 1
                left_a = a[si[u]] if u < si.size else 0.0
            else:
                left_a -= left_b
                v += 1
                left_b = b[ti[v]] if v < ti.size else 0.0
    rows.append(rng.integers(0, ns, 200))
    cols.append(rng.integers(0, nt, 200))
    key = np.unique(np.concatenate(rows) * nt + np.concatenate(cols))
    return (key // nt).astype(np.int64), (key % nt).astype(np.int64), rng.random(key.size), a, b, 100, 3000, \
        1e-8, None, None


@pytest.mark.parametrize("name", ["sparse", "warm", "hubs", "clustered"])
def test_pdhg_with_internal_node_numbers_matches_oracle(cuda, monkeypatch, name):
    """The solve renumbers nodes by neighbour averaging when the problem has at least HELLOOT_PDHG_REORDER nodes
    (2^20 by default; 1 here forces it): per-node and per-edge operations are unchanged, so the iterates, counts,
    restarts and the caller-ordered outputs match the oracle as without the numbering."""
    rows, cols, costs, a, b, freq, limit, tol, x0, y0 = _renumber_case(name)
    ref = oracle.pdhg_solve(rows, cols, costs, a, b, warm_start_primal=x0, warm_start_dual=y0,
                            evaluation_frequency=freq, iteration_limit=limit, tolerance=tol)
    out = {}
    for setting in ("off", "1"):
        monkeypatch.setenv("HELLOOT_PDHG_REORDER", setting)
        r = NativeRestrictedOTPDLP(device=cuda, evaluation_frequency=freq, iteration_limit=limit).solve_restricted(
            rows=rows, cols=cols, costs=costs, source_mass=a, target_mass=b, warm_start_primal=x0,
            warm_start_dual=y0, tolerance=tol)
        assert r.iterations == ref["iterations"] and r.termination_reason == ref["termination_reason"], setting
        assert r.solver_diag["restart_count"] == ref["restart_count"], setting
        np.testing.assert_allclose(r.x.cpu().numpy(), ref["x"], rtol=1e-9, atol=1e-12)
        np.testing.assert_allclose(r.y.cpu().numpy(), ref["y"], rtol=1e-9, atol=1e-12)
        out[setting] = r
    assert out["1"].obj_val == pytest.approx(out["off"].obj_val, rel=1e-12)


def test_pdhg_internal_numbering_validates_endpoints(cuda, monkeypatch):
    """The library's own check (the Python wrapper validates first), on the numbering path."""
    from hello_ot_amd.lp.native_pdlp import run_pdhg

    monkeypatch.setenv("HELLOOT_PDHG_REORDER", "1")
    t = lambda v, dt: torch.as_tensor(np.asarray(v), dtype=dt, device=cuda)  # noqa: E731
    with pytest.raises(ValueError, match="out of bounds"):
        run_pdhg(t([0, 0, 1, 1], torch.int64), t([0, 1, 0, 2], torch.int64), t([0.0, 2.0, 1.0, 0.0], torch.float64),
                 t([0.4, 0.6], torch.float64), t([0.5, 0.5], torch.float64), None, None, evaluation_frequency=20,
                 rescale=False, iteration_limit=100, objective_tolerance=1e-6, primal_tolerance=1e-6,
                 dual_tolerance=1e-6, time_limit_seconds=60.0, device=cuda)
