"""The streamed source side (pinned host rows read in chunks) against both sides on the device (GPU only).

The streamed scans price each source chunk against the device-resident target side and merge the column lists
across chunks (kernels/bilinear_topk.py:255-368 is the reference's split). Small chunk sizes force many chunks, a
ragged last one, and duplicated rows in different chunks (the column merge must keep the lowest row index among
equal values). Lists must be identical to the one-call scan, the certificate's count and maximum identical and its
sums fp32-grade equal (they gather fp32 partials per tile); pair costs bit-identical; a full solve lands on the same
objective.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from hello_ot_amd import SolverOptions, solve
from hello_ot_amd.resident import host as host_module
from hello_ot_amd.resident.cost import Cost, merge_columns
from hello_ot_amd.resident.host import HostRows

pytestmark = pytest.mark.gpu


def _streamed(cost: Cost, chunk: int) -> Cost:
    return Cost(HostRows(cost.source.cpu().contiguous(), cost.target.device, chunk), cost.target, cost.kind,
                cost.source_offset, cost.target_offset, cost.precision)


def _data(dev, n, m, d, seed, integer=False):
    rng = np.random.default_rng(seed)
    if integer:
        X = rng.integers(-3, 4, (n, d)).astype(np.float32)
        Y = rng.integers(-3, 4, (m, d)).astype(np.float32)
        X[n - 5:] = X[:5]                    # duplicates of the first chunk's rows in the last chunk
    else:
        X = rng.standard_normal((n, d)).astype(np.float32)
        Y = rng.standard_normal((m, d)).astype(np.float32)
    return rng, torch.as_tensor(X).to(dev), torch.as_tensor(Y).to(dev)


@pytest.mark.parametrize("kind,d,integer", [("l2^2", 300, False), ("l2^2", 300, True), ("l2^2", 40, True),
                                            ("l1", 8, True), ("linf", 5, False)])
def test_streamed_scans_equal_the_resident_scans(cuda, kind, d, integer):
    n, m = 2300, 1700
    rng, X, Y = _data(cuda, n, m, d, seed=d + (1 if integer else 0), integer=integer)
    resident = Cost.create(X, Y, kind)
    streamed = _streamed(resident, chunk=700)
    if kind == "l2^2":
        scale = float(resident.source_offset.mean())
        dual = torch.as_tensor(rng.normal(scale, 0.05 * scale, n + m)).to(cuda)
    else:
        dual = torch.as_tensor(rng.normal(0.5 * d, 0.1 * d, n + m)).to(cuda)
    if integer:
        dual = dual.round()
    for direction, k in ((None, 2), ("source", 16), ("target", 16), (None, 8)):
        cert = direction is None
        a = resident.scan(dual, k, certificate=cert, direction=direction)
        b = streamed.scan(dual, k, certificate=cert, direction=direction)
        for u, v in zip(a[:4], b[:4]):
            if u is not None:
                assert torch.equal(u, v), (direction, k)
        if cert:
            # the sums gather fp32 partials per tile, and the chunks change the tiles: fp32-grade agreement
            assert a[4]["count"] == b[4]["count"] and a[4]["max"] == b[4]["max"]
            assert a[4]["l2"] == pytest.approx(b[4]["l2"], rel=1e-6)
            assert a[4]["linf"] == pytest.approx(b[4]["linf"], rel=1e-6)
    rows = torch.as_tensor(rng.integers(0, n, 5000)).to(cuda)         # unsorted, with repeats
    cols = torch.as_tensor(rng.integers(0, m, 5000)).to(cuda)
    assert torch.equal(resident.pairs(rows, cols), streamed.pairs(rows, cols))


@pytest.mark.parametrize("kind", ["random", "reversal", "rotation", "swaps"])
def test_bounded_inplace_row_permutation(cuda, monkeypatch, kind):
    """permute_rows_inplace gives value[perm] in place on the device, walking the cycles in blocks of 300 positions
    (ragged last block; cycles crossing block boundaries, one cycle of all rows, 500 two-cycles)."""
    from hello_ot_amd.resident.host import permute_rows_inplace

    monkeypatch.setattr(host_module, "STREAM_CHUNK_BYTES", 300 * 17 * 4)
    rng = np.random.default_rng(3)
    value = torch.as_tensor(rng.standard_normal((1000, 17)).astype(np.float32)).to(cuda)
    perm = {"random": rng.permutation(1000), "reversal": np.arange(1000)[::-1].copy(),
            "rotation": np.roll(np.arange(1000), 1), "swaps": np.arange(1000).reshape(500, 2)[:, ::-1].ravel()}[kind]
    perm = torch.as_tensor(perm).to(cuda)
    want = value[perm].clone()
    assert permute_rows_inplace(value, perm) is value
    assert torch.equal(value, want)


def test_column_merge_keeps_the_lowest_index_among_equal_values(cuda):
    inf = float("inf")
    best = (torch.tensor([[3.0, 1.0], [2.0, -inf]], device=cuda), torch.tensor([[4, 9], [7, -1]], device=cuda))
    new = (torch.tensor([[3.0, 1.0], [5.0, 2.0]], device=cuda), torch.tensor([[12, 10], [20, 30]], device=cuda))
    v, i = merge_columns(best, new, 2)
    assert v.tolist() == [[3.0, 3.0], [5.0, 2.0]] and i.tolist() == [[4, 12], [20, 7]]


def test_streamed_solve_matches_the_resident_solve(cuda, monkeypatch):
    """Every level above the coarsest streams its source side in 500-row chunks (the coarsest level's prefix is
    copied to the device): same objective, support and duals as the solve with both sides on the device."""
    rng = np.random.default_rng(8)
    n, m, d = 3000, 2600, 300
    X = rng.standard_normal((n, d)).astype(np.float32)
    Y = (rng.standard_normal((m, d)) + 0.3).astype(np.float32)
    base = dict(coarsest_size_threshold=200, verbose="off", cost_perturbation="off")
    ref = solve(torch.as_tensor(X).to(cuda), torch.as_tensor(Y).to(cuda), options=SolverOptions(gpu_resident=True,
                                                                                                   **base))
    monkeypatch.setattr(host_module, "STREAM_MIN_BYTES", 200 * d * 4)
    monkeypatch.setattr(host_module, "STREAM_CHUNK_BYTES", 500 * d * 4)
    monkeypatch.setattr(host_module, "STREAM_POLICY", "always")
    monkeypatch.delenv("HELLOOT_STREAM_SOURCE", raising=False)
    # device inputs, consumed: the source side is copied to host memory in shuffle order, the target side is
    # reordered in place through the bounded permutation and put back afterwards
    Xd, Yd = torch.as_tensor(X).to(cuda), torch.as_tensor(Y).to(cuda)
    r = solve(Xd, Yd, options=SolverOptions(consume_input_features=True, **base))
    assert torch.equal(Xd.cpu(), torch.as_tensor(X)) and torch.equal(Yd.cpu(), torch.as_tensor(Y))
    assert r.metadata["streamed_source"] and not ref.metadata["streamed_source"]
    assert r.objective == pytest.approx(ref.objective, rel=1e-12)
    assert r.solution.values.numel() == ref.solution.values.numel()
    assert torch.equal(r.solution.rows, ref.solution.rows) and torch.equal(r.solution.cols, ref.solution.cols)
    np.testing.assert_allclose(r.solution.source_dual.cpu().numpy(), ref.solution.source_dual.cpu().numpy(),
                               rtol=1e-9, atol=1e-9)
