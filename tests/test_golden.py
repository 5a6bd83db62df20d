"""The oracle against the golden vectors in tests/golden/: inputs and outputs of the reference's own CPU modules
(scan.cpp's dot_tile epilogue, solver.cpp's Halpern-PDHG, the link-cut-tree sparsifier, compiled from the
reference's sources by oracle/Makefile and run by tests/golden/make_golden.py). These pin the oracle, and the
host-side sparsifier of the native library, wherever the reference itself is absent (the GPU box included).
CPU only."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

import oracle
from hello_ot_amd.resident.sparsify import sparsify_transport_support

GOLDEN = Path(__file__).resolve().parent / "golden"


def _cases(prefix):
    return sorted(GOLDEN.glob(f"{prefix}_*.npz"), key=lambda p: p.name)


@pytest.mark.parametrize("path", _cases("scan_l2sq"), ids=lambda p: p.stem)
def test_l2sq_oracle_matches_reference_epilogue_vectors(path):
    z = np.load(path)
    X, Y, f, g, k = z["X"], z["Y"], z["f"], z["g"], int(z["k"])
    p = (X.astype(np.float64) ** 2).sum(1)
    q = (Y.astype(np.float64) ** 2).sum(1)
    rv, ri, cv, ci, st = oracle.l2sq_scan(X, Y, p, q, f - p, g - q, k, 2.0)
    np.testing.assert_array_equal(ri, z["row_indices"])
    np.testing.assert_array_equal(ci, z["col_indices"])
    # the reference scores (f + g) - ((p + q) - 2 dot), the oracle (2 dot + (f - p)) + (g - q): same pairs, values
    # to fp64 rounding
    np.testing.assert_allclose(rv, z["row_values"], rtol=1e-13, atol=1e-12)
    np.testing.assert_allclose(cv, z["col_values"], rtol=1e-13, atol=1e-12)
    np.testing.assert_allclose(st, z["stats"], rtol=1e-12)


@pytest.mark.parametrize("path", _cases("pdhg"), ids=lambda p: p.stem)
def test_pdhg_oracle_reproduces_reference_solver_vectors(path):
    z = np.load(path)
    tol = float(z["tolerance"])
    r = oracle.pdhg_solve(z["rows"], z["cols"], z["costs"], z["source_mass"], z["target_mass"],
                          evaluation_frequency=int(z["frequency"]), iteration_limit=int(z["limit"]), tolerance=tol,
                          rescale=bool(z["rescale"]) if "rescale" in z else False)
    assert r["iterations"] == int(z["iterations"])
    assert r["termination_reason"] == str(z["termination_reason"])
    assert r["restart_count"] == int(z["restart_count"])
    np.testing.assert_array_equal(r["x"], z["x"])
    np.testing.assert_array_equal(r["y"], z["y"])


@pytest.mark.parametrize("path", _cases("sparsify"), ids=lambda p: p.stem)
def test_sparsifiers_reproduce_reference_vectors(path):
    z = np.load(path)
    ns, nt, target = int(z["n_source"]), int(z["n_target"]), int(z["target_nnz"])
    assert int(z["output_nnz"]) < np.count_nonzero(z["values"])        # the case cancels cycles
    ov, onnz, ocycles = oracle.sparsify_support(z["rows"], z["cols"], z["values"], z["costs"], ns, nt, target)
    np.testing.assert_allclose(ov, z["out_values"], rtol=1e-12, atol=1e-14)
    assert (onnz, ocycles) == (int(z["output_nnz"]), int(z["cycle_updates"]))
    mine = sparsify_transport_support(z["rows"], z["cols"], z["values"], z["costs"], n_source=ns, n_target=nt,
                                      target_nnz=target)
    np.testing.assert_array_equal(mine.values > 0, z["out_values"] > 0)
    np.testing.assert_allclose(mine.values, z["out_values"], rtol=1e-12, atol=1e-14)
    assert (mine.output_nnz, mine.cycle_updates, mine.tree_operations) == \
        (int(z["output_nnz"]), int(z["cycle_updates"]), int(z["tree_operations"]))
