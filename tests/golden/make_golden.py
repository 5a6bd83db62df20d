"""Writes the golden vectors under tests/golden/ from the reference's own CPU modules.

The modules are the reference's C++ sources compiled by oracle/Makefile into oracle/_ref (scan.cpp's dot_tile
epilogue, solver.cpp's Halpern-PDHG, the link-cut-tree sparsifier); nothing of the reference is copied. Each
fixture holds the inputs and the reference's outputs, so that tests/test_golden.py pins the oracle where the
reference is not present. Run from the repository root after `make -C oracle ref`:

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402

SCAN_CASES = [(40, 57, 16, 1), (33, 70, 9, 3), (64, 48, 130, 8)]
PDHG_CASES = [(5, 40, 0.0), (20, 3000, 1e-7)]
# scalar-rescaling mode (solve_once's rescale flag): costs in the hundreds and skewed masses; masses of 1e100 (only
# the rescaled solve converges); one huge cost that makes the first residual non-finite (NUMERICAL_DIVERGENCE)
PDHG_RESCALE_CASES = [("skewed", 10, 4000, 1e-8), ("heavy", 20, 2000, 1e-7), ("diverge", 20, 100, 1e-7)]
SPARSIFY_CASES = [(0, 12, 15, 120, 0), (1, 20, 9, 150, 4)]


def scan_cases(sc):
    for m, n, d, k in SCAN_CASES:
        rng = np.random.default_rng(1000 + m * 7 + n)
        X = rng.standard_normal((m, d)).astype(np.float32)
        Y = rng.standard_normal((n, d)).astype(np.float32)
        p = (X.astype(np.float64) ** 2).sum(1)
        q = (Y.astype(np.float64) ** 2).sum(1)
        f, g = rng.normal(d, 2, m), rng.normal(d, 2, n)
        dots, _ = oracle.l2sq_matrices(X, Y, np.zeros(m), np.zeros(n), np.zeros(m), np.zeros(n), 1.0)
        rv, ri = np.full((m, k), -np.inf), np.full((m, k), -1, np.int64)
        cv, ci = np.full((n, k), -np.inf), np.full((n, k), -1, np.int64)
        stats = sc.dot_tile(np.ascontiguousarray(dots), p, q, f, g, rv, ri, cv, ci, 2.0, 0, 0, 0, 1)
        np.savez(HERE / f"scan_l2sq_{m}x{n}_d{d}_k{k}.npz", X=X, Y=Y, f=f, g=g, k=k, row_values=rv, row_indices=ri,
                 col_values=cv, col_indices=ci, stats=np.array([stats[i] for i in range(5)], np.float64))


def pdhg_cases(lp):
    rng = np.random.default_rng(12)
    rows, cols = np.indices((7, 5))
    rows, cols = rows.ravel().astype(np.int64), cols.ravel().astype(np.int64)
    costs = rng.random(35)
    sm, tm = np.full(7, 1 / 7), np.full(5, 1 / 5)
    for freq, limit, tol in PDHG_CASES:
        r = lp.solve_once(rows, cols, costs, np.concatenate([sm, tm]), np.zeros(35), np.zeros(12), 7, 1, freq,
                          3600.0, limit, tol, tol, tol, False, False)
        np.savez(HERE / f"pdhg_7x5_freq{freq}_limit{limit}.npz", rows=rows, cols=cols, costs=costs, source_mass=sm,
                 target_mass=tm, frequency=freq, limit=limit, tolerance=tol, x=r["x"], y=r["y"],
                 iterations=r["iterations"], termination_reason=r["termination_reason"],
                 restart_count=r["solver_diag"]["restart_count"])
    for name, freq, limit, tol in PDHG_RESCALE_CASES:
        rng = np.random.default_rng(77)
        costs = 250.0 * rng.random(35)
        sm = rng.random(7) + 0.2
        tm = rng.random(5) + 0.2
        sm, tm = sm / sm.sum(), tm / tm.sum()
        if name == "heavy":
            sm, tm = sm * 1e100, tm * 1e100
        if name == "diverge":
            costs[3] = 1e200
        for rescale in (False, True):
            r = lp.solve_once(rows, cols, costs, np.concatenate([sm, tm]), np.zeros(35), np.zeros(12), 7, 1, freq,
                              3600.0, limit, tol, tol, tol, rescale, False)
            np.savez(HERE / f"pdhg_7x5_{name}_rescale{int(rescale)}.npz", rows=rows, cols=cols, costs=costs,
                     source_mass=sm, target_mass=tm, frequency=freq, limit=limit, tolerance=tol, rescale=rescale,
                     x=r["x"], y=r["y"], iterations=r["iterations"], termination_reason=r["termination_reason"],
                     restart_count=r["solver_diag"]["restart_count"])


def sparsify_cases(sp):
    for seed, ns, nt, edges, extra in SPARSIFY_CASES:
        rng = np.random.default_rng(seed)
        key = np.unique(rng.integers(0, ns, edges) * nt + rng.integers(0, nt, edges))
        rows, cols = key // nt, key % nt
        values = rng.random(len(key))
        values[rng.random(len(key)) < 0.2] = 0.0
        costs = rng.random(len(key))
        target = ns + nt - 1 + extra
        r = sp.sparsify_transport_support(ns, nt, rows, cols, values, costs, target, 1e-15)
        np.savez(HERE / f"sparsify_{ns}x{nt}_target{target}.npz", rows=rows, cols=cols, values=values, costs=costs,
                 n_source=ns, n_target=nt, target_nnz=target, out_values=r["values"], output_nnz=r["output_nnz"],
                 cycle_updates=r["cycle_updates"], tree_operations=r["tree_operations"])


def main():
    sc, lp, sp = oracle.ref_scan(), oracle.ref_lp(), oracle.ref_sparsify()
    if sc is None or lp is None or sp is None:
        raise SystemExit("oracle/_ref is not built (make -C oracle ref needs the reference sources)")
    scan_cases(sc)
    pdhg_cases(lp)
    sparsify_cases(sp)


if __name__ == "__main__":
    main()
