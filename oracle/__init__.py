"""CPU oracle for the HELLO hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import this
package, and only as the checker (or the timed CPU baseline); the product path never touches it.

``liborc.so`` (built from ``oracle.c`` by ``oracle/Makefile``) is a plain-C restatement of:

* the pricing-scan score/cost/top-k/certificate semantics
  (``_native/generic_scan/pricing.cu:38-51,112-123``, ``matrix_selection.cuh:20-26``,
  ``_native/cpp/scan.cpp:15-26,185-196``),
* SDDMM on the active support (``costs/pairs.py:394-407``, ``gpu_resident/cost.py:59-71``),
* sparse norm pair costs (``_native/norm_cost_scan/norm_cost_scan_kernel.cu:233-245``),
* the Halpern-PDHG restricted-OT LP (``_native/cpp/solver.cpp:39-378``).

``sparsify_support`` restates the support sparsifier (``support_sparsifier_lct.cpp:378-555``) in plain Python.

``oracle/_ref/`` optionally holds the reference's own CPU modules (``_scan``, ``_lp``, ``_sparsify``) compiled from
``/root/reference`` by ``make -C oracle ref``; they pin the restatement where they build.

Parity status per function (how each is pinned) is listed in ``parity_pins()``.
"""
from __future__ import annotations

import ctypes
import importlib.util
import os
import subprocess
import sys
from pathlib import Path

import numpy as np

_DIR = Path(__file__).resolve().parent
_LIB = None

_REASONS = {0: "UNSPECIFIED", 1: "OPTIMAL", 2: "ITERATION_LIMIT", 3: "NUMERICAL_DIVERGENCE"}


class _PdhgInfo(ctypes.Structure):
    _fields_ = [
        ("iterations", ctypes.c_int64), ("restarts", ctypes.c_int64), ("reason", ctypes.c_int32),
        ("pad", ctypes.c_int32), ("pobj", ctypes.c_double), ("dobj", ctypes.c_double),
        ("ap", ctypes.c_double), ("rp", ctypes.c_double), ("ad", ctypes.c_double),
        ("rd", ctypes.c_double), ("gap", ctypes.c_double), ("weight", ctypes.c_double),
    ]


def build(quiet: bool = True) -> None:
    """Compile liborc.so (and the reference CPU modules when /root/reference is present)."""
    targets = ["oracle"]
    if Path("/root/reference/src/hello_ot/_native/cpp/scan.cpp").exists():
        targets.append("ref")
    subprocess.run(["make", "-s", "-C", str(_DIR), *targets], check=True,
                   stdout=subprocess.DEVNULL if quiet else None)


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        path = _DIR / "liborc.so"
        if not path.exists():
            build()
        _LIB = ctypes.CDLL(str(path))
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        D = ctypes.c_double
        _LIB.orc_dot64.restype = D
        _LIB.orc_dot64.argtypes = [P, P, I64]
        _LIB.orc_l2sq_matrices.argtypes = [P, P, P, P, P, P, I64, I64, I64, D, P, P]
        _LIB.orc_norm_matrices.argtypes = [P, P, P, P, I64, I64, I64, ctypes.c_int, P, P]
        _LIB.orc_norm_matrices64.argtypes = [P, P, P, P, I64, I64, I64, ctypes.c_int, P, P]
        _LIB.orc_topk.argtypes = [P, I64, I64, ctypes.c_int, ctypes.c_int, P, P]
        _LIB.orc_stats.argtypes = [P, P, I64, I64, P]
        _LIB.orc_sddmm_l2sq.argtypes = [P, P, P, P, P, P, I64, I64, D, P]
        _LIB.orc_pair_costs_norm.argtypes = [P, P, P, P, I64, I64, ctypes.c_int, P]
        _LIB.orc_pdhg_solve.restype = ctypes.c_int
        _LIB.orc_pdhg_solve.argtypes = [P, P, P, P, I64, I64, I64, P, P, ctypes.c_int, I64, D, D, D,
                                        ctypes.c_int, P, P, ctypes.POINTER(_PdhgInfo)]
    return _LIB


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _f64(a):
    return np.ascontiguousarray(a, dtype=np.float64)


def _ptr(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data)


def dot64(x, y) -> float:
    x, y = _f32(x).ravel(), _f32(y).ravel()
    return float(lib().orc_dot64(_ptr(x), _ptr(y), x.size))


def l2sq_matrices(X, Y, p, q, qb, db, scale=2.0):
    X, Y, p, q, qb, db = _f32(X), _f32(Y), _f64(p), _f64(q), _f64(qb), _f64(db)
    m, d = X.shape
    n = Y.shape[0]
    sigma = np.empty((m, n), np.float64)
    cost = np.empty((m, n), np.float64)
    lib().orc_l2sq_matrices(_ptr(X), _ptr(Y), _ptr(p), _ptr(q), _ptr(qb), _ptr(db), m, n, d,
                            float(scale), _ptr(sigma), _ptr(cost))
    return sigma, cost


def norm_matrices(X, Y, f, g, kind: int, precision: int = 0):
    """Norm score / cost matrices: fp32 costs (precision 0, the chunked sums) or fp64 costs (precision 1, the
    reference's compute_precision = 1)."""
    X, Y, f, g = _f32(X), _f32(Y), _f64(f), _f64(g)
    m, d = X.shape
    n = Y.shape[0]
    sigma = np.empty((m, n), np.float64)
    cost = np.empty((m, n), np.float64)
    fn = lib().orc_norm_matrices64 if precision == 1 else lib().orc_norm_matrices
    fn(_ptr(X), _ptr(Y), _ptr(f), _ptr(g), m, n, d, int(kind), _ptr(sigma), _ptr(cost))
    return sigma, cost


def topk(sigma, k: int, transpose: bool = False):
    sigma = _f64(sigma)
    m, n = sigma.shape
    outer = n if transpose else m
    vals = np.empty((outer, k), np.float64)
    idx = np.empty((outer, k), np.int32)
    lib().orc_topk(_ptr(sigma), m, n, int(k), int(bool(transpose)), _ptr(vals), _ptr(idx))
    return vals, idx


def stats(sigma, cost):
    """(num, den, count, max sigma+, max|cost|)."""
    sigma, cost = _f64(sigma), _f64(cost)
    out = np.empty(5, np.float64)
    lib().orc_stats(_ptr(sigma), _ptr(cost), sigma.shape[0], sigma.shape[1], _ptr(out))
    return out


def l2sq_scan(X, Y, p, q, qb, db, k: int, scale=2.0):
    sigma, cost = l2sq_matrices(X, Y, p, q, qb, db, scale)
    rv, ri = topk(sigma, k, False)
    cv, ci = topk(sigma, k, True)
    return rv, ri, cv, ci, stats(sigma, cost)


def norm_scan(X, Y, f, g, k: int, kind: int, precision: int = 0):
    sigma, cost = norm_matrices(X, Y, f, g, kind, precision)
    rv, ri = topk(sigma, k, False)
    cv, ci = topk(sigma, k, True)
    return rv, ri, cv, ci, stats(sigma, cost)


def sddmm_l2sq(X, Y, p, q, rowptr, col, scale=2.0):
    X, Y, p, q = _f32(X), _f32(Y), _f64(p), _f64(q)
    rowptr = np.ascontiguousarray(rowptr, dtype=np.int32)
    col = np.ascontiguousarray(col, dtype=np.int32)
    out = np.empty(col.size, np.float64)
    lib().orc_sddmm_l2sq(_ptr(X), _ptr(Y), _ptr(p), _ptr(q), _ptr(rowptr), _ptr(col), X.shape[0],
                         X.shape[1], float(scale), _ptr(out))
    return out


def pair_costs_norm(X, Y, rows, cols, kind: int):
    X, Y = _f32(X), _f32(Y)
    rows = np.ascontiguousarray(rows, dtype=np.int64)
    cols = np.ascontiguousarray(cols, dtype=np.int64)
    out = np.empty(rows.size, np.float64)
    lib().orc_pair_costs_norm(_ptr(X), _ptr(Y), _ptr(rows), _ptr(cols), rows.size, X.shape[1], int(kind), _ptr(out))
    return out


def pdhg_solve(rows, cols, costs, source_mass, target_mass, *, warm_start_primal=None,
               warm_start_dual=None, evaluation_frequency=200, iteration_limit=2**31 - 1,
               tolerance=1e-6, rescale=False):
    """Single-thread Halpern-PDHG (solver.cpp:39-378). Returns a dict shaped like solve_once's result."""
    rows = np.ascontiguousarray(rows, dtype=np.int64)
    cols = np.ascontiguousarray(cols, dtype=np.int64)
    costs = _f64(costs)
    b = _f64(np.concatenate((np.asarray(source_mass, np.float64), np.asarray(target_mass, np.float64))))
    ns, nt, e = len(source_mass), len(target_mass), costs.size
    x0 = np.zeros(e) if warm_start_primal is None else _f64(warm_start_primal)
    y0 = np.zeros(ns + nt) if warm_start_dual is None else _f64(warm_start_dual)
    if isinstance(tolerance, dict):
        to = float(tolerance.get("objective", 1e-6))
        tp, td = float(tolerance.get("primal", to)), float(tolerance.get("dual", to))
    else:
        to = tp = td = float(tolerance)
    x = np.empty(e, np.float64)
    y = np.empty(ns + nt, np.float64)
    info = _PdhgInfo()
    rc = lib().orc_pdhg_solve(_ptr(rows), _ptr(cols), _ptr(costs), _ptr(b), ns, nt, e, _ptr(x0), _ptr(y0),
                              int(evaluation_frequency), int(iteration_limit), to, tp, td, int(bool(rescale)),
                              _ptr(x), _ptr(y), ctypes.byref(info))
    if rc != 0:
        raise ValueError(f"oracle PDHG rejected the problem (code {rc})")
    return {
        "x": x, "y": y, "obj_val": info.pobj, "dual_obj_val": info.dobj, "iterations": int(info.iterations),
        "termination_reason": _REASONS[info.reason], "primal_feas": info.rp, "dual_feas": info.rd,
        "gap": info.gap, "restart_count": int(info.restarts), "primal_weight": info.weight,
        "success": info.reason == 1,
    }


def sparsify_support(rows, cols, values, costs, n_source: int, n_target: int, target_nnz: int,
                     zero_tolerance: float = 1e-15):
    """Cycle cancelling on a restricted-OT primal (small inputs; plain Python with breadth-first tree paths).

    Restates the reference's sparsifier (restricted_ot/support_sparsification.py:52 ->
    support_sparsifier_lct.cpp:378-555): a spanning forest of the positive edges in edge order (union-find);
    every other positive edge, in edge order, pushes flow around the cycle it closes with the tree path from its
    source to its target -- edges at even positions of that path (counted from the source) lose what the entering
    edge gains, odd positions gain it -- in the direction whose cost c_e - C_even + C_odd is not positive, by the
    largest step keeping flows >= 0. If the entering edge stays positive, the first path edge (from the source)
    at the minimum leaves the forest; otherwise the entering edge drops to zero. The exact positive count is
    re-taken after every (count - target) cancelled cycles, and the loop stops once count <= target.
    Returns (values, output nnz, cycles cancelled)."""
    rows = np.asarray(rows, np.int64)
    cols = np.asarray(cols, np.int64)
    vals = np.array(values, dtype=np.float64)
    costs = np.asarray(costs, np.float64)
    vals[vals <= zero_tolerance] = 0.0
    V = n_source + n_target
    parent = list(range(V))

    def find(a):
        while parent[a] != a:
            parent[a] = parent[parent[a]]
            a = parent[a]
        return a

    rank = [0] * V
    adj = {v: {} for v in range(V)}   # vertex -> {neighbour: edge id} of the forest
    tree, entering = [], []
    for k in range(len(rows)):
        if vals[k] <= 0.0:
            continue
        a, b = find(int(rows[k])), find(n_source + int(cols[k]))
        if a == b:
            entering.append(k)
            continue
        if rank[a] < rank[b]:
            a, b = b, a
        parent[b] = a
        rank[a] += rank[a] == rank[b]
        tree.append(k)
        adj[int(rows[k])][n_source + int(cols[k])] = k
        adj[n_source + int(cols[k])][int(rows[k])] = k
    nnz = int(np.count_nonzero(vals > zero_tolerance))
    cycles = 0
    if nnz <= target_nnz or not entering:
        return vals, nnz, 0

    def tree_path(u, v):
        prev = {u: None}
        queue = [u]
        for x in queue:
            if x == v:
                break
            for y, k in adj[x].items():
                if y not in prev:
                    prev[y] = (x, k)
                    queue.append(y)
        path = []
        while v != u:
            x, k = prev[v]
            path.append(k)
            v = x
        return path[::-1]   # edges from u to v

    tree_set = set(tree)
    check_at = nnz - target_nnz
    for pos, k in enumerate(entering):
        if cycles >= check_at:
            count = (len(entering) - pos) + sum(1 for t in tree_set if vals[t] > zero_tolerance)
            if count <= target_nnz:
                break
            check_at = cycles + (count - target_nnz)
        flow = vals[k]
        if flow <= zero_tolerance:
            continue
        s, t = int(rows[k]), n_source + int(cols[k])
        path = tree_path(s, t)
        even, odd = path[0::2], path[1::2]
        gain = costs[k] - sum(costs[e] for e in even) + sum(costs[e] for e in odd)
        direction = 1.0 if gain <= 0.0 else -1.0
        losing = even if direction > 0 else odd
        step, leaving = np.inf, None
        for e in losing:
            if vals[e] < step:
                step, leaving = vals[e], e
        if direction < 0 and flow < step:
            step = flow
        step = max(0.0, step)
        for e in even:
            vals[e] -= direction * step
        for e in odd:
            vals[e] += direction * step
        flow += direction * step
        if flow > zero_tolerance:
            vals[leaving] = 0.0
            a, b = int(rows[leaving]), n_source + int(cols[leaving])
            del adj[a][b], adj[b][a]
            tree_set.discard(leaving)
            adj[s][t] = k
            adj[t][s] = k
            tree_set.add(k)
            vals[k] = flow
        else:
            vals[k] = 0.0
        cycles += 1
    vals[vals <= zero_tolerance] = 0.0
    return vals, int(np.count_nonzero(vals)), cycles


# ---------------------------------------------------------------------------------------------------
# Reference CPU modules compiled from /root/reference (optional; absent on the GPU box unless built here).
# ---------------------------------------------------------------------------------------------------

def _load_ref(name: str):
    ref = _DIR / "_ref"
    for path in sorted(ref.glob(f"{name}*.so")):
        spec = importlib.util.spec_from_file_location(name, path)
        module = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(module)
        return module
    return None


def ref_scan():
    """The reference's CPU scan epilogue module (_native/cpp/scan.cpp), or None if not built."""
    return _load_ref("_scan")


def ref_lp():
    """The reference's CPU PDHG module (_native/cpp/solver.cpp), or None if not built."""
    return _load_ref("_lp")


def ref_sparsify():
    """The reference's support sparsifier (_native/support_sparsifier/*.cpp), or None if not built."""
    return _load_ref("_sparsify")


def parity_pins() -> dict:
    """How each oracle function is pinned (documentation for the test suite)."""
    return {
        "dot64": "closed forms (integer-valued rows, exact sums) + brute force in numpy with the same lane order",
        "l2sq_matrices": "reference KAT tests/torch_scan_test.py:26-59 + reference _scan.dot_tile (scan.cpp:136-227) "
                         "fed the same fp64 products",
        "topk": "reference _scan.merge_topk/dot_tile strict-greater insertion + brute-force sort with lowest-index ties",
        "stats": "reference KAT tests/torch_scan_test.py:61-96 (certificate formula) + _scan.dot_tile mode 0 sums",
        "norm_matrices": "reference KAT tests/torch_scan_test.py:61-96 dense l1/l2/linf + numpy fp32 sequential sums",
        "sddmm_l2sq": "closed form (p+q-2<x,y>) against numpy float64 einsum at 1e-12 and exact integer-valued cases",
        "pair_costs_norm": "numpy float64 norms at 1e-13 and exact integer-valued cases",
        "pdhg_solve": "reference _lp.solve_once (solver.cpp) with one thread, bit-identical iterates; "
                      "KATs tests/torch_restricted_ot_pdlp_test.py:16-80 (obj 0.1); scipy linprog optimum",
        "sparsify_support": "reference _sparsify.sparsify_transport_support (support_sparsifier_lct.cpp) on random "
                            "supports (same flows to 1e-12, same counts); invariants: row/column sums, cost never "
                            "increases, flows >= 0, count <= target",
    }


__all__ = [
    "build", "lib", "dot64", "l2sq_matrices", "norm_matrices", "topk", "stats", "l2sq_scan", "norm_scan",
    "sddmm_l2sq", "pair_costs_norm", "pdhg_solve", "sparsify_support", "ref_scan", "ref_lp", "ref_sparsify",
    "parity_pins",
]
