"""The north-star instance solved end to end on the GPU and checked independently (GPU only).

1,280,000 x 1,280,000 points, d = 8192, each side from its own 64-component Gaussian mixture, uniform masses,
squared-Euclidean cost, default options (tolerance 1e-6 on the relative l2 dual infeasibility). The solve runs the
default int8 sweep; afterwards, on freshly generated copies of the same inputs in their original order:

* the plan's marginals and the last LP's residual and duality gap;
* the objective recomputed from the pair-cost kernel on the returned support;
* the returned duals' certificate recomputed over all 1.64e12 pairs by a sweep of another precision (split-bf16,
  whose candidates and near-zero scores come from different dot products), with the exact maximum violation;
* a certified optimality gap: the objective against the weak-duality lower bound of the c-transformed duals
  (``certified_lower_bounds``), from the exact row and column maxima of that scan.

The reference checks its GPU-resident solve on the same quantities at small sizes
(tests/hello_gpu_resident_test.py:73-104). The test takes about four minutes; its steps print as they finish.
"""
from __future__ import annotations

import time

import numpy as np
import pytest
import torch

from _shapes import certified_lower_bounds, gmm, plan_residual
from hello_ot_amd import SolverOptions, solve
from hello_ot_amd.costs.pairs import lowrank_pair_costs
from hello_ot_amd.kernels.generic_scan import pricing_l2sq
from hello_ot_amd.resident.cost import offsets

pytestmark = pytest.mark.gpu

C5_N, C5_D = 1_280_000, 8192
TOLERANCE = 1e-6
# Certified optimality gap at the default tolerance, relative to the objective (see test_gpu_full_shapes).
CERTIFIED_GAP = 1e-5


def _inputs(dev):
    return gmm(C5_N, C5_D, seed=1, dev=dev, means_seed=11), gmm(C5_N, C5_D, seed=2, dev=dev, means_seed=12)


@pytest.mark.timeout(900)
def test_c5_full_solve_certified(cuda, capsys):
    started = time.perf_counter()

    def say(msg):
        with capsys.disabled():
            print(f"\n[c5-solve {time.perf_counter() - started:6.1f}s] {msg}", flush=True)

    torch.cuda.empty_cache()
    say("generating 1,280,000 x 8192 per side")
    X, Y = _inputs(cuda)
    sample_x, sample_y = X[::997].clone(), Y[::997].clone()
    say("solving (progress lines of the finest levels follow)")
    with capsys.disabled():
        r = solve(X, Y, options=SolverOptions(verbose="detailed", consume_input_features=True))
    # the solve reorders the consumed inputs in place and puts them back when it ends
    assert torch.equal(X[::997], sample_x) and torch.equal(Y[::997], sample_y)
    torch.cuda.empty_cache()
    finest = r.solve_stage.levels[-1].solve
    last = finest.iterations[-1]
    say(f"solved in {r.total_wall_time:.1f} s, objective {r.objective!r}, peak {r.peak_gpu_memory_mib / 1024:.1f} "
        f"GiB, final dual infeasibility {last.convergence.dual_feasibility:.3e}")
    assert finest.summary.converged and last.convergence.dual_feasibility <= TOLERANCE
    assert last.solve_lp.primal_feasibility <= TOLERANCE and last.solve_lp.primal_dual_gap <= TOLERANCE

    n = m = C5_N
    a = np.full(n, 1.0 / n)
    b = np.full(m, 1.0 / m)
    sol = r.solution.to_cpu()
    residual = plan_residual(sol, a, b)
    say(f"support {sol.values.size} edges, marginal residual {np.linalg.norm(residual):.3e} (largest entry "
        f"{np.abs(residual).max() * n:.2e} of a point's mass)")
    assert np.linalg.norm(residual) <= TOLERANCE * (1.0 + np.sqrt(a @ a + b @ b))
    assert (sol.values >= 0).all()

    p, q = offsets(X), offsets(Y)
    rows = torch.as_tensor(sol.rows, device=cuda)
    cols = torch.as_tensor(sol.cols, device=cuda)
    costs = lowrank_pair_costs(X, Y, p, q, rows, cols)
    objective = float(costs @ torch.as_tensor(sol.values, device=cuda))
    say(f"objective of the returned plan, recomputed: {objective!r}")
    # the solver's objective also counts the support's flows at or below 1e-12, which the returned plan drops
    assert objective == pytest.approx(r.objective, rel=1e-9)
    del rows, cols, costs

    f, g = r.solution.source_dual, r.solution.target_dual
    say("certificate of the returned duals over all pairs, split-bf16 sweep")
    rv, _, cv, _, st = pricing_l2sq(X, Y, p, q, f - p, g - q, 1, linf=True, precision="bf16x3")
    num, den, count, mx, cmax = (float(v) for v in st.cpu())
    infeasibility = num ** 0.5 / (1.0 + den ** 0.5)
    row_max, col_max = rv[:, 0], cv[:, 0]
    at = torch.full((n,), 1.0 / n, dtype=torch.float64, device=cuda)
    bt = torch.full((m,), 1.0 / m, dtype=torch.float64, device=cuda)
    lb = certified_lower_bounds(at, bt, f, g, row_max, col_max)
    certified = (objective - lb["best"]) / abs(objective)
    say(f"recomputed: infeasibility {infeasibility:.3e} (solver {last.convergence.dual_feasibility:.3e}), violated "
        f"pairs {int(count)} (solver {last.dual_violation.violations_found}), max violation {mx!r} (solver "
        f"{last.convergence.max_dual_violation!r}), dual value {lb['dual_value']!r}, lower bounds row {lb['row']!r} "
        f"col {lb['col']!r} uniform {lb['uniform']!r}, certified relative gap {certified:.3e}")
    assert infeasibility <= TOLERANCE
    # the maximum violation is exact fp64 in both scans (the best entry of the exact row lists)
    assert mx == pytest.approx(last.convergence.max_dual_violation, rel=1e-12, abs=1e-9)
    assert max(float(row_max.max()), 0.0) == mx
    assert -TOLERANCE <= certified <= CERTIFIED_GAP
