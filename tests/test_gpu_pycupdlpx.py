"""``hello_ot_native.pycupdlpx`` on ``hm_pdhg_solve``, and the scalar-rescaling PDHG mode (GPU only).

The payloads are built the way the reference's GPU-resident loop builds them (``gpu_resident/support.py:97-109``:
int32 CSR over the support sorted by (row, col), source rows then target rows, all-one values, constant bounds),
plain, pre-rescaled by the degree-sqrt diagonal (``_internal/lp/cupdlpx.py:373-478``) and with the scalar
bound/objective rescaling appended (``cupdlpx.py:489-540``). The module must recover the support, costs and masses and
return the oracle's iterates for the same inputs. The scalar-rescaling mode is checked against the reference's own
solver.cpp vectors (tests/golden/pdhg_7x5_*_rescale*.npz), including a case that diverges numerically, where the
restricted-OT wrapper's one-shot retry must run and report the first attempt.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from hello_ot_amd.lp import NativeRestrictedOTPDLP
from hello_ot_native import pycupdlpx

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def _lp(seed, ns, nt, extra):
    rng = np.random.default_rng(seed)
    rows = np.concatenate([np.arange(ns), rng.integers(0, ns, extra), rng.integers(0, ns, nt)])
    cols = np.concatenate([rng.integers(0, nt, ns), rng.integers(0, nt, extra), np.arange(nt)])
    key = np.unique(rows * nt + cols)          # the support is a set of (row, col) keys in row-major order
    rows, cols = key // nt, key % nt
    a, b = rng.random(ns) + 0.1, rng.random(nt) + 0.1
    return rows.astype(np.int64), cols.astype(np.int64), rng.random(rows.size), a / a.sum(), b / b.sum()


def _payload(dev, rows, cols, costs, a, b, *, prescale=False, scalar=False):
    """The reference's device payload for one restricted LP; returns (payload, costs, masses) where costs and
    masses are what the module recovers from it (bit for bit: the same fp64 operations)."""
    ns, nt, e = a.size, b.size, rows.size
    r, c = torch.as_tensor(rows, device=dev), torch.as_tensor(cols, device=dev)
    counts = torch.cat((torch.bincount(r, minlength=ns), torch.bincount(c, minlength=nt)))
    row_ptr = torch.cat((torch.zeros(1, dtype=torch.int64, device=dev), counts.cumsum(0))).int()
    col_ind = torch.cat((torch.arange(e, device=dev), torch.argsort(c, stable=True))).int()
    cost_t = torch.as_tensor(costs, dtype=torch.float64, device=dev)
    rhs = torch.as_tensor(np.concatenate([a, b]), dtype=torch.float64, device=dev)
    p = dict(row_ptr=row_ptr, col_ind=col_ind, values=torch.ones(2 * e, dtype=torch.float64, device=dev),
             m=ns + nt, n=e, c=cost_t, rhs=rhs, lb=0.0, ub=float("inf"), nEqs=ns + nt,
             variable_bound_mode="constant", matrix_value_mode="implicit_aty")
    if not prescale:
        return p, costs, np.concatenate([a, b])
    con = torch.sqrt(counts.double())
    var = torch.sqrt(torch.bincount(col_ind.long(), minlength=e).double())
    row_of = torch.repeat_interleave(torch.arange(ns + nt, device=dev), counts)
    cs, bs = cost_t / var, rhs / con
    ovr = cbr = 1.0
    if scalar:
        ovr = 1.0 / (float(torch.linalg.vector_norm(cs)) + 1.0)
        cbr = 1.0 / (float(torch.linalg.vector_norm(bs)) + 1.0)
        cs, bs = cs * ovr, bs * cbr
    p.update(values=1.0 / (con[row_of] * var[col_ind.long()]), c=cs, rhs=bs, constraint_rescaling=con,
             variable_rescaling=var, constraint_bound_rescaling=cbr, objective_vector_rescaling=ovr,
             has_precomputed_rescaling=True)
    return p, ((cs * var) / ovr).cpu().numpy(), ((bs * con) / cbr).cpu().numpy()


def _load(p):
    s = pycupdlpx.cupdlpx()
    s.loadData_device_csr(p["row_ptr"], p["col_ind"], p["values"], p["m"], p["n"], p["c"], p["rhs"], p["lb"],
                          p["ub"], p["nEqs"], p["variable_bound_mode"], p["matrix_value_mode"],
                          p.get("constraint_rescaling"), p.get("variable_rescaling"),
                          p.get("constraint_bound_rescaling", 1.0), p.get("objective_vector_rescaling", 1.0),
                          None, None, p.get("has_precomputed_rescaling", False), None, None)
    return s


def _params(freq, limit, tol, **extra):
    return dict(termination_evaluation_frequency=freq, iteration_limit=limit, eps_optimal_relative=tol,
                eps_feasible_relative_primal=tol, eps_feasible_relative_dual=tol, **extra)


def _check(out, ref):
    assert out["termination_reason"] == ref["termination_reason"]
    assert out["iterations"] == ref["iterations"]
    assert out["restart_count"] == ref["restart_count"]
    x, y = (v.cpu().numpy() if torch.is_tensor(v) else v for v in (out["x"], out["y"]))
    np.testing.assert_allclose(x, ref["x"], rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(y, ref["y"], rtol=1e-9, atol=1e-12)


@pytest.mark.parametrize("prescale,scalar", [(False, False), (True, False), (True, True)])
def test_module_solves_reference_payloads_like_the_oracle(cuda, prescale, scalar):
    rows, cols, costs, a, b = _lp(5, 40, 31, 300)
    p, rc, masses = _payload(cuda, rows, cols, costs, a, b, prescale=prescale, scalar=scalar)
    s = _load(p)
    assert s.getLoadStats()["n_source"] == 40 and s.getLoadStats()["edges"] == rows.size
    out = s.solve(_params(50, 3000, 1e-9))
    ref = oracle.pdhg_solve(rows, cols, rc, masses[:40], masses[40:], evaluation_frequency=50,
                            iteration_limit=3000, tolerance=1e-9, rescale=scalar)
    _check(out, ref)
    assert isinstance(out["x"], np.ndarray)            # return_device defaults to the host
    assert out["primal_objective"] == pytest.approx(ref["obj_val"], rel=1e-10)
    sol = s.getSolution()
    assert sol["iters"] == out["iterations"] and sol["PrimalObj"] == out["primal_objective"]


def test_module_warm_start_device_output_and_pock_chambolle(cuda):
    rows, cols, costs, a, b = _lp(6, 30, 25, 150)
    rng = np.random.default_rng(1)
    x0, y0 = rng.random(rows.size) * 0.01, rng.normal(0, 0.1, 55)
    p, rc, masses = _payload(cuda, rows, cols, costs, a, b)
    s = _load(p)
    s.setInitSol(torch.as_tensor(x0, device=cuda), torch.as_tensor(y0, device=cuda))
    # Pock-Chambolle alpha = 1 is the degree-sqrt scaling the solver applies anyway
    out = s.solve(_params(40, 2000, 1e-9, return_device="cuda", has_pock_chambolle_alpha=True))
    ref = oracle.pdhg_solve(rows, cols, rc, masses[:30], masses[30:], warm_start_primal=x0, warm_start_dual=y0,
                            evaluation_frequency=40, iteration_limit=2000, tolerance=1e-9)
    assert out["x"].is_cuda and out["x"].dtype == torch.float64
    _check(out, ref)


def test_module_refuses_what_it_does_not_solve(cuda):
    rows, cols, costs, a, b = _lp(7, 6, 5, 10)
    p, _, _ = _payload(cuda, rows, cols, costs, a, b)
    s = _load(p)
    for bad in (dict(l_inf_ruiz_iterations=10), dict(has_pock_chambolle_alpha=True, pock_chambolle_alpha=2.0),
                dict(termination_norm="linf"), dict(step_size_method=1)):
        with pytest.raises(NotImplementedError):
            s.solve(_params(10, 10, 1e-6, **bad))
    with pytest.raises(NotImplementedError, match="equality"):
        _load(dict(p, nEqs=p["m"] - 1))
    with pytest.raises(NotImplementedError, match="bounds"):
        _load(dict(p, ub=1.0))
    broken = p["col_ind"].clone()
    broken[0] = broken[1]                                # variable 0 loses its source entry
    with pytest.raises(NotImplementedError, match="incidence"):
        _load(dict(p, col_ind=broken))
    with pytest.raises(NotImplementedError, match="values"):
        _load(dict(p, values=p["values"] * 2.0))


@pytest.mark.parametrize("name", ["skewed", "heavy", "diverge"])
@pytest.mark.parametrize("rescale", [0, 1])
def test_scalar_rescaling_mode_matches_reference_vectors(cuda, name, rescale):
    z = np.load(GOLDEN / f"pdhg_7x5_{name}_rescale{rescale}.npz")
    p, _, _ = _payload(cuda, z["rows"], z["cols"], z["costs"], z["source_mass"], z["target_mass"])
    tol = float(z["tolerance"])
    out = _load(p).solve(_params(int(z["frequency"]), int(z["limit"]), tol, bound_objective_rescaling=bool(rescale)))
    assert out["termination_reason"] == str(z["termination_reason"])
    assert out["iterations"] == int(z["iterations"]) and out["restart_count"] == int(z["restart_count"])
    # x spans 1e100 in the heavy case: relative agreement, with the absolute floor scaled to the masses
    floor = 1e-12 * float(np.abs(z["source_mass"]).max())
    np.testing.assert_allclose(out["x"], z["x"], rtol=1e-9, atol=floor)
    np.testing.assert_allclose(out["y"], z["y"], rtol=1e-9, atol=1e-12 * max(1.0, float(np.abs(z["y"]).max())))


def test_divergence_triggers_the_one_shot_rescaled_retry(cuda):
    """restricted_ot_pdlp.py:64-93: a first solve that ends in NUMERICAL_DIVERGENCE is run once more with scalar
    rescaling, and the result reports the first attempt. Both attempts are the reference's (golden vectors)."""
    first = np.load(GOLDEN / "pdhg_7x5_diverge_rescale0.npz")
    second = np.load(GOLDEN / "pdhg_7x5_diverge_rescale1.npz")
    assert str(first["termination_reason"]) == "NUMERICAL_DIVERGENCE"
    r = NativeRestrictedOTPDLP(device=cuda, evaluation_frequency=int(first["frequency"]),
                               iteration_limit=int(first["limit"])).solve_restricted(
        rows=first["rows"], cols=first["cols"], costs=first["costs"], source_mass=first["source_mass"],
        target_mass=first["target_mass"], tolerance=float(first["tolerance"]))
    diag = r.solver_diag
    assert diag["numerical_rescaling_retry"] is True
    assert diag["numerical_rescaling_first_termination_reason"] == "NUMERICAL_DIVERGENCE"
    assert diag["numerical_rescaling_first_iterations"] == int(first["iterations"])
    assert diag["scaling_mode"] == "degree_sqrt_with_scalar_retry"
    assert r.termination_reason == str(second["termination_reason"]) and r.iterations == int(second["iterations"])
    assert not r.success


def test_no_retry_when_the_first_solve_converges(cuda):
    z = np.load(GOLDEN / "pdhg_7x5_skewed_rescale0.npz")
    r = NativeRestrictedOTPDLP(device=cuda, evaluation_frequency=int(z["frequency"]),
                               iteration_limit=int(z["limit"])).solve_restricted(
        rows=z["rows"], cols=z["cols"], costs=z["costs"], source_mass=z["source_mass"], target_mass=z["target_mass"],
        tolerance=float(z["tolerance"]))
    assert r.success and r.solver_diag["numerical_rescaling_retry"] is False
    assert "numerical_rescaling_first_termination_reason" not in r.solver_diag
    assert r.iterations == int(z["iterations"])
    np.testing.assert_allclose(r.x.cpu().numpy(), z["x"], rtol=1e-9, atol=1e-12)
