"""The reference's native-module names (``hello_ot_native.*``, loaded by ``importlib.import_module`` in the
reference's release mode, ``_source_build.py:152-184``) served by the MI355X library. CPU: the package contract, the
served and the refused names, and the host-side sparsifier module against the reference's own compiled module."""
from __future__ import annotations

import importlib

import numpy as np
import pytest

import oracle

SERVED = {
    "hierot_generic_pricing_small_ext": ["raw_scan_tiled"],
    "hierot_generic_cost_ext": ["raw_initial", "raw_certificate_tiled", "norms"],
    "hierot_norm_cost_scan_ext": ["fused_gcost_pairs"],
    "_support_sparsifier_ext": ["sparsify_transport_support"],
}


def test_package_contract_and_served_names():
    package = importlib.import_module("hello_ot_native")
    assert package.API_VERSION == 1      # packaging/native/src/hello_ot_native/__init__.py:3
    for name, functions in SERVED.items():
        module = importlib.import_module(f"hello_ot_native.{name}")
        for fn in functions:
            assert callable(getattr(module, fn))


@pytest.mark.parametrize("module,name", [("hierot_generic_pricing_small_ext", "scan"),
                                         ("hierot_generic_pricing_small_ext", "matrix_initial"),
                                         ("hierot_generic_cost_ext", "dots"),
                                         ("hierot_generic_cost_ext", "direct_norm_fp64")])
def test_tile_level_names_are_refused_by_name(module, name):
    m = importlib.import_module(f"hello_ot_native.{module}")
    with pytest.raises(NotImplementedError, match=name):
        getattr(m, name)
    assert not hasattr(m, "__not_a_name__")


def test_sparsifier_module_matches_the_reference_module():
    ref = oracle.ref_sparsify()
    if ref is None:
        pytest.skip("reference sparsifier not built (make -C oracle ref needs /root/reference)")
    mine = importlib.import_module("hello_ot_native._support_sparsifier_ext")
    rng = np.random.default_rng(9)
    ns, nt = 45, 38
    key = np.unique(rng.integers(0, ns, 800) * nt + rng.integers(0, nt, 800))
    rows, cols = key // nt, key % nt
    values = rng.random(len(key))
    values[rng.random(len(key)) < 0.2] = 0.0
    costs = rng.random(len(key))
    target = ns + nt - 1 + 3
    want = ref.sparsify_transport_support(ns, nt, rows, cols, values, costs, target, 1e-15)
    got = mine.sparsify_transport_support(ns, nt, rows, cols, values, costs, target)
    assert set(got) == set(want)
    np.testing.assert_array_equal(got["values"] > 0, want["values"] > 0)
    np.testing.assert_allclose(got["values"], want["values"], rtol=1e-12, atol=1e-14)
    for key_ in ("output_nnz", "cycle_updates", "tree_operations"):
        assert got[key_] == want[key_]


def test_pycupdlpx_contract_on_the_host():
    """The CuPDLPx module name the reference loads for its GPU-resident LPs (gpu_resident/solver.py:239-241): the
    device-CSR loader is the served path; host loaders, CPU tensors and solving before loading are refused."""
    import torch

    m = importlib.import_module("hello_ot_native.pycupdlpx")
    assert m.GPU_ARRAY_IO_VERSION == 1
    params = m.make_default_params()
    assert params["termination_norm"] == "l2" and params["step_size_method"] == 3
    solver = m.cupdlpx()
    for loader in (solver.loadData, solver.loadData_csr, solver.loadData_csc):
        with pytest.raises(NotImplementedError, match="loadData_device_csr"):
            loader()
    with pytest.raises(RuntimeError, match="No problem loaded"):
        solver.solve({})
    with pytest.raises(RuntimeError, match="No solution"):
        solver.getSolution()
    one = torch.zeros(3, dtype=torch.int32)
    with pytest.raises(TypeError, match="CUDA tensors"):
        solver.loadData_device_csr(one, one, None, 2, 1, one.double(), one.double(), 0.0, float("inf"), 2)
    with pytest.raises(ValueError):
        m.set_free_mode(3)
