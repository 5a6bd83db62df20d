"""``_support_sparsifier_ext`` (reference ``_native/support_sparsifier/support_sparsifier_bindings.cpp:82-95``),
served by ``hm_sparsify_support``."""
from __future__ import annotations

from hello_ot_amd.resident.sparsify import sparsify_transport_support as _sparsify


def sparsify_transport_support(n_source, n_target, rows, cols, values, costs, target_nnz, zero_tolerance=1e-15):
    """-> {"values": f64(E), "output_nnz", "cycle_updates", "tree_operations"}: cycle cancelling until the positive
    support reaches target_nnz (the reference module's result dictionary)."""
    r = _sparsify(rows, cols, values, costs, n_source=n_source, n_target=n_target, target_nnz=target_nnz,
                  zero_tolerance=zero_tolerance)
    return {"values": r.values, "output_nnz": r.output_nnz, "cycle_updates": r.cycle_updates,
            "tree_operations": r.tree_operations}
