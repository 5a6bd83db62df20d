"""The reference's native-module names, served by the MI355X library.

The reference loads its compiled extensions by name (``load_native_module("hello_ot_native.<module>")``,
``src/hello_ot/_source_build.py:152-184``; ``importlib.import_module`` in release mode) and checks the package's
interface version (``packaging/native/src/hello_ot_native/__init__.py:3``). With this directory on ``sys.path`` in
place of the reference's binary wheel, the entry points below run on the HIP kernels of ``libhelloot_hip.so``:

* ``hierot_generic_pricing_small_ext.raw_scan_tiled``: l2^2 rows + columns top-k (k <= 2) with the certificate;
* ``hierot_generic_cost_ext.raw_initial`` / ``raw_certificate_tiled`` / ``norms``: the directional raw scan, the
  certificate without candidates, fp64 squared row norms;
* ``hierot_norm_cost_scan_ext.fused_gcost_pairs``: fp64 norm costs of selected pairs;
* ``_support_sparsifier_ext.sparsify``: cycle-cancelling support sparsification;
* ``pycupdlpx.cupdlpx`` (``loadData_device_csr`` / ``setInitSol`` / ``solve`` / ``getSolution``,
  ``GPU_ARRAY_IO_VERSION`` 1): the restricted transport LPs of the GPU-resident loop, on the Halpern-PDHG
  (``hm_pdhg_solve``); general LPs and the host loaders raise ``NotImplementedError``.

The reference's tile-level functions (``scan``, ``merge``, ``topk``, ``dots``, ``direct_norm``, ...) have no
counterpart: the MI355X kernels fuse the tile loop, so those names raise ``NotImplementedError`` naming the fused
entry point that replaces them.
"""

API_VERSION = 1
