"""The reference's native-module names, served by the MI355X library.

The reference loads its compiled extensions by name (``load_native_module("hello_ot_native.<module>")``,
``src/hello_ot/_source_build.py:152-184``; ``importlib.import_module`` in release mode) and checks the package's
interface version (``packaging/native/src/hello_ot_native/__init__.py:3``). With this directory on ``sys.path`` in
place of the reference's binary wheel, the entry points below run on the HIP kernels of ``libhelloot_hip.so``:

* ``hierot_generic_pricing_small_ext.raw_scan_tiled``: l2^2 rows + columns top-k (k <= 2) with the certificate;
* ``hierot_generic_cost_ext.raw_initial`` / ``raw_certificate_tiled`` / ``norms``: the directional raw scan, the
  certificate without candidates, fp64 squared row norms;
* ``hierot_norm_cost_scan_ext.fused_gcost_pairs``: fp64 norm costs of selected pairs;
* ``_support_sparsifier_ext.sparsify``: cycle-cancelling support sparsification.

The reference's tile-level functions (``scan``, ``merge``, ``topk``, ``dots``, ``direct_norm``, ...) have no
counterpart: the MI355X kernels fuse the tile loop, so those names raise ``NotImplementedError`` naming the fused
entry point that replaces them. The CuPDLPx module (``pycupdlpx``) is replaced by the restricted-OT PDHG
(``hello_ot_amd.lp.NativeRestrictedOTPDLP``), whose interface is the reference's restricted-OT contract rather than
CuPDLPx's general LP loader.
"""

API_VERSION = 1
