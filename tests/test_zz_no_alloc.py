"""The allocation-free norm scan (hm_pricing_norm_noalloc) against the workspace entry point (GPU only).

Both are called through the C ABI on the same inputs: identical lists and certificate on two calls in a row (the
second smaller, so stale scratch contents from the first would show), and a call too large for the static scratch
is rejected before any launch."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from hello_ot_amd import _lib

pytestmark = pytest.mark.gpu

FLAGS = _lib.HM_ROWS | _lib.HM_COLS | _lib.HM_STATS | _lib.HM_LINF


def _inputs(dev, m, n, d, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    X = torch.rand(m, d, generator=g).to(dev)
    Y = torch.rand(n, d, generator=g).to(dev)
    f = (0.3 + 0.2 * torch.randn(m, generator=g, dtype=torch.float64)).to(dev)
    gg = (0.3 + 0.2 * torch.randn(n, generator=g, dtype=torch.float64)).to(dev)
    return X, Y, f, gg


def _outputs(dev, m, n, k):
    return (torch.full((m, k), 7.0, dtype=torch.float64, device=dev), torch.full((m, k), 7, dtype=torch.int32, device=dev),
            torch.full((n, k), 7.0, dtype=torch.float64, device=dev), torch.full((n, k), 7, dtype=torch.int32, device=dev),
            torch.full((5,), 7.0, dtype=torch.float64, device=dev))


def _with_workspace(dev, X, Y, f, g, k, kind):
    lib = _lib.load()
    m, n, d = X.shape[0], Y.shape[0], X.shape[1]
    out = _outputs(dev, m, n, k)
    ws = torch.empty(max(int(lib.hm_pricing_norm_workspace_bytes(m, n, d, k, FLAGS)), 256), dtype=torch.uint8,
                     device=dev)
    rc = lib.hm_pricing_norm(_lib.stream_handle(dev), *map(_lib.ptr, (X, Y, f, g)), m, n, d, k, kind, FLAGS,
                             *map(_lib.ptr, out), _lib.ptr(ws), ws.numel())
    _lib.check(rc, "hm_pricing_norm")
    return out


def _no_alloc(dev, X, Y, f, g, k, kind):
    lib = _lib.load()
    m, n, d = X.shape[0], Y.shape[0], X.shape[1]
    out = _outputs(dev, m, n, k)
    rc = lib.hm_pricing_norm_noalloc(_lib.stream_handle(dev), *map(_lib.ptr, (X, Y, f, g)), m, n, d, k, kind, FLAGS,
                                     *map(_lib.ptr, out))
    _lib.check(rc, "hm_pricing_norm_noalloc")
    return out


@pytest.mark.parametrize("kind", [0, 1, 2])
def test_no_alloc_matches_the_workspace_entry_point(cuda, kind):
    for m, n, d, k, seed in ((3000, 2500, 8, 8, 1), (700, 900, 5, 2, 2)):   # second call smaller
        X, Y, f, g = _inputs(cuda, m, n, d, seed + kind)
        want = _with_workspace(cuda, X, Y, f, g, k, kind)
        got = _no_alloc(cuda, X, Y, f, g, k, kind)
        torch.cuda.synchronize()
        for a, b in zip(got, want):
            assert torch.equal(a, b)


def test_no_alloc_with_profiling_on_is_captured_into_a_graph(cuda):
    """With the library's timing report switched on, the allocation-free fused call (k <= 2, rows and columns)
    still makes no host readback and no stream synchronisation: it is captured into a HIP graph, and every replay,
    with eager work between replays, matches the workspace entry point."""
    lib = _lib.load()
    m, n, d, k, kind = 700, 900, 5, 2, 0
    X, Y, f, g = _inputs(cuda, m, n, d, 3)
    want = _with_workspace(cuda, X, Y, f, g, k, kind)
    _no_alloc(cuda, X, Y, f, g, k, kind)                # first call on the device: scratch address lookup
    out = _outputs(cuda, m, n, k)
    graph = torch.cuda.CUDAGraph()
    _lib.profile_enable(True)
    try:
        torch.cuda.synchronize()
        with torch.cuda.graph(graph):
            rc = lib.hm_pricing_norm_noalloc(_lib.stream_handle(cuda), *map(_lib.ptr, (X, Y, f, g)), m, n, d, k,
                                             kind, FLAGS, *map(_lib.ptr, out))
        _lib.check(rc, "hm_pricing_norm_noalloc (captured)")
        for _ in range(3):
            for t in out:
                t.fill_(7)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            for a, b in zip(out, want):
                assert torch.equal(a, b)
    finally:
        _lib.profile_enable(False)
        _lib.profile_reset()


def test_no_alloc_rejects_calls_beyond_its_scratch(cuda):
    lib = _lib.load()
    cap = int(lib.hm_pricing_norm_noalloc_max_bytes())
    assert cap == 64 << 20
    m = n = 1 << 23                                    # 8M x 8M: the partial lists alone exceed 64 MiB
    assert lib.hm_pricing_norm_workspace_bytes(m, n, 8, 32, FLAGS) > cap
    X = torch.empty(1, 8, device=cuda)
    f = torch.empty(1, dtype=torch.float64, device=cuda)
    dummy = torch.empty(1, dtype=torch.float64, device=cuda)
    idx = torch.empty(1, dtype=torch.int32, device=cuda)
    rc = lib.hm_pricing_norm_noalloc(_lib.stream_handle(cuda), _lib.ptr(X), _lib.ptr(X), _lib.ptr(f), _lib.ptr(f),
                                     m, n, 8, 32, 0, FLAGS, _lib.ptr(dummy), _lib.ptr(idx), _lib.ptr(dummy),
                                     _lib.ptr(idx), _lib.ptr(dummy))
    assert rc == _lib.HM_ENOSPC and "static scratch" in _lib.last_error()
