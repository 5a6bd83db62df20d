"""Benchmark of the MI355X HELLO hot path (one GPU).

Headline (BASELINE.json metric "pricing pairs/s ..., m=n=1.28M d=8192 l2^2"): one step = the l2^2
bidirectional pricing scan with the full-edge certificate (the work of ``check_optimality``) of one query chunk
against the resident side of the C5 instance: resident Y = 1,280,000 x 8192 fp32 drawn from a 64-component
Gaussian mixture (means ~ N(0, 4I), identity covariance, equal weights), query chunk X = ``--chunk`` rows of an
independent mixture; k = 2 (pricing_topk default). Inputs are resident in HBM before timing starts.
``value`` = pairs scanned per second (chunk x 1.28M per step).

The metric's second half, the full C5 solve (1.28M x 1.28M, d=8192, relative dual infeasibility 1e-6), runs
last and lands in ``solve_seconds.c5`` (seconds, convergence, final dual infeasibility, peak GPU memory, and the
initialization / scan / LP split); ``--no-c5-solve`` skips it.

Extra fields measure the other configurations: C2 (isolated 131072^2 d=64 k=8 scan), C3 (SDDMM + 1000 PDHG
iterations, m=n=262144 d=256, 16 nnz/row), C4 (l1 / linf scans, m=n=524288 d=8) and the full HELLO solve seconds
of C1 (Brenier, 2048, d=32) and C4 (l1 and linf, 524288, d=8).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "hello-ot_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

import numpy as np  # noqa: E402
import torch  # noqa: E402

PEAK_FP32_MFMA = 157.3e12   # MI355X dense fp32 matrix FLOP/s
PEAK_BF16_MFMA = 2.5e15     # MI355X dense bf16 matrix FLOP/s
PEAK_INT8_MFMA = 5.0e15     # MI355X dense int8 matrix OP/s
PEAK_HBM = 8.0e12           # MI355X HBM3E bytes/s
PEAK_VALU_OPS = 256 * 64 * 2.4e9  # non-packed fp32 VALU lane-ops/s (256 CU x 64 lanes/clk x 2.4 GHz)

# committed rocprofv3 summaries of each split sweep at the C5 step: (HBM traffic, shader counters)
SWEEP_PROFILES = {"bf16x3": (ROOT / "profiles" / "l2sq_sweep_c5_chunk8192.md",
                             ROOT / "profiles" / "l2sq_sweep_c5_counters.md"),
                  "int8x3": (ROOT / "profiles" / "l2sq_sweep_i8_c5_chunk8192.md",
                             ROOT / "profiles" / "l2sq_sweep_i8_c5_counters.md")}

C5_N = 1_280_000
C5_D = 8192


def roofline(precision, achieved):
    """Roofline of the sweep kernel. `achieved` is the algorithmic rate, 2*d flop per pair over the sweep's mean
    launch time, held against the peak of the matrix units the sweep runs on: the bf16 peak for the split-bf16
    sweep, the int8 peak for the int8 sweep, the fp32 peak for the fp32 sweep. The split sweeps execute three
    products per feature (hi*hi + hi*lo + lo*hi), so their executed MFMA rate (3x the algorithmic one) is reported
    beside it; their algorithmic fraction cannot exceed 1/3."""
    if precision == "bf16x3":
        products, peak = 3.0, PEAK_BF16_MFMA
    elif precision == "int8x3":
        products, peak = 3.0, PEAK_INT8_MFMA
    else:
        products, peak = 1.0, PEAK_FP32_MFMA
    kernel = {"bf16x3": "l2sq_sweep_split_w", "int8x3": "l2sq_sweep_i8_w"}.get(precision, "l2sq_sweep")
    return {"bound": "mfma", "achieved": achieved / 1e12, "peak": peak / 1e12, "unit": "TFLOP/s",
            "frac": achieved / peak, "traffic": sweep_traffic(precision),
            "traffic_source": SWEEP_PROFILES[precision][0].name if precision in SWEEP_PROFILES else None,
            "kernel": kernel, "sweep": precision,
            "work_per_pair": "2*d flop (algorithmic)", "algorithmic_flops_per_pair": 2 * C5_D,
            "executed_products_per_feature": products, "executed_tflops": products * achieved / 1e12,
            "executed_frac": products * achieved / peak,
            "counters": sweep_counters(precision)}


def sweep_traffic(precision):
    """HBM bytes per split-sweep launch at the C5 workload, from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE
    summary (scaled by a plain copy kernel's counters); None when no such summary is present."""
    try:
        if precision not in SWEEP_PROFILES:
            return None
        for line in SWEEP_PROFILES[precision][0].read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch"):
                return float(line.split("=")[1])
    except OSError:
        pass
    return None


def sweep_counters(precision):
    """The split sweep's sustained engine clock and MFMA-busy fraction at the C5 workload, from the committed
    rocprofv3 shader-counter summary (GRBM_GUI_ACTIVE and SQ_VALU_MFMA_BUSY_CYCLES over the dispatch); None when
    no such summary is present."""
    out = {}
    if precision not in SWEEP_PROFILES:
        return None
    profile = SWEEP_PROFILES[precision][1]
    try:
        for line in profile.read_text().splitlines():
            for key in ("sustained_clock_ghz", "mfma_busy_frac"):
                if line.startswith(key + " ="):
                    out[key] = float(line.split("=")[1])
    except OSError:
        return None
    if not out:
        return None
    out["source"] = profile.name
    return out


NORM_COUNTER_PROFILE = ROOT / "profiles" / "norm_sweep_c4_counters.md"


def norm_counters(name):
    """Executed VALU work of the C4 norm sweep from the committed rocprofv3 counter summary (SQ_INSTS_VALU wave
    instructions per pair over both sweeps of a call, and VALU instructions issued per SIMD per cycle); None when
    absent."""
    out = {}
    try:
        for line in NORM_COUNTER_PROFILE.read_text().splitlines():
            for key in ("valu_insts_per_pair", "valu_issue_per_simd_cycle", "duration_ms"):
                if line.startswith(f"{name}_{key} ="):
                    out[key] = float(line.split("=")[1])
    except OSError:
        return None
    if not out:
        return None
    out["source"] = NORM_COUNTER_PROFILE.name
    return out


def host_info():
    """CPU model and core count of the host the CPU baseline runs on."""
    model = None
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "cpu_model": model}


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def sync():
    torch.cuda.synchronize()


def gmm(rows, d, seed, dev, means_seed, chunk=32768):
    """Rows of a 64-component Gaussian mixture (means ~ N(0, 4I), identity covariance), generated on device."""
    g = torch.Generator(device=dev)
    g.manual_seed(means_seed)
    means = 2.0 * torch.randn(64, d, generator=g, device=dev)
    g.manual_seed(seed)
    out = torch.empty(rows, d, dtype=torch.float32, device=dev)
    for s in range(0, rows, chunk):
        e = min(rows, s + chunk)
        lab = torch.randint(0, 64, (e - s,), generator=g, device=dev)
        out[s:e] = torch.randn(e - s, d, generator=g, device=dev) + means[lab]
    return out


def gmm_host(rows, d, seed, dev, means_seed, chunk=32768):
    """The same rows as gmm(...) (same generator stream), generated chunk by chunk on the device and kept in host
    memory: the device never holds the whole side."""
    g = torch.Generator(device=dev)
    g.manual_seed(means_seed)
    means = 2.0 * torch.randn(64, d, generator=g, device=dev)
    g.manual_seed(seed)
    out = torch.empty(rows, d, dtype=torch.float32)
    for s in range(0, rows, chunk):
        e = min(rows, s + chunk)
        lab = torch.randint(0, 64, (e - s,), generator=g, device=dev)
        out[s:e].copy_(torch.randn(e - s, d, generator=g, device=dev) + means[lab])
    return out


def sqnorms(x, chunk=65536):
    out = torch.empty(x.shape[0], dtype=torch.float64, device=x.device)
    for s in range(0, x.shape[0], chunk):
        out[s:s + chunk] = (x[s:s + chunk].double() ** 2).sum(1)
    return out


def time_steps(fn, steps, warmup):
    for _ in range(warmup):
        fn()
    sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    sync()
    return (time.perf_counter() - t0) / steps


# ----------------------------------------------------------------------------------------------------------
# headline: C5 pricing chunk
# ----------------------------------------------------------------------------------------------------------

def c5_inputs(dev, chunk):
    log(f"[bench] generating C5 resident side {C5_N} x {C5_D} fp32 ({C5_N * C5_D * 4 / 2**30:.1f} GiB) ...")
    Y = gmm(C5_N, C5_D, seed=2, dev=dev, means_seed=12)
    X = gmm(chunk, C5_D, seed=1, dev=dev, means_seed=11)
    p, q = sqnorms(X), sqnorms(Y)
    f = c_transform_sample(X, Y, p, q)
    g = torch.zeros(C5_N, dtype=torch.float64, device=dev)
    sync()
    return X, Y, p, q, f, g


def c_transform_sample(X, Y, p, q, sample=4096):
    """Duals of a refinement-like state: g = 0 and f_i = min_j c_ij over `sample` sampled resident rows (a
    c-transform estimate), so a few hundred pairs per row have sigma > 0."""
    gen = torch.Generator(device=X.device)
    gen.manual_seed(13)
    idx = torch.randperm(Y.shape[0], device=X.device, generator=gen)[:sample]
    Ys = Y[idx]
    f = torch.empty(X.shape[0], dtype=torch.float64, device=X.device)
    for s in range(0, X.shape[0], 4096):
        dots = (X[s:s + 4096] @ Ys.T).double()
        f[s:s + 4096] = (p[s:s + 4096, None] + q[idx][None, :] - 2.0 * dots).min(1).values
    return f


def bench_c5(dev, chunk, steps, warmup, inputs=None, precision="auto", keep=None):
    """One C5 pricing step timed over `steps` runs; with `keep` (a list) the last run's row and column outputs
    are appended to it. The resident side (the 1.28M rows: norms, sweep copy, int8 scales) is prepared once before
    the timed steps, as the reference places its resident side once per chunked scan
    (kernels/bilinear_topk.py:255-293); its preparation time is reported in the detail."""
    from hello_ot_amd import _lib
    from hello_ot_amd.kernels.generic_scan import ResidentSide, pricing_l2sq, sweep_precision

    X, Y, p, q, f, g = c5_inputs(dev, chunk) if inputs is None else inputs
    qb, db = f - p, g - q
    k = 2
    sync()
    t0 = time.perf_counter()
    side = ResidentSide(Y, sweep_precision(precision, C5_D))
    sync()
    prepare_s = time.perf_counter() - t0

    def step():
        return pricing_l2sq(X, Y, p, q, qb, db, k, dot_scale=2.0, rows=True, cols=True, stats=True, linf=True,
                            resident=side)

    log(f"[bench] C5 chunk {chunk} x {C5_N}, d={C5_D}, k={k}: warmup {warmup}, steps {steps}")
    for _ in range(warmup):
        step()
    sync()
    _lib.profile_reset()
    _lib.profile_enable(True)
    t0 = time.perf_counter()
    for _ in range(steps):
        out = step()
    sync()
    sec = (time.perf_counter() - t0) / steps
    sweep_ms, sweeps = _lib.profile_query("l2sq_sweep")
    fin_ms, fins = _lib.profile_query("l2sq_finalize")
    res_ms, _ = _lib.profile_query("l2sq_rescan")
    _lib.profile_enable(False)
    pairs = chunk * C5_N
    sweep_avg = sweep_ms / max(sweeps, 1) / 1e3
    achieved = 2.0 * C5_D * pairs / sweep_avg
    st = out[4].cpu().numpy()
    info = {
        "sweep_ms_avg": sweep_ms / max(sweeps, 1), "sweep_launches": sweeps,
        "finalize_ms_avg": fin_ms / max(fins, 1), "rescan_ms_total": res_ms,
        "positive_pairs": float(st[2]), "max_violation": float(st[3]),
        "resident_prepare_ms": prepare_s * 1e3,
    }
    if keep is not None:
        keep.extend(t.clone() for t in out[:4])
    del qb, db, out, side
    return sec, pairs, achieved, info


def cpu_baseline_c5(dev, sample_rows=4096, sample_cols=196608, threads=16):
    """Reference CPU backend path (cpp_scan.fused_dot_tile: torch.mm fp32 dots + _scan.dot_tile epilogue,
    kernels/cpp_scan.py:9-21, _native/cpp/scan.cpp:136-227) on a sample of the C5 pricing work."""
    import oracle

    threads = min(threads, os.cpu_count() or 1)
    torch.set_num_threads(threads)
    Xd = gmm(sample_rows, C5_D, seed=1, dev=dev, means_seed=11)
    Yd = gmm(sample_cols, C5_D, seed=2, dev=dev, means_seed=12)
    pd_, qd = sqnorms(Xd), sqnorms(Yd)
    # the same kind of duals as the GPU step: f from a sampled c-transform, g = 0
    fd = c_transform_sample(Xd, Yd, pd_, qd)
    X, Y = Xd.cpu(), Yd.cpu()
    p, q, f = pd_.cpu().numpy(), qd.cpu().numpy(), fd.cpu().numpy()
    g = np.zeros(sample_cols)
    sc = oracle.ref_scan()
    k = 2
    rv = np.full((sample_rows, k), -np.inf)
    ri = np.full((sample_rows, k), -1, np.int64)
    cv = np.full((sample_cols, k), -np.inf)
    ci = np.full((sample_cols, k), -1, np.int64)
    if sc is not None:
        kind = "reference"
        tile = 8192
        t0 = time.perf_counter()
        for s in range(0, sample_cols, tile):
            dots = torch.mm(X, Y[s:s + tile].T).numpy()
            cvv = np.ascontiguousarray(cv[s:s + tile])
            cii = np.ascontiguousarray(ci[s:s + tile])
            sc.dot_tile(dots, p, q[s:s + tile], f, g[s:s + tile], rv, ri, cvv, cii, 2.0, 0, s, 0, threads)
            cv[s:s + tile], ci[s:s + tile] = cvv, cii
        sec = time.perf_counter() - t0
        agreement = _agreement_with_reference(Xd, Yd, pd_, qd, fd, rv, ri, cv, ci, k)
    else:
        kind = "port"
        agreement = None
        sample_cols = 4096
        Y = Y[:sample_cols]
        q = q[:sample_cols]
        t0 = time.perf_counter()
        oracle.l2sq_scan(X.numpy(), Y.numpy(), p, q, f - p, g[:sample_cols] - q, k, 2.0)
        sec = time.perf_counter() - t0
    del Xd, Yd
    pairs = sample_rows * sample_cols
    return {"value": pairs / sec, "unit": "pairs/s", "cores": threads, "kind": kind,
            "agreement_with_gpu": agreement,
            "sample": f"{sample_rows} query x {sample_cols} resident rows of the C5 mixture, d={C5_D}, k=2, "
                      f"bidirectional + certificate, sampled c-transform duals as the GPU step ({sec:.1f} s)",
            **host_info()}


def _agreement_with_reference(Xd, Yd, pd_, qd, fd, rv, ri, cv, ci, k):
    """The GPU step on the CPU baseline's sample against the reference CPU path's own lists: the share of rows and
    columns whose top-k index lists are identical, and the largest score difference over the entries both name
    (same pair). The reference ranks by scores from fp32 dot products (torch.mm) with a (f + g) - cost epilogue; the
    GPU ranks by exact fp64 scores (scale * dot64 + (f - p)) + (g - q), so lists differ where near-equal scores trade
    places under the fp32 dot error."""
    from hello_ot_amd.kernels.generic_scan import pricing_l2sq

    g = torch.zeros(len(Yd), dtype=torch.float64, device=Yd.device)
    out = pricing_l2sq(Xd, Yd, pd_, qd, fd - pd_, g - qd, k, dot_scale=2.0, rows=True, cols=True, stats=False)
    grv, gri, gcv, gci = (t.cpu().numpy() for t in out[:4])

    def share(a, b):
        return float((a == b).all(axis=1).mean())

    def spread(a, ia, b, ib):
        same = (ia == ib) & np.isfinite(a) & np.isfinite(b)
        return float(np.max(np.abs(a - b)[same])) if same.any() else None

    return {"rows_identical": share(gri, ri), "columns_identical": share(gci, ci),
            "row_score_max_abs_diff": spread(grv, gri, rv, ri), "column_score_max_abs_diff": spread(gcv, gci, cv, ci),
            "score_magnitude": float(np.max(np.abs(rv[np.isfinite(rv)]))) if np.isfinite(rv).any() else None}


# ----------------------------------------------------------------------------------------------------------
# extras: C2, C3, C4
# ----------------------------------------------------------------------------------------------------------

def bench_library_gemm(dev, warmup=10, steps=40):
    """Reference point for the sweep's MFMA rate: the vendor library's plain bf16 GEMM (`torch.matmul`, which
    calls hipBLASLt) on the sweep's product shape, the 8192-row query chunk times 131072 resident rows at
    d = 8192, bf16 in and out, timed with events on torch's stream after a warm-up long enough to reach the
    sustained clock. It computes one product per pair; the split sweep computes three plus the selection."""
    m, n, d = 8192, 131072, C5_D
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    A = torch.randn(m, d, device=dev, dtype=torch.bfloat16, generator=gen)
    B = torch.randn(d, n, device=dev, dtype=torch.bfloat16, generator=gen)
    C = torch.empty(m, n, device=dev, dtype=torch.bfloat16)
    for _ in range(warmup):
        torch.matmul(A, B, out=C)
    sync()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        torch.matmul(A, B, out=C)
    end.record()
    sync()
    sec = start.elapsed_time(end) / 1e3 / steps
    flops = 2.0 * m * n * d
    del A, B, C
    torch.cuda.empty_cache()
    return {"shape_m_n_d": [m, n, d], "ms": sec * 1e3, "tflops": flops / sec / 1e12,
            "frac_of_bf16_peak": flops / sec / PEAK_BF16_MFMA}


def bench_library_int8_gemm(dev, warmup=10, steps=40):
    """Reference point for the int8 sweep's MFMA rate: the vendor library's plain int8 GEMM (`torch._int_mm`, int8
    in, int32 out, hipBLASLt) on the same product shape, B given column-major (the faster of the two layouts
    measured), timed like the bf16 GEMM. It computes one int8 product per pair; the int8 sweep computes three limb
    products plus the selection and the certificate."""
    m, n, d = 8192, 131072, C5_D
    gen = torch.Generator(device=dev)
    gen.manual_seed(6)
    A = torch.randint(-127, 128, (m, d), device=dev, dtype=torch.int8, generator=gen)
    B = torch.randint(-127, 128, (n, d), device=dev, dtype=torch.int8, generator=gen).t()
    for _ in range(warmup):
        C = torch._int_mm(A, B)
    sync()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        C = torch._int_mm(A, B)
    end.record()
    sync()
    sec = start.elapsed_time(end) / 1e3 / steps
    ops = 2.0 * m * n * d
    del A, B, C
    torch.cuda.empty_cache()
    return {"shape_m_n_d": [m, n, d], "ms": sec * 1e3, "tops": ops / sec / 1e12,
            "frac_of_int8_peak": ops / sec / PEAK_INT8_MFMA}


def bench_c2(dev, steps=3):
    from hello_ot_amd import _lib
    from hello_ot_amd.kernels.generic_scan import pricing_l2sq, sweep_precision

    m = n = 131072
    d, k = 64, 8
    rng = np.random.default_rng(42)
    X = torch.as_tensor(rng.standard_normal((m, d)).astype(np.float32)).to(dev)
    Y = torch.as_tensor(rng.standard_normal((n, d)).astype(np.float32)).to(dev)
    f = torch.as_tensor(rng.normal(64.0, 2.0, m)).to(dev)
    g = torch.as_tensor(rng.normal(64.0, 2.0, n)).to(dev)
    p, q = sqnorms(X), sqnorms(Y)
    qb, db = f - p, g - q
    out = {}
    for name, kw in (("rows", dict(rows=True, cols=False, stats=False)),
                     ("bidir_stats", dict(rows=True, cols=True, stats=True, linf=True)),
                     ("bidir_stats_bf16x3", dict(rows=True, cols=True, stats=True, linf=True, precision="bf16x3"))):
        fn = lambda: pricing_l2sq(X, Y, p, q, qb, db, k, **kw)  # noqa: E731
        fn()
        sync()
        _lib.profile_reset()
        _lib.profile_enable(True)
        sec = time_steps(fn, steps, 0)
        sw_ms, sw_n = _lib.profile_query("l2sq_sweep")
        _lib.profile_enable(False)
        sweep_s = sw_ms / max(steps, 1) / 1e3   # all sweep launches of one call (one per internal query chunk)
        prec = sweep_precision(kw.get("precision", "auto"), d)
        peak, products = (PEAK_BF16_MFMA, 3.0) if prec == "bf16x3" else (PEAK_FP32_MFMA, 1.0)
        alg = 2 * d * m * n / sweep_s
        out[name] = {"seconds": sec, "pairs_per_s": m * n / sec, "sweep": prec,
                     "sweep_launches_per_call": sw_n // max(steps, 1), "sweep_ms_per_call": sweep_s * 1e3,
                     "sweep_algorithmic_tflops": alg / 1e12, "peak_tflops": peak / 1e12,
                     "sweep_algorithmic_frac": alg / peak, "sweep_executed_frac": products * alg / peak}
    return out


def _c3_csr(rng, m, n, per_row):
    """CSR with `per_row` distinct uniformly random columns per row, sorted within each row."""
    cols = np.empty((m, per_row), np.int64)
    todo = np.arange(m)
    while todo.size:
        draw = np.sort(rng.integers(0, n, (todo.size, per_row + 8)), axis=1)
        dup = np.zeros_like(draw, bool)
        dup[:, 1:] = draw[:, 1:] == draw[:, :-1]
        ok = (~dup).sum(1) >= per_row
        prio = rng.random(draw.shape)
        prio[dup] = np.inf
        pick = np.argsort(prio, axis=1)[:, :per_row]  # a uniform subset of the distinct draws
        chosen = np.sort(np.take_along_axis(draw, pick, axis=1), axis=1)
        cols[todo[ok]] = chosen[ok]
        todo = todo[~ok]
    rowptr = np.arange(0, m * per_row + 1, per_row, dtype=np.int32)
    return rowptr, cols.reshape(-1).astype(np.int32)


def bench_c3(dev):
    from hello_ot_amd import _lib
    from hello_ot_amd.costs.pairs import lowrank_csr_costs
    from hello_ot_amd.lp import NativeRestrictedOTPDLP

    m = n = 262144
    d, per = 256, 16
    rng = np.random.default_rng(3)
    X = torch.as_tensor(rng.standard_normal((m, d)).astype(np.float32)).to(dev)
    Y = torch.as_tensor(rng.standard_normal((n, d)).astype(np.float32)).to(dev)
    rowptr, col = _c3_csr(rng, m, n, per)
    nnz = col.size
    p, q = sqnorms(X), sqnorms(Y)
    trp, tcol = torch.as_tensor(rowptr).to(dev), torch.as_tensor(col).to(dev)
    costs = lowrank_csr_costs(X, Y, p, q, trp, tcol)
    sync()
    _lib.profile_reset()
    _lib.profile_enable(True)
    reps = 5
    for _ in range(reps):
        costs = lowrank_csr_costs(X, Y, p, q, trp, tcol)
    sync()
    sd_ms, sd_n = _lib.profile_query("sddmm_l2sq_csr")
    sd_s = sd_ms / max(sd_n, 1) / 1e3
    gather_bytes = m * d * 4 + nnz * d * 4 + nnz * (4 + 8) + (m + 1) * 4 + (m + n) * 8
    rows = torch.as_tensor(np.repeat(np.arange(m), per)).to(dev)
    a = torch.full((m,), 1.0 / m, dtype=torch.float64, device=dev)
    b = torch.full((n,), 1.0 / n, dtype=torch.float64, device=dev)
    solver = NativeRestrictedOTPDLP(device=dev, evaluation_frequency=200, iteration_limit=1000)
    # the solve timed as a caller runs it (no per-iteration events), then once more with the per-iteration
    # HIP-event profile for the iteration's own duration
    _lib.profile_enable(False)
    solver.solve_restricted(rows=rows, cols=tcol, costs=costs, source_mass=a, target_mass=b, tolerance=0.0)
    sync()
    t0 = time.perf_counter()
    r = solver.solve_restricted(rows=rows, cols=tcol, costs=costs, source_mass=a, target_mass=b, tolerance=0.0)
    sync()
    pd_s = time.perf_counter() - t0
    _lib.profile_reset()
    _lib.profile_enable(True)
    solver.solve_restricted(rows=rows, cols=tcol, costs=costs, source_mass=a, target_mass=b, tolerance=0.0)
    sync()
    it_ms, it_n = _lib.profile_query("pdhg_iteration")
    _lib.profile_enable(False)
    E, V = nnz, m + n
    iter_bytes = 120 * E + 76 * V
    it_s = it_ms / max(it_n, 1) / 1e3
    return {
        "sddmm_ms": sd_s * 1e3, "sddmm_gather_model_GBps": gather_bytes / sd_s / 1e9,
        "sddmm_hbm_frac_gather_model": gather_bytes / sd_s / PEAK_HBM,
        "pdhg_1000_iterations_s": pd_s, "pdhg_device_loop_s": r.solver_diag["device_loop_sec"],
        "pdhg_iteration_us": it_s * 1e6, "pdhg_model_GBps": iter_bytes / it_s / 1e9,
        "pdhg_hbm_frac_model": iter_bytes / it_s / PEAK_HBM, "pdhg_iterations": r.iterations,
        "pdhg_restarts": r.solver_diag["restart_count"], "pdhg_objective": r.obj_val,
    }


def bench_c4(dev):
    from hello_ot_amd import _lib
    from hello_ot_amd.kernels.generic_scan import pricing_norm

    m = n = 524288
    d = 8
    rng = np.random.default_rng(4)
    X = torch.as_tensor(rng.random((m, d)).astype(np.float32)).to(dev)
    Y = torch.as_tensor(rng.random((n, d)).astype(np.float32)).to(dev)
    f = torch.as_tensor(rng.normal(1.2, 0.1, m)).to(dev)
    g = torch.as_tensor(rng.normal(1.2, 0.1, n)).to(dev)
    out = {}
    for kind, name in ((0, "l1"), (1, "linf")):
        pricing_norm(X, Y, f, g, 2, kind)
        sync()
        _lib.profile_reset()
        _lib.profile_enable(True)
        t0 = time.perf_counter()
        pricing_norm(X, Y, f, g, 2, kind)
        sync()
        sec = time.perf_counter() - t0
        sw_ms, sw_n = _lib.profile_query("norm_sweep")
        _lib.profile_enable(False)
        out[name] = {"bidir_stats_seconds": sec, "pairs_per_s": m * n / sec, "sweep_launches": sw_n,
                     "sweep_ms_total": sw_ms, "valu_counters": norm_counters(name)}
    return out


def _level_summary(result):
    out = []
    for level in result.solve_stage.levels:
        if level.kind == "refined":
            its = level.solve.iterations
            pdhg = sum(int(i.solve_lp.backend_iterations or 0) for i in its)
            lp = sum(i.solve_lp.wall_time for i in its)
            out.append({"n": level.n_source, "m": level.n_target, "iterations": len(its),
                        "seconds": round(level.wall_time, 3),
                        "lp_seconds": round(lp, 3), "pdhg_iterations": pdhg,
                        "lp_us_per_pdhg_iteration": round(lp / pdhg * 1e6, 1) if pdhg else None,
                        "scan_seconds": round(sum(i.full_scan_time for i in its), 3),
                        "init_seconds": round(level.initialization.wall_time, 3)})
        else:
            out.append({"n": level.n_source, "m": level.n_target, "coarsest": True, "seconds": round(level.wall_time, 3)})
    return out


def bench_solves(dev):
    """Solve seconds of the full HELLO loop: C1 (Brenier, m=n=2048, d=32, examples/quickstart.py:83-94) and C4
    (l1 and linf, m=n=524288, d=8, U[0,1]^8 features, U(0.5,1.5) masses normalised, seed 4), tolerance 1e-6."""
    from hello_ot_amd import SolverOptions, solve

    out = {}
    rng = np.random.default_rng(42)
    n, dim = 2048, 32
    src = rng.normal(size=(n, dim)).astype(np.float32)
    mapped = src + np.float32(2.0) * np.tanh(src)
    tgt = mapped[rng.permutation(n)]
    truth = float(np.mean(np.sum((src.astype(np.float64) - mapped.astype(np.float64)) ** 2, axis=1)))
    solve(src, tgt, options=SolverOptions(verbose="off"))  # warm-up (library load, first kernels)
    r = solve(src, tgt, options=SolverOptions(verbose="off"))
    out["c1_brenier_2048_d32"] = {"seconds": r.total_wall_time, "objective": r.objective,
                                  "closed_form": truth, "rel_error": abs(r.objective - truth) / truth,
                                  "levels": _level_summary(r)}
    rng = np.random.default_rng(4)
    m = 524288
    X = torch.as_tensor(rng.random((m, 8)).astype(np.float32)).to(dev)
    Y = torch.as_tensor(rng.random((m, 8)).astype(np.float32)).to(dev)
    a, b = rng.uniform(0.5, 1.5, m), rng.uniform(0.5, 1.5, m)
    a, b = a / a.sum(), b / b.sum()
    for kind in ("l1", "linf"):
        log(f"[bench] C4 solve {kind} ...")
        r = solve(X, Y, source_mass=a, target_mass=b, cost=kind, options=SolverOptions(verbose="off"))
        finest = r.solve_stage.levels[-1].solve.summary
        out[f"c4_{kind}_524288_d8"] = {"seconds": r.total_wall_time, "objective": r.objective,
                                       "converged": bool(finest.converged),
                                       "peak_gpu_memory_mib": r.peak_gpu_memory_mib,
                                       "refinement_iterations": r.metadata["total_refinement_iterations"],
                                       "levels": _level_summary(r)}
    return out


def bench_c5_solve(dev, rows, stream="auto"):
    """C5 full solve: rows x 8192 fp32 on each side from independent 64-component Gaussian mixtures (means
    ~ N(0, 4I), identity covariance, equal weights), uniform masses, squared-Euclidean cost, default options,
    tolerance 1e-6; the sides are reordered in place (consume_input_features).

    ``stream``: "auto" hands both sides over on the device and lets the solver's memory planner choose (at C5 on
    one MI355X both sides stay resident); "always" hands the source side over in host memory and streams it, which
    bounds the device memory (the reference's non-resident path and its 41.6 GiB figure)."""
    from hello_ot_amd import SolverOptions, _lib, solve
    from hello_ot_amd.resident import host as host_module

    log(f"[bench] C5 solve ({stream}): generating {rows} x {C5_D} per side "
        f"({2 * rows * C5_D * 4 / 2**30:.1f} GiB) ...")
    X = gmm_host(rows, C5_D, seed=1, dev=dev, means_seed=11) if stream == "always" else \
        gmm(rows, C5_D, seed=1, dev=dev, means_seed=11)
    Y = gmm(rows, C5_D, seed=2, dev=dev, means_seed=12)
    sync()
    torch.cuda.empty_cache()
    log(f"[bench] C5 solve ({stream}): solving ...")
    policy = host_module.STREAM_POLICY
    host_module.STREAM_POLICY = stream
    # the library's kernel timing on for the PDHG iterations' own device time (HIP events around each iteration)
    _lib.profile_reset()
    _lib.profile_enable(True)
    try:
        r = solve(X, Y, options=SolverOptions(verbose="detailed", consume_input_features=True))
    finally:
        host_module.STREAM_POLICY = policy
        _lib.profile_enable(False)
    del X, Y
    torch.cuda.empty_cache()
    finest = r.solve_stage.levels[-1].solve.summary
    return {"rows": rows, "d": C5_D, "seconds": r.total_wall_time, "objective": r.objective,
            "streamed_source": bool(r.metadata["streamed_source"]),
            "converged": bool(finest.converged),
            "final_dual_infeasibility": r.solve_stage.levels[-1].solve.iterations[-1].convergence.dual_feasibility,
            "peak_gpu_memory_gib": r.peak_gpu_memory_mib / 1024.0,
            "refinement_iterations": r.metadata["total_refinement_iterations"],
            "scan_seconds": r.metadata["total_scan_time"], "lp_seconds": r.metadata["total_lp_solve_time"],
            "init_seconds": sum(l.initialization.wall_time for l in r.solve_stage.levels
                                if l.kind == "refined" and l.initialization is not None),
            "finest_pdhg": _finest_pdhg(r),
            "levels": _level_summary(r)}


def _finest_pdhg(result):
    """The finest level's PDHG: iterations, seconds inside hm_pdhg_solve, the iterations' own average device time
    (HIP events) and that time against the 120 E + 76 V byte model of one iteration (E: the level's final support,
    V: its nodes)."""
    device = next((d for d in result.metadata.get("lp_device_by_level", []) if d["level"] == 0), None)
    finest = result.solve_stage.levels[-1]
    if device is None or not device.get("passes"):
        return None
    E = int(finest.solve.summary.final_active_support_size)
    V = finest.n_source + finest.n_target
    us = device["pass_ms"] / device["passes"] * 1e3
    return {"iterations": device["iterations"], "hm_pdhg_solve_seconds": round(device["seconds"], 3),
            "pass_us": round(us, 1), "edges": E, "nodes": V,
            "model_bytes_per_iteration": 120 * E + 76 * V,
            "hbm_frac_model": (120 * E + 76 * V) / (us * 1e-6) / PEAK_HBM}


# ----------------------------------------------------------------------------------------------------------

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--chunk", type=int, default=8192, help="query rows per step against the 1.28M resident rows")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--no-c5-solve", action="store_true",
                    help="skip the full C5 solve (1.28M x 1.28M, d=8192) that the default run times last")
    ap.add_argument("--sweep", default="auto", choices=("auto", "fp32", "bf16x3", "int8x3"),
                    help="sweep precision of the C5 step (all give the same exact lists)")
    ap.add_argument("--fp32-sweep", action="store_true",
                    help="also time the C5 step on the fp32 MFMA sweep and check its outputs against the split sweep")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run a plain 1 GiB device-to-device copy kernel three times (the reference point "
                         "for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes)")
    ap.add_argument("--only", default="", metavar="LIST",
                    help="instead of the default run, run only the listed secondary workloads (comma-separated: "
                         "c2, c3, c4) and print their figures as one JSON line (for counter passes)")
    ap.add_argument("--c5-solve", type=int, default=0, metavar="ROWS",
                    help="instead of the default run, solve the C5 instance with ROWS points per side "
                         "(1280000 = the full instance) and print its JSON line")
    ap.add_argument("--stream", default="auto", choices=("auto", "always", "never"),
                    help="with --c5-solve: where the source side lives (auto: the solver's memory planner; always: "
                         "host memory, streamed; never: on the device)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        if int(os.environ.get("RANK", "0")) == 0:
            print("bench.py measures one MI355X: this build runs the hot path on a single GPU "
                  "(multi-GPU sharding is a design note, not an implemented path).", file=sys.stderr)
        sys.exit(2)
    from hello_ot_amd import _lib

    _lib.load()
    dev = torch.device("cuda", 0)
    if args.copy_calibration:
        src = torch.ones(2**28, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        sync()
        log("[bench] copy calibration: 3 x 1 GiB read + 1 GiB written")
        del src, dst
    if args.only:
        names = [x.strip() for x in args.only.split(",") if x.strip()]
        runs = {"c2": ("c2_scan_131072x131072_d64_k8", bench_c2), "c3": ("c3_sddmm_pdhg_262144_d256", bench_c3),
                "c4": ("c4_norm_scan_524288_d8", bench_c4), "solves": ("solve_seconds", bench_solves)}
        bad = [x for x in names if x not in runs]
        if bad:
            raise SystemExit(f"--only: unknown workload(s) {bad}; choose from {sorted(runs)}")
        extras = {}
        for x in names:
            log(f"[bench] {x} ...")
            extras[runs[x][0]] = runs[x][1](dev)
        print(json.dumps({"only": names, "extras": extras}), flush=True)
        return
    if args.c5_solve:
        print(json.dumps({"metric": "C5 solve seconds to relative dual infeasibility 1e-6 (l2^2, d=8192)",
                          **bench_c5_solve(dev, args.c5_solve, stream=args.stream)}), flush=True)
        return
    from hello_ot_amd.kernels.generic_scan import sweep_precision

    inputs = c5_inputs(dev, args.chunk)
    precision = sweep_precision(args.sweep, C5_D)
    split_out = []
    sec, pairs, achieved, info = bench_c5(dev, args.chunk, args.steps, args.warmup, inputs, precision, split_out)
    extras = {}
    if args.fp32_sweep and precision != "fp32":
        # the same step on the fp32 MFMA sweep (identical outputs), against the fp32 matrix peak
        log("[bench] C5 step on the fp32 sweep ...")
        fp32_out = []
        s32, _, a32, i32 = bench_c5(dev, args.chunk, args.steps, 0, inputs, "fp32", fp32_out)
        # the exact fp64 re-check makes both sweeps' row and column lists (values and indices) identical
        same = all(bool(torch.equal(a, b)) for a, b in zip(split_out, fp32_out))
        extras["c5_step_fp32_sweep"] = {"pairs_per_s": pairs / s32, "ms_per_step": s32 * 1e3,
                                        "sweep_ms_avg": i32["sweep_ms_avg"], "sweep_tflops": a32 / 1e12,
                                        "sweep_frac_of_fp32_peak": a32 / PEAK_FP32_MFMA,
                                        "outputs_identical_to_split_sweep": same}
        del fp32_out
    del inputs, split_out
    torch.cuda.empty_cache()
    if not args.no_extras:
        log("[bench] hipBLASLt bf16 GEMM of the sweep's product shape ...")
        extras["library_bf16_gemm_same_shape"] = bench_library_gemm(dev)
        log("[bench] hipBLASLt int8 GEMM of the sweep's product shape ...")
        extras["library_int8_gemm_same_shape"] = bench_library_int8_gemm(dev)
        log("[bench] C2 ...")
        extras["c2_scan_131072x131072_d64_k8"] = bench_c2(dev)
        log("[bench] C3 ...")
        extras["c3_sddmm_pdhg_262144_d256"] = bench_c3(dev)
        log("[bench] C4 ...")
        extras["c4_norm_scan_524288_d8"] = bench_c4(dev)
        log("[bench] solves (C1, C4) ...")
        extras["solve_seconds"] = bench_solves(dev)
    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] CPU baseline ...")
        cpu = cpu_baseline_c5(dev)
    solve_c5 = solve_c5_streamed = None
    if not args.no_c5_solve:
        torch.cuda.empty_cache()
        solve_c5 = bench_c5_solve(dev, C5_N)
        solve_c5_streamed = bench_c5_solve(dev, C5_N, stream="always")
    line = {
        "metric": "pricing pairs/s (l2^2 bidirectional scan + certificate, m=n=1.28M d=8192)",
        "value": pairs / sec,
        "unit": "pairs/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": sec * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"bf16x3": "bf16x3+f64", "int8x3": "int8x3+f64"}.get(precision, "f32+f64"),
        "data": "synthetic 64-component Gaussian mixtures (C5 recipe), generated on device",
        "config": {"workload": f"C5 pricing step: {args.chunk} query rows x 1,280,000 resident rows, d=8192, k=2, "
                               "rows+cols top-k + certificate", "chunk": args.chunk, "n_resident": C5_N,
                   "d": C5_D, "k": 2},
        "roofline": roofline(precision, achieved),
        "cpu_baseline": cpu,
        "solve_seconds": {"c5": solve_c5, "c5_streamed_source": solve_c5_streamed},
        "detail": info,
        "extras": extras,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
