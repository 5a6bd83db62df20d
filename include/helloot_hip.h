/*
 * helloot_hip.h -- C ABI of the MI355X (gfx950) HELLO hot path.
 *
 * Conventions
 *   - Every array argument is a DEVICE pointer (e.g. torch.Tensor.data_ptr() of a ROCm tensor) unless the
 *     parameter comment says "host".
 *   - `stream` is a hipStream_t passed as void* (0 = the legacy default stream). All work is ordered on
 *     that stream. Functions that must read a device scalar back to decide what to launch next say so.
 *   - Outputs are caller-allocated. Scratch memory comes from `workspace` (device, 256-byte aligned,
 *     size from the matching *_workspace_bytes() query). Nothing here calls hipMalloc.
 *   - Return value: HM_OK (0) or an HM_E* code; hm_last_error() then describes the failure (thread-local).
 *     No function aborts the process (the reference's CuPDLPx exits on CUDA errors, cupdlpx/utils.h:104-138).
 *   - Scores follow the reference's dual score sigma_ij = f_i + g_j - c_ij ("reduced cost" r_ij = -sigma_ij);
 *     candidate lists are sorted by sigma descending, ties to the lowest index, missing slots (-inf, -1).
 */
#ifndef HELLOOT_HIP_H
#define HELLOOT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HM_OK 0
#define HM_EINVAL 1   /* invalid argument (ValueError in the Python mirror) */
#define HM_EHIP 2     /* HIP runtime / launch error (RuntimeError) */
#define HM_ENOSPC 3   /* workspace too small (RuntimeError) */
#define HM_ESOLVE 4   /* a solver stopped without an optimum (RuntimeError) */

/* Pricing flags */
#define HM_ROWS 1u    /* per-row (query-side) top-k */
#define HM_COLS 2u    /* per-column (database-side) top-k */
#define HM_STATS 4u   /* certificate sums num, den, count, max */
#define HM_LINF 8u    /* also max|cost| (collect_linf_stats) */
#define HM_BF16X3 16u /* l2^2 sweep on split-bf16 MFMA (hi*hi + hi*lo + lo*hi) instead of fp32 MFMA; same outputs */
#define HM_INT8X3 32u /* l2^2 sweep on int8 MFMA over a 16-bit fixed-point split (h*h + h*l + l*h); same outputs */
#define HM_FP64 64u   /* norm scans: fp64 costs (compute_precision = 1 of the reference, direct_norm_fp64) */

/* Norm cost kinds (generic_scan.py cost_type: 0=l1, 1=linf, 2=l2) */
#define HM_COST_L1 0
#define HM_COST_LINF 1
#define HM_COST_L2 2

const char* hm_last_error(void);
int hm_abi_version(void); /* 1 */

/*
 * Kernel timing. No reference counterpart: the reference returns a zeroed timing slot
 * (generic_scan.py:577-597, "collect_timing"). When enabled, every hot-path launch is bracketed by HIP
 * events on its own stream; hm_profile_query waits for the pending events and returns the accumulated
 * milliseconds and launch count for one kernel name: "l2sq_sweep", "l2sq_finalize", "l2sq_col_finalize",
 * "l2sq_wide" (wide pass of uncertified rows), "l2sq_rescan" (exact full rescan), "norm_sweep",
 * "sddmm_l2sq_csr", "pdhg_iteration" (passes of one PDHG iteration). Counters without timing report their
 * total in `launches` (total_ms = 0): "l2sq_wide_rows" / "l2sq_wide_columns" (rows / columns sent to the wide
 * pass) and "l2sq_rescan_rows" / "l2sq_rescan_columns" (rows / columns rescanned in full).
 */
void hm_profile_enable(int on);
void hm_profile_reset(void);
int hm_profile_query(const char* name, double* total_ms, int64_t* launches);

/* ---------------------------------------------------------------------------------------------------- */
/* (a) Full-space pricing scan                                                                           */
/* ---------------------------------------------------------------------------------------------------- */

/*
 * l2^2 ("raw lowrank") bidirectional pricing scan with the full-edge certificate.
 * Replaces ScanExtension.fused_bidir_topk_stats_raw (kernels/generic_scan.py:577-597), i.e. the native
 * modules pricing_small.raw_scan_tiled (pricing_small.cu:281-304) and pricing.scan + merge
 * (pricing.cu:185-229) with their cuBLAS SGEMM tiles.
 *
 *   sigma_ij = (scale*<x_i,y_j> + qb_i) + db_j,   c_ij = (p_i + q_j) - scale*<x_i,y_j>
 *   X: m x d fp32 row-major, Y: n x d fp32 row-major; p, q (query_cost/db_cost), qb = f - p, db = g - q fp64.
 *   scale (dot_scale) must be 1 or 2.  1 <= k <= 32.
 * Outputs (each may be NULL when its flag is off):
 *   row_val[m*k] fp64, row_idx[m*k] int32  -- per X row, best k columns (HM_ROWS)
 *   col_val[n*k] fp64, col_idx[n*k] int32  -- per Y row, best k X rows    (HM_COLS)
 *   stats[5] fp64 = (num = sum sigma+^2, den = sum c^2, count #{sigma>0}, max sigma+, max|c| (HM_LINF))
 * Values are exact fp64 re-evaluations (fixed-order fp64 dot) of candidates found by an MFMA sweep (fp32,
 * split-bf16 with HM_BF16X3, or the int8 split with HM_INT8X3, d <= 65536) with a rigorous error bound b. A row whose kept candidates cannot be separated
 * from the dropped ones by 2b goes through a wide pass (its candidates with approximate score >= k-th - 2b are
 * collected by a second sweep and evaluated exactly) and, past 512 such candidates, an exact full rescan.
 * Certificate: the maximum violation is the exact fp64 maximum (from the row lists, computed internally when
 * HM_ROWS is off); count and num use the sweep's fp32-accumulated dot with an fp64 score for every pair within
 * the fp32 rounding slack of zero (the reference's arithmetic: fp32 dots, fp64 epilogue); den and max|c| are
 * accumulated from fp32 costs. The call synchronises the stream once per finalize to read the number of queued
 * rows back.
 */
size_t hm_pricing_l2sq_workspace_bytes(int64_t m, int64_t n, int32_t d, int32_t k, uint32_t flags);
int hm_pricing_l2sq(void* stream, const float* X, const float* Y, const double* p, const double* q,
                    const double* qb, const double* db, int64_t m, int64_t n, int32_t d, int32_t k,
                    double scale, uint32_t flags, double* row_val, int32_t* row_idx, double* col_val,
                    int32_t* col_idx, double* stats, void* workspace, size_t workspace_bytes);

/*
 * Resident side of an l2^2 scan. The reference's chunked check places one side on the device once and streams
 * query chunks against it (kernels/bilinear_topk.py:255-293, the plan of kernels/scan_contract.py:113-211);
 * hm_l2sq_resident_prepare does the same for Y: its fp64 norms, its sweep copy for the precision bits of
 * `flags` (HM_BF16X3 / HM_INT8X3 / neither) and, for the int8 sweep, its scales and error terms, into a
 * caller-allocated buffer of hm_l2sq_resident_bytes(n, d, flags) bytes. hm_pricing_l2sq_resident is then
 * hm_pricing_l2sq for one query chunk X against that Y (same arguments and outputs; Y must be the tensor the
 * side was prepared from, unchanged, and `flags` must carry the same precision bits: otherwise HM_EINVAL), and
 * skips Y's preparation; only Y's biases (db, q + db) are converted per call. Its workspace is
 * hm_pricing_l2sq_resident_workspace_bytes. The call reads the buffer's header back (one stream synchronisation).
 */
size_t hm_l2sq_resident_bytes(int64_t n, int32_t d, uint32_t flags);
int hm_l2sq_resident_prepare(void* stream, const float* Y, int64_t n, int32_t d, uint32_t flags, void* resident,
                             size_t resident_bytes);
size_t hm_pricing_l2sq_resident_workspace_bytes(int64_t m, int64_t n, int32_t d, int32_t k, uint32_t flags);
int hm_pricing_l2sq_resident(void* stream, const float* X, const float* Y, const double* p, const double* q,
                             const double* qb, const double* db, int64_t m, int64_t n, int32_t d, int32_t k,
                             double scale, uint32_t flags, double* row_val, int32_t* row_idx, double* col_val,
                             int32_t* col_idx, double* stats, const void* resident, size_t resident_bytes,
                             void* workspace, size_t workspace_bytes);

/*
 * hm_pricing_l2sq_resident with a floor per column: col_floor[n] (fp64, HM_COLS only; NULL = none) holds for each
 * Y row a score that the caller's own running list of that column already reaches k times, and entries whose
 * exact score is below it may then be left out of the column's output (padded with -inf / -1). The outputs keep
 * every entry of the column's exact top k that scores at least the floor, so merging them into the caller's lists
 * gives the same lists as without a floor. No counterpart in the reference, whose streamed chunks merge full
 * per-chunk lists (kernels/bilinear_topk.py:255-368, torch.topk): it is for a caller that streams the X side in
 * chunks and keeps the column lists across them, where the floor lets each chunk skip the exact re-evaluation of
 * columns that the chunk cannot change. col_floor = NULL is hm_pricing_l2sq_resident.
 */
int hm_pricing_l2sq_resident_floor(void* stream, const float* X, const float* Y, const double* p, const double* q,
                                   const double* qb, const double* db, int64_t m, int64_t n, int32_t d, int32_t k,
                                   double scale, uint32_t flags, const double* col_floor, double* row_val,
                                   int32_t* row_idx, double* col_val, int32_t* col_idx, double* stats,
                                   const void* resident, size_t resident_bytes, void* workspace,
                                   size_t workspace_bytes);

/*
 * Norm-cost (l1 / linf / l2) bidirectional pricing scan on VALU with the full-edge certificate.
 * Replaces ScanExtension.fused_gcost_bidir_certificate (kernels/generic_scan.py:533-543) ->
 * bidirectional(kind 0/1/2) (generic_scan.py:328-405), i.e. pricing.cu scan_kernel (pricing.cu:71-161)
 * and the direct_norm tiles (cost.cu:10-157) for fp32 cost precision.
 *   c_ij = fp32 distance (l1 sum|x-y|, linf max|x-y|, l2 sqrt(sum (x-y)^2), 32-feature chunks),
 *   sigma_ij = (g_j - c_ij) + f_i in fp64. Exact (bit-reproducible) values; no perturbation.
 * With HM_FP64 the costs are fp64 instead, as the reference's compute_precision = 1 (generic_scan.py:166-167 ->
 * direct_norm_fp64, cost.cu:84-104): per pair every feature difference in fp64 from the fp32 inputs, combined in
 * feature order (l1 sum|z|, linf max|z|, l2 sqrt of fma(z, z, acc)); scores and certificate are then fp64 throughout
 * and the column lists come from a second, role-swapped sweep.
 * With k <= 2 and both HM_ROWS and HM_COLS, the column lists come from the row sweep through a candidate buffer in
 * the workspace: hm_pricing_norm_workspace_bytes returns the size with the full buffer. A smaller workspace (at
 * least the two-sweep size, which a too-small call names in its HM_ENOSPC message) gets a smaller buffer or none;
 * the outputs are the same, as they are when the buffer overflows (the columns then come from a second sweep).
 */
size_t hm_pricing_norm_workspace_bytes(int64_t m, int64_t n, int32_t d, int32_t k, uint32_t flags);
int hm_pricing_norm(void* stream, const float* X, const float* Y, const double* f, const double* g,
                    int64_t m, int64_t n, int32_t d, int32_t k, int32_t kind, uint32_t flags,
                    double* row_val, int32_t* row_idx, double* col_val, int32_t* col_idx, double* stats,
                    void* workspace, size_t workspace_bytes);

/*
 * hm_pricing_norm without a workspace and without any allocation. No counterpart in the reference: this entry
 * point is for callers that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Its scratch is a file-scope device array of hm_pricing_norm_noalloc_max_bytes()
 * bytes (64 MiB) per GPU, held until the process ends; calls whose two-sweep workspace exceeds it fail with HM_ENOSPC
 * (524288 x 524288 at d = 8, k = 2 needs 12 MiB), and k <= 2 calls use the row sweep's column buffer only when all
 * of it fits (else two sweeps, same outputs). The scratch of the CURRENT device is used, so the
 * stream must belong to it. Every call on a GPU shares that GPU's array: calls that overlap on one GPU (other host
 * threads, other streams) race. Nothing in the array has to start at zero (the call clears what it accumulates,
 * with a kernel). Kernel timing (hm_profile_enable) records no events for these launches. Same outputs as
 * hm_pricing_norm.
 */
size_t hm_pricing_norm_noalloc_max_bytes(void);
int hm_pricing_norm_noalloc(void* stream, const float* X, const float* Y, const double* f, const double* g,
                            int64_t m, int64_t n, int32_t d, int32_t k, int32_t kind, uint32_t flags,
                            double* row_val, int32_t* row_idx, double* col_val, int32_t* col_idx, double* stats);

/* ---------------------------------------------------------------------------------------------------- */
/* (b) SDDMM cost evaluation on the active support                                                       */
/* ---------------------------------------------------------------------------------------------------- */

/*
 * l2^2 costs on a CSR support: out[e] = (p_i + q_j) - scale*dot64(x_i, y_j) for e in [rowptr[i], rowptr[i+1]).
 * Replaces costs/pairs._cost_pairs_lowrank_batched (pairs.py:221-437, torch.sparse.sampled_addmm at
 * :394-407) and gpu_resident/cost.Cost.pairs (gpu_resident/cost.py:59-71), with fp64 accumulation.
 * rowptr[m+1] int32, col[nnz] int32 (any order within a row).
 */
int hm_sddmm_l2sq_csr(void* stream, const float* X, const float* Y, const double* p, const double* q,
                      const int32_t* rowptr, const int32_t* col, int64_t m, int64_t nnz, int32_t d,
                      double scale, double* out);

/* Same costs for an arbitrary pair list (rows[e], cols[e]) int64, as HierarchicalOTSolver passes new pairs
 * (core/solver.py:331-362). */
int hm_pair_costs_l2sq(void* stream, const float* X, const float* Y, const double* p, const double* q,
                       const int64_t* rows, const int64_t* cols, int64_t count, int32_t d, double scale,
                       double* out);

/* fp64 l1 / linf / l2 pair costs. Replaces fused_gcost_pairs without perturbation
 * (norm_cost_scan_kernel.cu:233-275, costs/metric.py:85-159). */
int hm_pair_costs_norm(void* stream, const float* X, const float* Y, const int64_t* rows,
                       const int64_t* cols, int64_t count, int32_t d, int32_t kind, double* out);

/* fp32 l1 / linf / l2 pair costs, bit-identical to the cost the norm pricing scan ranks with (32-feature chunks
 * accumulated in fp32, chunks combined in order, l2 = sqrt rounded once to fp32), widened to fp64. Replaces the
 * reference's fp32 batched pair costs for cost_precision="fp32" (costs/pairs.py:88-218, costs/metric.py:85-159). */
int hm_pair_costs_norm_fp32(void* stream, const float* X, const float* Y, const int64_t* rows,
                            const int64_t* cols, int64_t count, int32_t d, int32_t kind, double* out);

/* ---------------------------------------------------------------------------------------------------- */
/* (c) Restricted-LP Halpern-PDHG                                                                          */
/* ---------------------------------------------------------------------------------------------------- */

typedef struct {
    int32_t evaluation_frequency;  /* restart / termination checks every this many iterations (200) */
    int32_t rescale;               /* scalar bound/objective rescaling (the NUMERICAL_DIVERGENCE retry) */
    int64_t iteration_limit;
    double tol_objective, tol_primal, tol_dual;
    double time_limit_seconds;
} hm_pdhg_params;

typedef struct {
    int64_t iterations;
    int64_t restarts;
    int32_t reason;                /* 0 UNSPECIFIED, 1 OPTIMAL, 2 ITERATION_LIMIT, 3 NUMERICAL_DIVERGENCE,
                                      4 TIME_LIMIT */
    int32_t pad;
    double primal_objective, dual_objective;
    double abs_primal, rel_primal, abs_dual, rel_dual, rel_gap;
    double primal_weight;
    double seconds;
} hm_pdhg_result;

/*
 * Balanced restricted OT: min c^T x  s.t.  sum_{e: rows[e]=i} x_e = a_i, sum_{e: cols[e]=j} x_e = b_j, x >= 0.
 * Halpern-reflected PDHG with degree-sqrt constraint scaling, variable scale sqrt(2), step 0.998,
 * PID primal-weight restarts and relative L2 KKT termination, as _native/cpp/solver.cpp:39-378 and
 * _internal/lp/torch_restricted_ot.py:105-393 (the same update CuPDLPx runs: cupdlpx/solver.cu:581-715).
 * Replaces TorchRestrictedOTPDLP._solve_once / CppRestrictedOTPDLP._solve_once / CuPDLPxSolver.solve
 * (_internal/lp/cupdlpx.py:658) for one scaling mode; the NUMERICAL_DIVERGENCE retry
 * (restricted_ot_pdlp.py:76-100) is the caller's.
 *   rows[e], cols[e] int64 endpoints; costs[e]; masses[n_source + n_target] (source then target);
 *   x0[e], y0[n_source+n_target] warm start (NULL = zeros). Outputs x_out[e], y_out[nodes] (unscaled).
 * Reads device scalars back to the host at every evaluation (every evaluation_frequency iterations).
 */
size_t hm_pdhg_workspace_bytes(int64_t n_source, int64_t n_target, int64_t e);
int hm_pdhg_solve(void* stream, const int64_t* rows, const int64_t* cols, const double* costs,
                  const double* masses, const double* x0, const double* y0, int64_t n_source,
                  int64_t n_target, int64_t e, const hm_pdhg_params* params /* host */, double* x_out,
                  double* y_out, hm_pdhg_result* result /* host */, void* workspace, size_t workspace_bytes);

/* ---------------------------------------------------------------------------------------------------- */
/* Support sparsification (host)                                                                          */
/* ---------------------------------------------------------------------------------------------------- */

/*
 * Cycle cancelling on a restricted-OT primal until at most target_nnz edges carry flow > zero_tolerance, never
 * increasing the cost c^T x and keeping every row and column sum. Replaces
 * restricted_ot/support_sparsification.py:52 (sparsify_transport_support, engine "cpp_lct") ->
 * _support_sparsifier_ext.sparsify_transport_support (support_sparsifier_lct.cpp:378-555), which the
 * GPU-resident solver calls when the LP's positive support exceeds its cap (gpu_resident/support.py:124-137).
 *   rows[e], cols[e] int64 endpoints (HOST arrays), values[e] fp64 flows (HOST, in/out), costs[e] fp64 (HOST).
 *   A spanning forest of the positive edges is built in edge order; the remaining positive edges enter in edge
 *   order, each pushing flow around its forest cycle in the direction that does not increase the cost until an
 *   edge reaches zero (the first such edge along the path from the entering edge's source leaves). The forest is
 *   a parent-pointer forest with eager updates, O(cycle length) per cycle. The positive count is checked whenever
 *   enough cycles have been cancelled to reach target_nnz, and the work stops once it is reached.
 *   stats[3] (HOST): output nnz, cycles cancelled, tree operations. Flows <= zero_tolerance come back as 0.
 * Runs on the calling thread; touches no device memory.
 */
int hm_sparsify_support(int64_t n_source, int64_t n_target, int64_t e, const int64_t* rows, const int64_t* cols,
                        double* values, const double* costs, int64_t target_nnz, double zero_tolerance,
                        int64_t* stats);

/* ---------------------------------------------------------------------------------------------------- */
/* Exact coarsest level (host)                                                                            */
/* ---------------------------------------------------------------------------------------------------- */

/*
 * Exact optimal vertex and duals of a small dense balanced transport problem, by the primal network simplex with
 * strongly feasible trees (block-search pricing). Replaces the coarsest-level POT call ot.emd(a, b, M, log=True)
 * of the GPU-resident solver (gpu_resident/solver.py:168-191; hierarchy/coarsest.py:38-60), which returns the
 * plan and the duals log["u"], log["v"].
 *   costs[n_source * n_target] row-major fp64, a[n_source], b[n_target] fp64 (HOST arrays, equal totals).
 *   Outputs (HOST): the basic transport arcs basis_rows/cols[] int32 with basis_flows[] (capacity
 *   n_source + n_target entries; *basis_count of them used, degenerate zero flows included), duals u[n_source],
 *   v[n_target] with u_i + v_j = c_ij on basic arcs and u_i + v_j <= c_ij + 1e-12 (max|c| + 1) on all arcs, and the
 *   pivot count (*pivots_out, may be NULL). HM_ESOLVE when no optimum is reached within max_pivots.
 * Runs on the calling thread; touches no device memory.
 */
int hm_transport_simplex(int64_t n_source, int64_t n_target, const double* costs, const double* a, const double* b,
                         int64_t max_pivots, int32_t* basis_rows, int32_t* basis_cols, double* basis_flows,
                         int64_t* basis_count, double* u, double* v, int64_t* pivots_out);

#ifdef __cplusplus
}
#endif

#endif /* HELLOOT_HIP_H */
