// l2^2 pricing scan: C ABI entry points (kernels and the per-K1 drivers live in l2sq_impl.h and the
// pricing_l2sq_k*.hip translation units, compiled in parallel).
#include "l2sq_impl.h"
namespace hm {
int l2sq_run_k8(L2SQ_RUN_ARGS);
int l2sq_run_k16(L2SQ_RUN_ARGS);
int l2sq_run_k40(L2SQ_RUN_ARGS);
namespace {
int run_direction_k(hipStream_t st, const float* X, const float* Y, int64_t m, int64_t n, int d, int k, double scale,
                    bool stats, bool transposed, const double* qb, const double* db, const double* xnorm,
                    const unsigned long long* ymaxima, const float* qb32, const float* db32, const float* p32,
                    const float* ge32, DirPlan plan, Entry* part, double* blockstats, int* redo, int* redo_count,
                    double* out_val, int* out_idx, double* stats_out, int linf, bool want_rows) {
    switch (bucket_k1(k)) {
        case 8:
            return l2sq_run_k8(L2SQ_RUN_PASS);
        case 16:
            return l2sq_run_k16(L2SQ_RUN_PASS);
        default:
            return l2sq_run_k40(L2SQ_RUN_PASS);
    }
}

}  // namespace
}  // namespace hm

using namespace hm;

extern "C" size_t hm_pricing_l2sq_workspace_bytes(int64_t m, int64_t n, int32_t d, int32_t k, uint32_t flags) {
    (void)d;
    if (m < 1 || n < 1 || k < 1 || k > 32) return 0;
    Sizer s;
    double *a, *b, *bs;
    float *c, *e, *f, *g;
    unsigned long long* mx;
    Entry* part;
    int *redo, *rc;
    layout(s, m, n, k, flags, plan_dir(m, n, k), plan_dir(n, m, k), &a, &b, &c, &e, &f, &g, &mx, &part, &bs, &redo, &rc);
    return s.used;
}

extern "C" int hm_pricing_l2sq(void* stream, const float* X, const float* Y, const double* p, const double* q,
                               const double* qb, const double* db, int64_t m, int64_t n, int32_t d, int32_t k,
                               double scale, uint32_t flags, double* row_val, int32_t* row_idx, double* col_val,
                               int32_t* col_idx, double* stats, void* workspace, size_t workspace_bytes) {
    HM_CHECK_ARG(X && Y && p && q && qb && db, "l2sq pricing: feature, cost and bias pointers are required");
    HM_CHECK_ARG(m >= 1 && n >= 1 && d >= 1 && m < INT32_MAX && n < INT32_MAX,
                 "l2sq pricing requires nonempty inputs with int32 dimensions (m=%lld n=%lld d=%d)",
                 (long long)m, (long long)n, d);
    HM_CHECK_ARG(k >= 1 && k <= 32, "l2sq pricing requires 1 <= k <= 32 (k=%d)", k);
    HM_CHECK_ARG(scale == 1.0 || scale == 2.0, "dot_scale must be exactly 1 or 2");
    HM_CHECK_ARG(!(flags & HM_ROWS) || (row_val && row_idx), "HM_ROWS requires row outputs");
    HM_CHECK_ARG(!(flags & HM_COLS) || (col_val && col_idx), "HM_COLS requires column outputs");
    HM_CHECK_ARG(!(flags & HM_STATS) || stats, "HM_STATS requires a stats output");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const DirPlan pr = plan_dir(m, n, k), pc = plan_dir(n, m, k);
    const size_t need = hm_pricing_l2sq_workspace_bytes(m, n, d, k, flags);
    HM_CHECK_ARG(workspace != nullptr, "workspace is required");
    if (workspace_bytes < need)
        return fail(HM_ENOSPC, "l2sq pricing workspace too small: %zu < %zu bytes", workspace_bytes, need);
    Arena a(workspace, workspace_bytes);
    double *xnorm, *ynorm, *blockstats;
    float *qb32, *p32, *db32, *ge32;
    unsigned long long* maxima;
    Entry* part;
    int *redo, *redo_count;
    layout(a, m, n, k, flags, pr, pc, &xnorm, &ynorm, &qb32, &p32, &db32, &ge32, &maxima, &part, &blockstats, &redo,
           &redo_count);
    hipLaunchKernelGGL(zero_words, dim3(1), dim3(64), 0, st, maxima, 4);
    HM_LAUNCH_CHECK("zero_words");
    // X side: ||x||, qb32, p32 (maxima[0..1] = max||x||, max|qb|); Y side: ||y||, db32, ge32 = q + db
    hipLaunchKernelGGL(l2sq_prep_rows, dim3((unsigned)((m + 3) / 4)), dim3(256), 0, st, X, m, d, p, qb,
                       (const double*)nullptr, xnorm, qb32, p32, maxima);
    HM_LAUNCH_CHECK("l2sq_prep_rows");
    hipLaunchKernelGGL(l2sq_prep_rows, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, st, Y, n, d, q, db, db, ynorm,
                       db32, ge32, maxima + 2);
    HM_LAUNCH_CHECK("l2sq_prep_rows");
    const bool want_stats = (flags & HM_STATS) != 0;
    const int linf = (flags & HM_LINF) ? 1 : 0;
    // rows (and certificate)
    if (flags & (HM_ROWS | HM_STATS)) {
        // ymaxima for the row direction = (max||y||, max|db|) = maxima[2..3]
        int rc = run_direction_k(st, X, Y, m, n, d, k, scale, want_stats, false, qb, db, xnorm, maxima + 2, qb32, db32,
                                 p32, ge32, pr, part, blockstats, redo, redo_count, row_val, row_idx, stats, linf,
                                 (flags & HM_ROWS) != 0);
        if (rc != HM_OK) return rc;
        if (want_stats && (flags & HM_ROWS)) {
            hipLaunchKernelGGL(exact_row_max, dim3(1), dim3(256), 0, st, row_val, m, k, stats);
            HM_LAUNCH_CHECK("exact_row_max");
        }
    }
    if (flags & HM_COLS) {
        // swapped roles: rows are Y, columns are X; biases swap, the exact score keeps the original association
        int rc = run_direction_k(st, Y, X, n, m, d, k, scale, false, true, db, qb, ynorm, maxima, db32, qb32, ge32,
                                 p32, pc, part, blockstats, redo, redo_count, col_val, col_idx, nullptr, 0, true);
        if (rc != HM_OK) return rc;
    }
    return HM_OK;
}
