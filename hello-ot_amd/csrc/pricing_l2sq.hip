// l2^2 pricing scan: C ABI entry points (kernels and the drivers live in l2sq_impl.h; the pricing_l2sq_l*_m*.hip
// translation units instantiate the driver per (partial list size, merged list size) and compile in parallel).
#include "l2sq_impl.h"
namespace hm {
int l2sq_run_l8_m8(L2SQ_RUN_ARGS);
int l2sq_run_l8_m16(L2SQ_RUN_ARGS);
int l2sq_run_l16_m16(L2SQ_RUN_ARGS);
int l2sq_run_l8_m40(L2SQ_RUN_ARGS);
int l2sq_run_l16_m40(L2SQ_RUN_ARGS);
int l2sq_run_l40_m40(L2SQ_RUN_ARGS);
namespace {
int run_k(L2SQ_RUN_ARGS) {
    const CallPlan c = plan_call(m, n, d, k, flags);
    if (c.km == 8) return l2sq_run_l8_m8(L2SQ_RUN_PASS);
    if (c.km == 16) return c.kl == 8 ? l2sq_run_l8_m16(L2SQ_RUN_PASS) : l2sq_run_l16_m16(L2SQ_RUN_PASS);
    if (c.kl == 8) return l2sq_run_l8_m40(L2SQ_RUN_PASS);
    return c.kl == 16 ? l2sq_run_l16_m40(L2SQ_RUN_PASS) : l2sq_run_l40_m40(L2SQ_RUN_PASS);
}

}  // namespace
}  // namespace hm

using namespace hm;

extern "C" size_t hm_pricing_l2sq_workspace_bytes(int64_t m, int64_t n, int32_t d, int32_t k, uint32_t flags) {
    if (m < 1 || n < 1 || k < 1 || k > 32) return 0;
    Sizer s;
    double *a, *b, *bs, *cv;
    float *c, *e, *f, *g;
    unsigned long long* mx;
    Entry *part, *colpart;
    unsigned int* thr;
    int *redo, *rc, *ci;
    float *xs, *ys;
    double* rpv;
    int* rpi;
    layout(s, m, n, d, k, flags, &a, &b, &c, &e, &f, &g, &mx, &part, &colpart, &thr, &cv, &ci, &bs, &redo, &rc, &xs,
           &ys, &rpv, &rpi);
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
    const size_t need = hm_pricing_l2sq_workspace_bytes(m, n, d, k, flags);
    HM_CHECK_ARG(workspace != nullptr, "workspace is required");
    if (workspace_bytes < need)
        return fail(HM_ENOSPC, "l2sq pricing workspace too small: %zu < %zu bytes", workspace_bytes, need);
    Arena a(workspace, workspace_bytes);
    double *xnorm, *ynorm, *blockstats, *cval;
    float *qb32, *p32, *db32, *ge32;
    unsigned long long* maxima;
    Entry *part, *colpart;
    unsigned int* colthr;
    int *redo, *redo_count, *cidx;
    float *xsplit, *ysplit;
    double* rpv;
    int* rpi;
    layout(a, m, n, d, k, flags, &xnorm, &ynorm, &qb32, &p32, &db32, &ge32, &maxima, &part, &colpart, &colthr, &cval,
           &cidx, &blockstats, &redo, &redo_count, &xsplit, &ysplit, &rpv, &rpi);
    hipLaunchKernelGGL(zero_words, dim3(1), dim3(64), 0, st, maxima, 4);
    HM_LAUNCH_CHECK("zero_words");
    // X side: ||x||, qb32, p32 (maxima[0..1] = max||x||, max|qb|); Y side: ||y||, db32, ge32 = q + db
    hipLaunchKernelGGL(l2sq_prep_rows, dim3(prep_grid(m)), dim3(256), 0, st, X, m, d, p, qb,
                       (const double*)nullptr, xnorm, qb32, p32, maxima);
    HM_LAUNCH_CHECK("l2sq_prep_rows");
    hipLaunchKernelGGL(l2sq_prep_rows, dim3(prep_grid(n)), dim3(256), 0, st, Y, n, d, q, db, db, ynorm,
                       db32, ge32, maxima + 2);
    HM_LAUNCH_CHECK("l2sq_prep_rows");
    return run_k(st, X, Y, m, n, d, k, scale, flags, qb, db, xnorm, ynorm, maxima, qb32, db32, p32, ge32, part,
                 colpart, colthr, cval, cidx, blockstats, redo, redo_count, row_val, row_idx, col_val, col_idx, stats,
                 xsplit, ysplit, rpv, rpi);
}
