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
    const CallPlan c = plan_call(m, n, d, k, flags, q8.y_ready);
    if (c.km == 8) return l2sq_run_l8_m8(L2SQ_RUN_PASS);
    if (c.km == 16) return c.kl == 8 ? l2sq_run_l8_m16(L2SQ_RUN_PASS) : l2sq_run_l16_m16(L2SQ_RUN_PASS);
    if (c.kl == 8) return l2sq_run_l8_m40(L2SQ_RUN_PASS);
    return c.kl == 16 ? l2sq_run_l16_m40(L2SQ_RUN_PASS) : l2sq_run_l40_m40(L2SQ_RUN_PASS);
}

}  // namespace

namespace {

int read_count(hipStream_t st, const int* count_dev, int* out) {
    HM_HIP(hipMemcpyAsync(out, count_dev, sizeof(int), hipMemcpyDeviceToHost, st));
    HM_HIP(hipStreamSynchronize(st));
    return HM_OK;
}

// Steps 3 and 4 of the wide pass for queued rows q0 .. q0+Q-1 whose candidates (w.cnt, w.buf) are collected: exact
// evaluation in slices, then the merge into the outputs (rows past `cap` go to the next queue).
int wide_exact(hipStream_t st, const float* A, const float* B, int d, const double* abias, const double* bbias,
               double scale, int k, const int* queue, int q0, int Q, int cap, double* out_val, int* out_idx, int cols,
               int cbase, const WideBufs& w, double* rpv, int* rpi, int* next, float* next_thr, int* next_count) {
    const int spr = cap / WIDE_SLICE;
    const int64_t items = (int64_t)Q * spr;
    const unsigned eg = (unsigned)((items + 3) / 4 < 8192 ? (items + 3) / 4 : 8192);
    const unsigned mg = (unsigned)((Q + 255) / 256);
#define HM_WIDE_EXACT(KK)                                                                                           \
    do {                                                                                                            \
        hipLaunchKernelGGL((l2sq_wide_slices<KK>), dim3(eg), dim3(256), 0, st, A, B, d, abias, bbias, scale, k,       \
                           queue, q0, Q, w.cnt, w.buf, cap, spr, cols, cbase, rpv, rpi);                            \
        hipLaunchKernelGGL((l2sq_wide_merge<KK>), dim3(mg), dim3(256), 0, st, rpv, rpi, Q, spr, k, w.cnt, cap, queue, \
                           w.thr, q0, out_val, out_idx, next, next_thr, next_count);                                \
    } while (0)
    if (k <= 2) HM_WIDE_EXACT(2);
    else if (k <= 8) HM_WIDE_EXACT(8);
    else HM_WIDE_EXACT(32);
#undef HM_WIDE_EXACT
    HM_LAUNCH_CHECK("l2sq_wide_exact");
    return HM_OK;
}

// One round of the wide pass over `count` queued rows: per batch, gather the rows' sweep copies, re-sweep them
// against all candidates collecting ids with w >= threshold (up to `cap` per row), evaluate the collected ids
// exactly in slices, merge; rows past `cap` go to (next, next_thr, next_count).
int wide_round(hipStream_t st, bool split, bool two_level, const float* A, const float* Asw, const float* B,
               const float* Bsw, int64_t nb, int d, int sd, int ld, const float* cand32, const double* abias,
               const double* bbias, double scale, int k, const int* queue, const float* queue_thr, int count,
               int cap, double* out_val, int* out_idx, int cols, int cbase, const WideBufs& w, double* rpv, int* rpi,
               int* next, float* next_thr, int* next_count, const float* aqs, const float* bqs) {
    const bool i8 = aqs != nullptr;  // the int8 sweep: the gathered rows carry their scales
    const int gld = split ? ld : d;  // row stride of the gathered sweep rows
    const int batch = (int)(WIDE_BUF / cap) < WIDE_ROWS ? (int)(WIDE_BUF / cap) : WIDE_ROWS;
    const int vec4 = split || (d % 4) == 0;
    for (int q0 = 0; q0 < count; q0 += batch) {
        const int Q = count - q0 < batch ? count - q0 : batch;
        const int bx = (split && two_level) ? BXW : BX;  // X rows per sweep workgroup
        const int Qpad = (int)panel_rows(Q, bx);
        if (split)
            hipLaunchKernelGGL(l2sq_wide_gather_split, dim3(2048), dim3(256), 0, st, Asw, gld, sd, queue, q0, Q, Qpad,
                               queue_thr, w.rows, w.thr, w.cnt, aqs, w.qs);
        else
            hipLaunchKernelGGL(l2sq_wide_gather, dim3(2048), dim3(256), 0, st, Asw, gld, queue, q0, Q, Qpad, queue_thr,
                               w.rows, w.thr, w.cnt);
        HM_LAUNCH_CHECK("l2sq_wide_gather");
        const DirPlan plan = plan_dir(Qpad, nb, 0, 256, bx, 1);
        const dim3 grid(sweep_grid(Qpad / bx, plan.S));
#define HM_WIDE(KERNEL, THREADS, ...)                                                                               \
    hipLaunchKernelGGL(KERNEL, grid, dim3(THREADS), 0, st, w.rows, Bsw, (int64_t)0, (int64_t)Q, nb, sd, gld,        \
                       (const float*)nullptr, cand32, (const float*)nullptr, (const float*)nullptr, (float)scale,    \
                       plan.seg_len, Qpad / bx, plan.S, (Entry*)nullptr, (Entry*)nullptr, (unsigned int*)nullptr,    \
                       (double*)nullptr, __VA_ARGS__, w.thr, w.cnt, w.buf, cap)
        if (i8) {
            HM_WIDE((l2sq_sweep_i8_w<8, false, true>), THREADS_W, 0, CertArgs{}, w.qs, bqs);
        } else if (split) {
            if (two_level) HM_WIDE((l2sq_sweep_split_w<8, false, true>), THREADS_W, 0, CertArgs{});
            else HM_WIDE((l2sq_sweep_split<8, false, true>), 256, 0, CertArgs{});
        } else {
            if (two_level) HM_WIDE((l2sq_sweep<8, true, false, true>), 256, vec4, 0, CertArgs{});
            else HM_WIDE((l2sq_sweep<8, false, false, true>), 256, vec4, 0, CertArgs{});
        }
#undef HM_WIDE
        HM_LAUNCH_CHECK("l2sq_sweep (wide)");
        if (int rc = wide_exact(st, A, B, d, abias, bbias, scale, k, queue, q0, Q, cap, out_val, out_idx, cols, cbase,
                                w, rpv, rpi, next, next_thr, next_count))
            return rc;
    }
    return HM_OK;
}

// The rows of the list queue: per batch, each row's partial-list entries at or above its threshold are collected
// (l2sq_list_collect) and evaluated exactly as in the wide pass; rows past `cap` go to (next, next_thr,
// next_count), the second round's sweep.
int list_round(hipStream_t st, const ListSource& ls, const float* A, const float* B, int d, const double* abias,
               const double* bbias, double scale, int k, const int* queue, const float* queue_thr, int count, int cap,
               double* out_val, int* out_idx, int cols, int cbase, const WideBufs& w, double* rpv, int* rpi,
               int* next, float* next_thr, int* next_count) {
    const int batch = (int)(WIDE_BUF / cap) < WIDE_ROWS ? (int)(WIDE_BUF / cap) : WIDE_ROWS;
    for (int q0 = 0; q0 < count; q0 += batch) {
        const int Q = count - q0 < batch ? count - q0 : batch;
        const unsigned cg = (unsigned)((Q + 3) / 4 < 8192 ? (Q + 3) / 4 : 8192);
#define HM_COLLECT(KK)                                                                                              \
    hipLaunchKernelGGL((l2sq_list_collect<KK>), dim3(cg), dim3(256), 0, st, ls.lists, ls.R, ls.nlists, ls.G, queue, \
                       q0, Q, queue_thr, cbase, cap, w.thr, w.cnt, w.buf)
        if (ls.KL == 8) HM_COLLECT(8);
        else if (ls.KL == 16) HM_COLLECT(16);
        else if (ls.KL == 40) HM_COLLECT(40);
        else return fail(HM_EINVAL, "internal: partial lists of %d entries", ls.KL);
#undef HM_COLLECT
        HM_LAUNCH_CHECK("l2sq_list_collect");
        if (int rc = wide_exact(st, A, B, d, abias, bbias, scale, k, queue, q0, Q, cap, out_val, out_idx, cols, cbase,
                                w, rpv, rpi, next, next_thr, next_count))
            return rc;
    }
    return HM_OK;
}

}  // namespace

int wide_resolve(hipStream_t st, bool split, bool two_level, const float* A, const float* Asw, const float* B,
                 const float* Bsw, int64_t nb, int d, int sd, int ld, const float* cand32, const double* abias,
                 const double* bbias, double scale, int k, const int* redo, const int* redo_count,
                 double* out_val, int* out_idx, int cols, int cbase, const WideBufs& w, double* rpv, int* rpi,
                 const float* aqs, const float* bqs, const ListSource& ls) {
    static_assert(WIDE_CAP1 % WIDE_SLICE == 0 && WIDE_CAP2 % WIDE_SLICE == 0, "whole slices per row");
    static_assert((WIDE_BUF / WIDE_CAP1) * (WIDE_CAP1 / WIDE_SLICE) <= RESCAN_ITEMS &&
                      (WIDE_BUF / WIDE_CAP2) * (WIDE_CAP2 / WIDE_SLICE) <= RESCAN_ITEMS,
                  "slice lists of a batch fit the rescan scratch");
    // queue 0 (a new sweep) and queue 1 (resolved from the partial lists): both counts in one read
    int counts[2] = {0, 0};
    HM_HIP(hipMemcpyAsync(counts, redo_count, 2 * sizeof(int), hipMemcpyDeviceToHost, st));
    HM_HIP(hipStreamSynchronize(st));
    const int count = counts[0];
    const int lcount = ls.lists ? counts[1] : 0;
    prof_count(cols ? "l2sq_wide_columns" : "l2sq_wide_rows", count);
    prof_count(cols ? "l2sq_list_columns" : "l2sq_list_rows", lcount);
    if (count <= 0 && lcount <= 0) return HM_OK;
    hipLaunchKernelGGL(zero_words, dim3(1), dim3(64), 0, st, reinterpret_cast<unsigned long long*>(w.counts), 2);
    HM_LAUNCH_CHECK("zero_words");
    prof_begin(st, "l2sq_wide");
    int rc = HM_OK;
    if (lcount > 0)
        rc = list_round(st, ls, A, B, d, abias, bbias, scale, k, w.redo_l, w.redo_l_thr, lcount, WIDE_CAP1, out_val,
                        out_idx, cols, cbase, w, rpv, rpi, w.redo2, w.redo2_thr, w.counts);
    if (!rc && count > 0)
        rc = wide_round(st, split, two_level, A, Asw, B, Bsw, nb, d, sd, ld, cand32, abias, bbias, scale, k, redo,
                        w.redo_thr, count, WIDE_CAP1, out_val, out_idx, cols, cbase, w, rpv, rpi, w.redo2, w.redo2_thr,
                        w.counts, aqs, bqs);
    int count2 = 0;
    if (!rc) rc = read_count(st, w.counts, &count2);
    if (!rc && count2 > 0)
        rc = wide_round(st, split, two_level, A, Asw, B, Bsw, nb, d, sd, ld, cand32, abias, bbias, scale, k, w.redo2,
                        w.redo2_thr, count2, WIDE_CAP2, out_val, out_idx, cols, cbase, w, rpv, rpi, w.redo3,
                        w.redo3_thr, w.counts + 1, aqs, bqs);
    prof_end(st);
    if (rc) return rc;
    // rows with more than WIDE_CAP2 candidates near their k-th value: exact scan over all candidates
    if (count2 <= 0) return HM_OK;
    return rescan_exact(st, A, B, nb, d, abias, bbias, scale, k, w.redo3, w.counts + 1, out_val, out_idx, cols, cbase,
                        rpv, rpi);
}

}  // namespace hm

using namespace hm;

namespace {
// A certificate needs the fp64 row lists (its maximum violation is the best row score); a call that asks for the
// certificate without them computes them into the workspace.
uint32_t effective_flags(uint32_t flags) { return (flags & HM_STATS) ? (flags | HM_ROWS) : flags; }
bool internal_rows(uint32_t flags) { return (flags & HM_STATS) && !(flags & HM_ROWS); }
}  // namespace

namespace {

size_t workspace_need(int64_t m, int64_t n, int32_t d, int32_t k, uint32_t flags, bool y_resident) {
    if (m < 1 || n < 1 || d < 1 || k < 1 || k > 32) return 0;
    const bool own_rows = internal_rows(flags);
    flags = effective_flags(flags);
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
    WideBufs wide;
    I8Bufs q8;
    layout(s, m, n, d, k, flags, &a, &b, &c, &e, &f, &g, &mx, &part, &colpart, &thr, &cv, &ci, &bs, &redo, &rc, &xs,
           &ys, &rpv, &rpi, &wide, &q8, y_resident);
    if (own_rows) {
        s.template take<double>((size_t)m * k);
        s.template take<int>((size_t)m * k);
    }
    return s.used;
}

// Header of a resident buffer (device memory, written by hm_l2sq_resident_prepare, read back by the calls)
constexpr uint64_t RESIDENT_MAGIC = 0x4d4933353552455aull;
struct ResidentHead {
    uint64_t magic;
    int64_t n;
    int32_t d;
    uint32_t precision;  // HM_BF16X3 / HM_INT8X3 bits of the preparation
    const void* y;       // the Y the side was prepared from
};
constexpr uint32_t PRECISION_BITS = HM_BF16X3 | HM_INT8X3;

size_t resident_bytes(int64_t n, int32_t d, uint32_t flags) {
    Sizer s;
    s.template take<ResidentHead>(1);
    ResidentY r;
    resident_layout(s, n, d, flags, &r);
    return s.used;
}

int check_call(const float* X, const float* Y, const double* p, const double* q, const double* qb, const double* db,
               int64_t m, int64_t n, int32_t d, int32_t k, double scale, uint32_t flags, const double* row_val,
               const int32_t* row_idx, const double* col_val, const int32_t* col_idx, const double* stats) {
    HM_CHECK_ARG(X && Y && p && q && qb && db, "l2sq pricing: feature, cost and bias pointers are required");
    HM_CHECK_ARG(m >= 1 && n >= 1 && d >= 1 && m < INT32_MAX && n < INT32_MAX,
                 "l2sq pricing requires nonempty inputs with int32 dimensions (m=%lld n=%lld d=%d)",
                 (long long)m, (long long)n, d);
    HM_CHECK_ARG(k >= 1 && k <= 32, "l2sq pricing requires 1 <= k <= 32 (k=%d)", k);
    HM_CHECK_ARG(scale == 1.0 || scale == 2.0, "dot_scale must be exactly 1 or 2");
    HM_CHECK_ARG(!((flags & HM_BF16X3) && (flags & HM_INT8X3)), "HM_BF16X3 and HM_INT8X3 exclude each other");
    HM_CHECK_ARG(!(flags & HM_INT8X3) || d <= 65536, "the int8 sweep supports d <= 65536 (d=%d)", d);
    HM_CHECK_ARG(!(flags & HM_ROWS) || (row_val && row_idx), "HM_ROWS requires row outputs");
    HM_CHECK_ARG(!(flags & HM_COLS) || (col_val && col_idx), "HM_COLS requires column outputs");
    HM_CHECK_ARG(!(flags & HM_STATS) || stats, "HM_STATS requires a stats output");
    return HM_OK;
}

// One pricing call; `res` (or null) is a validated resident Y side
int pricing_call(hipStream_t st, const float* X, const float* Y, const double* p, const double* q, const double* qb,
                 const double* db, int64_t m, int64_t n, int32_t d, int32_t k, double scale, uint32_t flags,
                 double* row_val, int32_t* row_idx, double* col_val, int32_t* col_idx, double* stats,
                 const ResidentY* res, void* workspace, size_t workspace_bytes, const double* col_floor = nullptr) {
    const size_t need = workspace_need(m, n, d, k, flags, res != nullptr);
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
    WideBufs wide;
    I8Bufs q8;
    const bool own_rows = internal_rows(flags);
    flags = effective_flags(flags);
    layout(a, m, n, d, k, flags, &xnorm, &ynorm, &qb32, &p32, &db32, &ge32, &maxima, &part, &colpart, &colthr, &cval,
           &cidx, &blockstats, &redo, &redo_count, &xsplit, &ysplit, &rpv, &rpi, &wide, &q8, res != nullptr);
    wide.col_floor = col_floor;
    if (own_rows) {
        row_val = a.template take<double>((size_t)m * k);
        row_idx = a.template take<int>((size_t)m * k);
    }
    if (res) {
        ynorm = res->ynorm;
        ysplit = res->ysplit;
        q8.yqs = res->q8.yqs;
        q8.yl1 = res->q8.yl1;
        q8.yterm = res->q8.yterm;
        q8.qmax_y = res->q8.qmax_y;
        q8.y_ready = true;
    }
    hipLaunchKernelGGL(zero_words, dim3(1), dim3(64), 0, st, maxima, 4);
    HM_LAUNCH_CHECK("zero_words");
    // X side: ||x||, qb32, p32 (maxima[0..1] = max||x||, max|qb|); Y side: ||y||, db32, ge32 = q + db
    // (maxima[2..3]); with HM_INT8X3 also the int8 row maxima and ||.||_1 of both sides. A resident Y side has its
    // norms and int8 data already: only its biases are converted.
    hipLaunchKernelGGL(l2sq_prep_rows, dim3(prep_grid(m)), dim3(256), 0, st, X, m, d, p, qb,
                       (const double*)nullptr, xnorm, qb32, p32, maxima, q8.xqs, q8.xl1);
    HM_LAUNCH_CHECK("l2sq_prep_rows");
    if (res)
        hipLaunchKernelGGL(l2sq_prep_bias, dim3(prep_grid(n)), dim3(256), 0, st, n, q, db, res->ynorm_max, db32, ge32,
                           maxima + 2);
    else
        hipLaunchKernelGGL(l2sq_prep_rows, dim3(prep_grid(n)), dim3(256), 0, st, Y, n, d, q, db, db, ynorm,
                           db32, ge32, maxima + 2, q8.yqs, q8.yl1);
    HM_LAUNCH_CHECK("l2sq_prep_rows");
    return run_k(st, X, Y, m, n, d, k, scale, flags, qb, db, xnorm, ynorm, maxima, qb32, db32, p32, ge32, part,
                 colpart, colthr, cval, cidx, blockstats, redo, redo_count, row_val, row_idx, col_val, col_idx, stats,
                 xsplit, ysplit, rpv, rpi, wide, q8);
}

}  // namespace

extern "C" size_t hm_pricing_l2sq_workspace_bytes(int64_t m, int64_t n, int32_t d, int32_t k, uint32_t flags) {
    return workspace_need(m, n, d, k, flags, false);
}

extern "C" int hm_pricing_l2sq(void* stream, const float* X, const float* Y, const double* p, const double* q,
                               const double* qb, const double* db, int64_t m, int64_t n, int32_t d, int32_t k,
                               double scale, uint32_t flags, double* row_val, int32_t* row_idx, double* col_val,
                               int32_t* col_idx, double* stats, void* workspace, size_t workspace_bytes) {
    if (int rc = check_call(X, Y, p, q, qb, db, m, n, d, k, scale, flags, row_val, row_idx, col_val, col_idx, stats))
        return rc;
    return pricing_call(reinterpret_cast<hipStream_t>(stream), X, Y, p, q, qb, db, m, n, d, k, scale, flags, row_val,
                        row_idx, col_val, col_idx, stats, nullptr, workspace, workspace_bytes);
}

extern "C" size_t hm_l2sq_resident_bytes(int64_t n, int32_t d, uint32_t flags) {
    if (n < 1 || d < 1 || n >= INT32_MAX) return 0;
    return resident_bytes(n, d, flags);
}

extern "C" int hm_l2sq_resident_prepare(void* stream, const float* Y, int64_t n, int32_t d, uint32_t flags,
                                        void* resident, size_t bytes) {
    HM_CHECK_ARG(Y && resident, "resident side: feature and buffer pointers are required");
    HM_CHECK_ARG(n >= 1 && d >= 1 && n < INT32_MAX, "resident side requires n >= 1, d >= 1 (n=%lld d=%d)",
                 (long long)n, d);
    HM_CHECK_ARG(!((flags & HM_BF16X3) && (flags & HM_INT8X3)), "HM_BF16X3 and HM_INT8X3 exclude each other");
    HM_CHECK_ARG(!(flags & HM_INT8X3) || d <= 65536, "the int8 sweep supports d <= 65536 (d=%d)", d);
    const size_t need = resident_bytes(n, d, flags);
    if (bytes < need) return fail(HM_ENOSPC, "resident buffer too small: %zu < %zu bytes", bytes, need);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    Arena a(resident, bytes);
    ResidentHead* head = a.template take<ResidentHead>(1);
    ResidentY r;
    resident_layout(a, n, d, flags, &r);
    const bool i8 = (flags & HM_INT8X3) != 0, split = (flags & PRECISION_BITS) != 0;
    const int sd = i8 ? i8_words(d) : split_features(d), ld = i8 ? i8_ld(d) : split_ld(d);
    hipLaunchKernelGGL(zero_words, dim3(1), dim3(64), 0, st, r.ynorm_max, 2);
    hipLaunchKernelGGL(l2sq_prep_rows, dim3(prep_grid(n)), dim3(256), 0, st, Y, n, d, (const double*)nullptr,
                       (const double*)nullptr, (const double*)nullptr, r.ynorm, (float*)nullptr, (float*)nullptr,
                       r.ynorm_max, r.q8.yqs, r.q8.yl1);
    HM_LAUNCH_CHECK("l2sq_prep_rows");
    if (i8) {
        launch_split_i8(st, Y, n, d, sd, ld, r.q8.yqs, r.q8.yl1, r.ynorm, r.ysplit, r.q8.yterm, r.q8.qmax_y);
        HM_LAUNCH_CHECK("l2sq_split_i8");
    } else if (split) {
        hipLaunchKernelGGL(l2sq_split_bf16, dim3(4096), dim3(256), 0, st, Y, n, panel_rows(n, BXW), d, sd, ld,
                           reinterpret_cast<unsigned short*>(r.ysplit));
        HM_LAUNCH_CHECK("l2sq_split_bf16");
    }
    const ResidentHead h{RESIDENT_MAGIC, n, d, flags & PRECISION_BITS, Y};
    HM_HIP(hipMemcpyAsync(head, &h, sizeof(h), hipMemcpyHostToDevice, st));
    HM_HIP(hipStreamSynchronize(st));  // `h` lives on this stack frame
    return HM_OK;
}

extern "C" size_t hm_pricing_l2sq_resident_workspace_bytes(int64_t m, int64_t n, int32_t d, int32_t k,
                                                           uint32_t flags) {
    return workspace_need(m, n, d, k, flags, true);
}

extern "C" int hm_pricing_l2sq_resident_floor(void* stream, const float* X, const float* Y, const double* p,
                                              const double* q, const double* qb, const double* db, int64_t m,
                                              int64_t n, int32_t d, int32_t k, double scale, uint32_t flags,
                                              const double* col_floor, double* row_val, int32_t* row_idx,
                                              double* col_val, int32_t* col_idx, double* stats, const void* resident,
                                              size_t resident_bytes_, void* workspace, size_t workspace_bytes) {
    if (int rc = check_call(X, Y, p, q, qb, db, m, n, d, k, scale, flags, row_val, row_idx, col_val, col_idx, stats))
        return rc;
    HM_CHECK_ARG(!col_floor || (flags & HM_COLS), "a column floor needs HM_COLS");
    HM_CHECK_ARG(resident != nullptr, "resident side buffer is required");
    if (resident_bytes_ < sizeof(ResidentHead))
        return fail(HM_EINVAL, "resident buffer smaller than a side of n=%lld d=%d needs", (long long)n, d);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    ResidentHead h{};
    HM_HIP(hipMemcpyAsync(&h, resident, sizeof(h), hipMemcpyDeviceToHost, st));
    HM_HIP(hipStreamSynchronize(st));
    if (h.magic != RESIDENT_MAGIC) return fail(HM_EINVAL, "resident buffer was not prepared");
    if (h.n != n || h.d != d || h.y != (const void*)Y)
        return fail(HM_EINVAL, "resident side was prepared for other features (n=%lld d=%d)", (long long)h.n, h.d);
    if (h.precision != (flags & PRECISION_BITS))
        return fail(HM_EINVAL, "resident side was prepared for another sweep precision");
    if (resident_bytes_ < resident_bytes(n, d, flags))
        return fail(HM_EINVAL, "resident buffer smaller than a side of n=%lld d=%d needs", (long long)n, d);
    Arena a(const_cast<void*>(resident), resident_bytes_);
    a.template take<ResidentHead>(1);
    ResidentY r;
    resident_layout(a, n, d, flags, &r);
    return pricing_call(st, X, Y, p, q, qb, db, m, n, d, k, scale, flags, row_val, row_idx, col_val, col_idx, stats,
                        &r, workspace, workspace_bytes, col_floor);
}

extern "C" int hm_pricing_l2sq_resident(void* stream, const float* X, const float* Y, const double* p, const double* q,
                                        const double* qb, const double* db, int64_t m, int64_t n, int32_t d, int32_t k,
                                        double scale, uint32_t flags, double* row_val, int32_t* row_idx,
                                        double* col_val, int32_t* col_idx, double* stats, const void* resident,
                                        size_t resident_bytes_, void* workspace, size_t workspace_bytes) {
    return hm_pricing_l2sq_resident_floor(stream, X, Y, p, q, qb, db, m, n, d, k, scale, flags, nullptr, row_val,
                                          row_idx, col_val, col_idx, stats, resident, resident_bytes_, workspace,
                                          workspace_bytes);
}
