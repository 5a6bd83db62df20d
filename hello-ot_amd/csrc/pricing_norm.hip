// Norm-cost (l1 / linf / l2) pricing scan on VALU for gfx950.
//
// Semantics (pricing.cu:65-161 VALU scan, cost.cu:10-85 direct_norm tiles, matrix_selection.cuh:20-26):
//   c_ij = fp32 distance; features are combined sequentially inside 32-feature chunks and the chunk results
//          are then combined in order (l1: sum |x-y|, linf: max |x-y|, l2: sqrtf(sum fmaf(z, z, .))),
//   sigma_ij = (g_j - (double)c_ij) + f_i   (fp64).
// Every value is reproduced bit for bit, so the per-row lists hold exact fp64 scores: an fp32 estimate of
// sigma with a rigorous slack only decides whether a pair needs its fp64 score.
//
// One thread owns one X row (features in registers); Y tiles of 256 rows are staged in LDS and read by
// broadcast. Column lists come from a second sweep with the roles swapped (the score keeps the original
// association). Certificate sums are accumulated in fp32 per tile and flushed to fp64.
#include <mutex>

#include "common.h"

namespace hm {
namespace {

constexpr int NB_ROWS = 256;   // X rows per workgroup (one per thread)
constexpr int NT = 256;        // Y rows per LDS tile (fewer when d is large: the tile stays within 64 KiB)
constexpr int LDS_FLOATS = 15872;  // 62 KiB of dynamic LDS, leaving room for the static reduction buffer

template <int KIND>
__device__ inline float feature_op(float part, float z) {
    if (KIND == HM_COST_L1) return part + fabsf(z);
    if (KIND == HM_COST_LINF) return fmaxf(part, fabsf(z));
    return fmaf(z, z, part);
}

// distance with x in registers (DR >= d) and y in LDS (row-major, stride ys)
template <int KIND, int DR>
__device__ inline float distance_reg(const float (&x)[DR], const float* __restrict__ y, int d) {
    float acc = 0.0f;
#pragma unroll
    for (int base = 0; base < DR; base += 32) {
        if (base < d) {
            float part = 0.0f;
#pragma unroll
            for (int k = base; k < base + 32 && k < DR; ++k)
                if (k < d) part = feature_op<KIND>(part, x[k] - y[k]);
            acc = (KIND == HM_COST_LINF) ? fmaxf(acc, part) : acc + part;
        }
    }
    return (KIND == HM_COST_L2) ? (float)sqrt((double)acc) : acc;  // fp64 sqrt rounded once: correctly rounded
}

// distance with x in registers and exactly DR features (DR % 4 == 0, y 16-byte aligned): the same operations in the
// same order as distance_reg, with y read from LDS as float4 and no per-feature bounds
template <int KIND, int DR>
__device__ inline float distance_exact(const float (&x)[DR], const float* __restrict__ y) {
    static_assert(DR % 4 == 0, "whole float4 rows");
    float yv[DR];
#pragma unroll
    for (int k = 0; k < DR; k += 4) {
        const float4 t = *reinterpret_cast<const float4*>(y + k);
        yv[k] = t.x;
        yv[k + 1] = t.y;
        yv[k + 2] = t.z;
        yv[k + 3] = t.w;
    }
    float acc = 0.0f;
#pragma unroll
    for (int base = 0; base < DR; base += 32) {
        float part = 0.0f;
#pragma unroll
        for (int k = base; k < base + 32 && k < DR; ++k) part = feature_op<KIND>(part, x[k] - yv[k]);
        acc = (KIND == HM_COST_LINF) ? fmaxf(acc, part) : acc + part;
    }
    return (KIND == HM_COST_L2) ? (float)sqrt((double)acc) : acc;  // fp64 sqrt rounded once: correctly rounded
}

// distance with x streamed from global memory (any d)
template <int KIND>
__device__ inline float distance_mem(const float* __restrict__ x, const float* __restrict__ y, int d) {
    float acc = 0.0f;
    for (int base = 0; base < d; base += 32) {
        float part = 0.0f;
        const int end = base + 32 < d ? base + 32 : d;
        for (int k = base; k < end; ++k) part = feature_op<KIND>(part, x[k] - y[k]);
        acc = (KIND == HM_COST_LINF) ? fmaxf(acc, part) : acc + part;
    }
    return (KIND == HM_COST_L2) ? (float)sqrt((double)acc) : acc;  // fp64 sqrt rounded once: correctly rounded
}

__global__ void norm_prep(const float* __restrict__ Y, int64_t n, int d, const double* __restrict__ g,
                          unsigned long long* __restrict__ maxima /*[max ||y||_1, max |g|]*/) {
    const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= n) return;
    double s = 0.0;
    for (int k = 0; k < d; ++k) s += fabs((double)Y[j * d + k]);
    atomicMax(&maxima[0], double_key(s));
    atomicMax(&maxima[1], double_key(fabs(g[j])));
}

// EXACT: d == DR (a multiple of 4), so Y rows in LDS are whole float4s
template <int KIND, int K, int DR, bool EXACT>
__global__ __launch_bounds__(256) void norm_sweep(const float* __restrict__ X, const float* __restrict__ Y, int64_t m,
                                                  int64_t n, int d, const double* __restrict__ rb,
                                                  const double* __restrict__ cb,
                                                  const unsigned long long* __restrict__ ymaxima, int k,
                                                  int64_t seg_len, double* __restrict__ part_v, int* __restrict__ part_i,
                                                  double* __restrict__ blockstats, int STATS, int TRANSPOSED, int ntile) {
    extern __shared__ float4 smem4[];
    float* smem = reinterpret_cast<float*>(smem4);
    float* sy = smem;                            // ntile * d
    float* scb = smem + (size_t)ntile * d;       // ntile (column duals as fp32)
    __shared__ double sRed[4][5];
    const int tid = threadIdx.x;
    const int64_t row = (int64_t)blockIdx.x * NB_ROWS + tid;
    const bool row_ok = row < m;
    const int64_t seg = blockIdx.y;
    const int64_t y_begin = seg * seg_len;
    const int64_t y_end = y_begin + seg_len < n ? y_begin + seg_len : n;

    float x[DR > 0 ? DR : 1];
    double x1 = 0.0;
    if (DR > 0) {
#pragma unroll
        for (int t = 0; t < (DR > 0 ? DR : 1); ++t) x[t] = (row_ok && t < d) ? X[row * d + t] : 0.0f;
#pragma unroll
        for (int t = 0; t < (DR > 0 ? DR : 1); ++t) x1 += fabs((double)x[t]);
    } else if (row_ok) {
        for (int t = 0; t < d; ++t) x1 += fabs((double)X[row * d + t]);
    }
    const double fi = row_ok ? rb[row] : 0.0;
    const float fi32 = (float)fi;
    // slack >= |sigma32 - sigma64|: every fp32 operand is within u of its fp64 value and the two fp32 sums
    // round by at most u each; magnitudes are bounded by |g| + c + |f| with c <= ||x||_1 + max||y||_1.
    const double ymax1 = key_double(ymaxima[0]);
    const double gmax = key_double(ymaxima[1]);
    const float slack = (float)((x1 + ymax1 + gmax + fabs(fi)) * 4.0 * 5.9604644775390625e-08 * (1.0 + 1e-6) + 1e-37);

    double v[K];
    int id[K];
#pragma unroll
    for (int s = 0; s < K; ++s) { v[s] = -INFINITY; id[s] = -1; }
    float thr = -INFINITY;
    double num64 = 0.0, den64 = 0.0, cnt64 = 0.0;
    float cmax = 0.0f;

    for (int64_t t0 = y_begin; t0 < y_end; t0 += ntile) {
        const int cnt = (int)((y_end - t0) < ntile ? (y_end - t0) : ntile);
        __syncthreads();
        for (int e = tid; e < cnt * d; e += 256) sy[e] = Y[t0 * d + e];
        for (int e = tid; e < cnt; e += 256) scb[e] = (float)cb[t0 + e];
        __syncthreads();
        float tnum = 0.0f, tden = 0.0f;
        unsigned tc = 0;
        if (row_ok) {
            for (int jj = 0; jj < cnt; ++jj) {
                const float* yj = sy + (size_t)jj * d;
                float c;
                if constexpr (EXACT) c = distance_exact<KIND, DR>(x, yj);
                else if (DR > 0) c = distance_reg<KIND, (DR > 0 ? DR : 1)>(x, yj, d);
                else c = distance_mem<KIND>(X + row * d, yj, d);
                const float s32 = (scb[jj] - c) + fi32;
                if (s32 > thr) {
                    const int64_t j = t0 + jj;
                    const double cd = (double)c;
                    const double sig = TRANSPOSED ? (fi - cd) + cb[j] : (cb[j] - cd) + fi;
                    if (sig == sig && better(sig, (int)j, v[k - 1], id[k - 1])) {
                        put_sorted<K>(v, id, k, sig, (int)j);
                        const double kth = v[k - 1];
                        // (float) rounds to nearest; one ulp down keeps thr strictly below kth - slack
                        thr = (kth == -INFINITY) ? -INFINITY : nextafterf((float)(kth - (double)slack), -INFINITY);
                    }
                }
                if (STATS) {
                    tden = fmaf(c, c, tden);
                    cmax = fmaxf(cmax, c);
                    // beyond the slack the fp32 score decides; within it the exact fp64 score does (the maximum
                    // comes from the exact row lists afterwards)
                    if (s32 > slack) {
                        tnum = fmaf(s32, s32, tnum);
                        ++tc;
                    } else if (s32 > -slack) {
                        const double cd = (double)c;
                        const double sig = TRANSPOSED ? (fi - cd) + cb[t0 + jj] : (cb[t0 + jj] - cd) + fi;
                        if (sig > 0.0) {
                            num64 = fma(sig, sig, num64);
                            ++tc;
                        }
                    }
                }
            }
        }
        if (STATS) {
            num64 += (double)tnum;
            den64 += (double)tden;
            cnt64 += (double)tc;
        }
    }
    if (row_ok) {
        double* ov = part_v + (seg * m + row) * k;
        int* oi = part_i + (seg * m + row) * k;
        for (int s = 0; s < k; ++s) { ov[s] = v[s]; oi[s] = id[s]; }
    }
    if (STATS) {
        const int lane = tid & 63, wave = tid >> 6;
        double r[5] = {num64, den64, cnt64, 0.0, (double)cmax};  // slot 3: exact row maximum later
#pragma unroll
        for (int e = 0; e < 5; ++e)
            for (int o = 32; o >= 1; o >>= 1) {
                const double t = __shfl_xor(r[e], o, 64);
                r[e] = e >= 3 ? fmax(r[e], t) : r[e] + t;
            }
        if (lane == 0)
            for (int e = 0; e < 5; ++e) sRed[wave][e] = r[e];
        __syncthreads();
        if (tid == 0) {
            double* dst = blockstats + ((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * 5;
            for (int e = 0; e < 5; ++e) {
                double o = sRed[0][e];
                for (int w = 1; w < 4; ++w) o = e >= 3 ? fmax(o, sRed[w][e]) : o + sRed[w][e];
                dst[e] = o;
            }
        }
    }
}

// merge S exact segment lists per row (tie rule), one thread per row
template <int K>
__global__ void norm_merge(const double* __restrict__ part_v, const int* __restrict__ part_i, int64_t m, int S, int k,
                           double* __restrict__ out_v, int* __restrict__ out_i) {
    const int64_t row = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= m) return;
    double v[K];
    int id[K];
#pragma unroll
    for (int s = 0; s < K; ++s) { v[s] = -INFINITY; id[s] = -1; }
    for (int sg = 0; sg < S; ++sg) {
        const double* pv = part_v + ((int64_t)sg * m + row) * k;
        const int* pi = part_i + ((int64_t)sg * m + row) * k;
        for (int s = 0; s < k; ++s)
            if (pi[s] >= 0) put_sorted<K>(v, id, k, pv[s], pi[s]);
    }
    for (int s = 0; s < k; ++s) { out_v[row * k + s] = v[s]; out_i[row * k + s] = id[s]; }
}

__global__ void norm_reduce_stats(const double* __restrict__ blockstats, int64_t blocks, double* __restrict__ stats,
                                  int linf) {
    __shared__ double s[256][5];
    const int t = threadIdx.x;
    double v[5] = {0, 0, 0, 0, 0};
    for (int64_t b = t; b < blocks; b += 256)
        for (int e = 0; e < 5; ++e) v[e] = e >= 3 ? fmax(v[e], blockstats[b * 5 + e]) : v[e] + blockstats[b * 5 + e];
    for (int e = 0; e < 5; ++e) s[t][e] = v[e];
    __syncthreads();
    for (int w = 128; w >= 1; w >>= 1) {
        if (t < w)
            for (int e = 0; e < 5; ++e) s[t][e] = e >= 3 ? fmax(s[t][e], s[t + w][e]) : s[t][e] + s[t + w][e];
        __syncthreads();
    }
    if (t == 0) {
        stats[0] = s[0][0];
        stats[1] = s[0][1];
        stats[2] = s[0][2];
        stats[3] = s[0][3];
        stats[4] = linf ? s[0][4] : 0.0;
    }
}

__global__ void norm_exact_max(const double* __restrict__ row_val, int64_t m, int k, double* __restrict__ stats) {
    __shared__ double s[256];
    double v = 0.0;
    for (int64_t i = threadIdx.x; i < m; i += 256) v = fmax(v, row_val[i * k]);
    s[threadIdx.x] = v;
    __syncthreads();
    for (int w = 128; w >= 1; w >>= 1) {
        if ((int)threadIdx.x < w) s[threadIdx.x] = fmax(s[threadIdx.x], s[threadIdx.x + w]);
        __syncthreads();
    }
    if (threadIdx.x == 0) stats[3] = s[0];
}

__global__ void norm_zero(unsigned long long* p, int count) {
    if ((int)threadIdx.x < count) p[threadIdx.x] = 0ull;
}

struct NormPlan {
    int S;
    int64_t seg_len;
};

inline NormPlan norm_plan(int64_t rows, int64_t cols) {
    const int64_t blocks = (rows + NB_ROWS - 1) / NB_ROWS;
    int64_t s = (1024 + blocks - 1) / blocks;
    const int64_t tiles = (cols + NT - 1) / NT;
    if (s > tiles) s = tiles;
    if (s > 64) s = 64;
    if (s < 1) s = 1;
    const int64_t per = (tiles + s - 1) / s;
    NormPlan p;
    p.seg_len = per * NT;
    p.S = (int)((cols + p.seg_len - 1) / p.seg_len);
    return p;
}

inline int kbucket(int k) { return k <= 2 ? 2 : (k <= 8 ? 8 : 32); }

template <class A>
void norm_layout(A& a, int64_t m, int64_t n, int k, uint32_t flags, double** pv, int** pi, double** bs,
                 unsigned long long** maxima) {
    const NormPlan pr = norm_plan(m, n), pc = norm_plan(n, m);
    size_t entries = 0;
    if (flags & (HM_ROWS | HM_STATS)) entries = (size_t)pr.S * m * k;
    if (flags & HM_COLS) {
        const size_t c = (size_t)pc.S * n * k;
        if (c > entries) entries = c;
    }
    *pv = a.template take<double>(entries > 0 ? entries : 1);
    *pi = a.template take<int>(entries > 0 ? entries : 1);
    const int64_t br = ((m + NB_ROWS - 1) / NB_ROWS) * pr.S, bc = ((n + NB_ROWS - 1) / NB_ROWS) * pc.S;
    *bs = a.template take<double>((size_t)5 * (br > bc ? br : bc));
    *maxima = a.template take<unsigned long long>(4);
}

template <int KIND, int K, int DR, bool EXACT>
int norm_direction_t(hipStream_t st, const float* X, const float* Y, int64_t m, int64_t n, int d, const double* rb,
                     const double* cb, const unsigned long long* ymaxima, int k, bool stats, bool transposed,
                     NormPlan plan, double* pv, int* pi, double* bs, double* out_v, int* out_i, double* stats_out,
                     int linf) {
    dim3 grid((unsigned)((m + NB_ROWS - 1) / NB_ROWS), (unsigned)plan.S);
    int ntile = NT;
    while (ntile > 1 && (size_t)ntile * (d + 1) > LDS_FLOATS) ntile >>= 1;
    if ((size_t)ntile * (d + 1) > LDS_FLOATS) return fail(HM_EINVAL, "norm pricing supports d <= %d", LDS_FLOATS - 1);
    const size_t shmem = ((size_t)ntile * d + ntile) * sizeof(float);
    prof_begin(st, "norm_sweep");
    hipLaunchKernelGGL((norm_sweep<KIND, K, DR, EXACT>), grid, dim3(256), shmem, st, X, Y, m, n, d, rb, cb, ymaxima, k,
                       plan.seg_len, pv, pi, bs, (int)stats, (int)transposed, ntile);
    prof_end(st);
    HM_LAUNCH_CHECK("norm_sweep");
    hipLaunchKernelGGL((norm_merge<K>), dim3((unsigned)((m + 255) / 256)), dim3(256), 0, st, pv, pi, m, plan.S, k,
                       out_v, out_i);
    HM_LAUNCH_CHECK("norm_merge");
    if (stats) {
        hipLaunchKernelGGL(norm_reduce_stats, dim3(1), dim3(256), 0, st, bs, (int64_t)grid.x * grid.y, stats_out, linf);
        HM_LAUNCH_CHECK("norm_reduce_stats");
    }
    return HM_OK;
}

template <int KIND, int K>
int norm_direction_d(hipStream_t st, const float* X, const float* Y, int64_t m, int64_t n, int d, const double* rb,
                     const double* cb, const unsigned long long* ymaxima, int k, bool stats, bool transposed,
                     NormPlan plan, double* pv, int* pi, double* bs, double* out_v, int* out_i, double* stats_out,
                     int linf) {
    if (d == 8)
        return norm_direction_t<KIND, K, 8, true>(st, X, Y, m, n, d, rb, cb, ymaxima, k, stats, transposed, plan, pv, pi,
                                                  bs, out_v, out_i, stats_out, linf);
    if (d <= 8)
        return norm_direction_t<KIND, K, 8, false>(st, X, Y, m, n, d, rb, cb, ymaxima, k, stats, transposed, plan, pv, pi, bs,
                                            out_v, out_i, stats_out, linf);
    if (d <= 64)
        return norm_direction_t<KIND, K, 64, false>(st, X, Y, m, n, d, rb, cb, ymaxima, k, stats, transposed, plan, pv, pi, bs,
                                             out_v, out_i, stats_out, linf);
    return norm_direction_t<KIND, K, 0, false>(st, X, Y, m, n, d, rb, cb, ymaxima, k, stats, transposed, plan, pv, pi, bs,
                                        out_v, out_i, stats_out, linf);
}

template <int KIND>
int norm_direction(hipStream_t st, const float* X, const float* Y, int64_t m, int64_t n, int d, const double* rb,
                   const double* cb, const unsigned long long* ymaxima, int k, bool stats, bool transposed,
                   NormPlan plan, double* pv, int* pi, double* bs, double* out_v, int* out_i, double* stats_out,
                   int linf) {
    switch (kbucket(k)) {
#define HM_K(KK) \
    case KK:     \
        return norm_direction_d<KIND, KK>(st, X, Y, m, n, d, rb, cb, ymaxima, k, stats, transposed, plan, pv, pi, bs, \
                                          out_v, out_i, stats_out, linf);
        HM_K(2)
        HM_K(8)
        HM_K(32)
#undef HM_K
    }
    return fail(HM_EINVAL, "unsupported k");
}

}  // namespace
}  // namespace hm

using namespace hm;

extern "C" size_t hm_pricing_norm_workspace_bytes(int64_t m, int64_t n, int32_t d, int32_t k, uint32_t flags) {
    (void)d;
    if (m < 1 || n < 1 || k < 1 || k > 32) return 0;
    Sizer s;
    double *pv, *bs;
    int* pi;
    unsigned long long* mx;
    norm_layout(s, m, n, k, flags, &pv, &pi, &bs, &mx);
    return s.used;
}

namespace {

// The scan with its scratch in `workspace` (caller memory, or the static scratch array of hm_pricing_norm_noalloc).
// Everything the scratch holds is written before it is read; the maxima are cleared by a kernel, not a memset.
int norm_scan_run(void* stream, const float* X, const float* Y, const double* f, const double* g, int64_t m,
                  int64_t n, int32_t d, int32_t k, int32_t kind, uint32_t flags, double* row_val, int32_t* row_idx,
                  double* col_val, int32_t* col_idx, double* stats, void* workspace, size_t workspace_bytes) {
    HM_CHECK_ARG(X && Y && f && g, "norm pricing: feature and dual pointers are required");
    HM_CHECK_ARG(m >= 1 && n >= 1 && d >= 1 && m < INT32_MAX && n < INT32_MAX,
                 "norm pricing requires nonempty inputs with int32 dimensions");
    HM_CHECK_ARG(k >= 1 && k <= 32, "norm pricing requires 1 <= k <= 32 (k=%d)", k);
    HM_CHECK_ARG(kind == HM_COST_L1 || kind == HM_COST_LINF || kind == HM_COST_L2, "unsupported norm cost %d", kind);
    HM_CHECK_ARG(!(flags & HM_ROWS) || (row_val && row_idx), "HM_ROWS requires row outputs");
    HM_CHECK_ARG(!(flags & HM_COLS) || (col_val && col_idx), "HM_COLS requires column outputs");
    HM_CHECK_ARG(!(flags & HM_STATS) || stats, "HM_STATS requires a stats output");
    HM_CHECK_ARG(workspace != nullptr, "workspace is required");
    const size_t need = hm_pricing_norm_workspace_bytes(m, n, d, k, flags);
    if (workspace_bytes < need)
        return fail(HM_ENOSPC, "norm pricing workspace too small: %zu < %zu bytes", workspace_bytes, need);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    Arena a(workspace, workspace_bytes);
    double *pv, *bs;
    int* pi;
    unsigned long long* maxima;
    norm_layout(a, m, n, k, flags, &pv, &pi, &bs, &maxima);
    hipLaunchKernelGGL(norm_zero, dim3(1), dim3(64), 0, st, maxima, 4);
    HM_LAUNCH_CHECK("norm_zero");
    // maxima[0..1] for the row sweep (Y side), maxima[2..3] for the column sweep (X side)
    hipLaunchKernelGGL(norm_prep, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, Y, n, d, g, maxima);
    HM_LAUNCH_CHECK("norm_prep");
    hipLaunchKernelGGL(norm_prep, dim3((unsigned)((m + 255) / 256)), dim3(256), 0, st, X, m, d, f, maxima + 2);
    HM_LAUNCH_CHECK("norm_prep");
    const bool want_stats = (flags & HM_STATS) != 0;
    const int linf = (flags & HM_LINF) ? 1 : 0;
    double* rows_v = row_val;
    int* rows_i = row_idx;
    // certificate without row outputs still needs a row sweep: write its lists into the column buffers' place
    if (!(flags & HM_ROWS) && want_stats) { rows_v = pv; rows_i = pi; }
    int rc = HM_OK;
    auto dispatch = [&](const float* A, const float* B, int64_t ma, int64_t nb, const double* rb, const double* cb,
                        const unsigned long long* mxs, bool stt, bool tr, double* ov, int* oi) {
        const NormPlan pl = norm_plan(ma, nb);
        if (kind == HM_COST_L1)
            return norm_direction<HM_COST_L1>(st, A, B, ma, nb, d, rb, cb, mxs, k, stt, tr, pl, pv, pi, bs, ov, oi,
                                              stats, linf);
        if (kind == HM_COST_LINF)
            return norm_direction<HM_COST_LINF>(st, A, B, ma, nb, d, rb, cb, mxs, k, stt, tr, pl, pv, pi, bs, ov, oi,
                                                stats, linf);
        return norm_direction<HM_COST_L2>(st, A, B, ma, nb, d, rb, cb, mxs, k, stt, tr, pl, pv, pi, bs, ov, oi, stats,
                                          linf);
    };
    if ((flags & HM_ROWS) || want_stats) {
        if (!(flags & HM_ROWS)) return fail(HM_EINVAL, "norm pricing: HM_STATS requires HM_ROWS");
        rc = dispatch(X, Y, m, n, f, g, maxima, want_stats, false, rows_v, rows_i);
        if (rc != HM_OK) return rc;
        if (want_stats) {
            hipLaunchKernelGGL(norm_exact_max, dim3(1), dim3(256), 0, st, row_val, m, k, stats);
            HM_LAUNCH_CHECK("norm_exact_max");
        }
    }
    if (flags & HM_COLS) {
        rc = dispatch(Y, X, n, m, g, f, maxima + 2, false, true, col_val, col_idx);
        if (rc != HM_OK) return rc;
    }
    return HM_OK;
}

// Scratch of the allocation-free entry point: one array per GPU, for the life of the process. Host code reaches it
// only through the device address hipGetSymbolAddress returns (looked up once per device, under a lock).
constexpr size_t NORM_SCRATCH_BYTES = size_t(64) << 20;
__device__ __align__(256) unsigned char scratch[NORM_SCRATCH_BYTES];
constexpr int SCRATCH_DEVICES = 64;
std::mutex scratch_lock;
void* scratch_address[SCRATCH_DEVICES] = {};

int scratch_for_current_device(void** out) {
    int dev = -1;
    HM_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= SCRATCH_DEVICES) return fail(HM_EINVAL, "norm pricing (no-alloc): device %d out of range", dev);
    std::lock_guard<std::mutex> hold(scratch_lock);
    if (scratch_address[dev] == nullptr) {
        void* p = nullptr;
        HM_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (p == nullptr) return fail(HM_EHIP, "norm pricing (no-alloc): no device address for the scratch array");
        scratch_address[dev] = p;
    }
    *out = scratch_address[dev];
    return HM_OK;
}

}  // namespace

extern "C" int hm_pricing_norm(void* stream, const float* X, const float* Y, const double* f, const double* g,
                               int64_t m, int64_t n, int32_t d, int32_t k, int32_t kind, uint32_t flags,
                               double* row_val, int32_t* row_idx, double* col_val, int32_t* col_idx, double* stats,
                               void* workspace, size_t workspace_bytes) {
    return norm_scan_run(stream, X, Y, f, g, m, n, d, k, kind, flags, row_val, row_idx, col_val, col_idx, stats,
                         workspace, workspace_bytes);
}

extern "C" size_t hm_pricing_norm_noalloc_max_bytes(void) { return NORM_SCRATCH_BYTES; }

extern "C" int hm_pricing_norm_noalloc(void* stream, const float* X, const float* Y, const double* f,
                                       const double* g, int64_t m, int64_t n, int32_t d, int32_t k, int32_t kind,
                                       uint32_t flags, double* row_val, int32_t* row_idx, double* col_val,
                                       int32_t* col_idx, double* stats) {
    HM_CHECK_ARG(m >= 1 && n >= 1 && k >= 1 && k <= 32, "norm pricing requires nonempty inputs and 1 <= k <= 32");
    const size_t need = hm_pricing_norm_workspace_bytes(m, n, d, k, flags);
    if (need > NORM_SCRATCH_BYTES)
        return fail(HM_ENOSPC, "norm pricing (no-alloc): this call needs %zu bytes of scratch, above the %zu-byte static "
                               "scratch array; call hm_pricing_norm with a workspace instead",
                    need, NORM_SCRATCH_BYTES);
    void* scratch_ptr = nullptr;
    if (int rc = scratch_for_current_device(&scratch_ptr)) return rc;
    const ProfileOff no_events;  // timing events would be created on demand
    return norm_scan_run(stream, X, Y, f, g, m, n, d, k, kind, flags, row_val, row_idx, col_val, col_idx, stats,
                         scratch_ptr, NORM_SCRATCH_BYTES);
}
