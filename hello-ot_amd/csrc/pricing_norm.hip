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
// broadcast. Certificate sums are accumulated in fp32 per tile and flushed to fp64.
//
// Column lists, k <= 2 with rows and columns requested: they ride on the row sweep, so every pair is evaluated
// once. Every column keeps its running top-2 values in global memory (the largest and second largest score
// inserted so far, two atomic maxima: inserting v raises the first to max(v, first) and the second to
// min(v, previous first)); the running k-th value is a lower bound of the column's true k-th value. Each lane holds
// the fp32 entry thresholds of four of the tile's Y rows in registers; per pair a ballot compares the scores with
// the column's threshold (read from its lane), and only when some lane beats it does the wave take the exact fp64
// scores of the passing lanes, insert its k best of them into the running values and append those at or above the
// running k-th value to a candidate buffer. Workgroups start their Y sweep at staggered tiles, so most workgroups
// reach a column after its running values are set. The buffer is then grouped by column (counting sort) and each
// column keeps its k best. Should the buffer overflow, the column lists come from the role-swapped sweep instead
// (the same launches, gated on the overflow count).
// Otherwise, column lists come from a second sweep with the roles swapped (the score keeps the original
// association).
#include <hipcub/hipcub.hpp>

#include <mutex>

#include "common.h"

namespace hm {
namespace {

constexpr int NB_ROWS = 256;   // X rows per workgroup (one per thread)
constexpr int NT = 256;        // Y rows per LDS tile (fewer when d is large: the tile stays within 64 KiB)
constexpr int LDS_FLOATS = 15872;  // 62 KiB of dynamic LDS, leaving room for the static reduction buffer

// one appended column candidate of the fused sweep
struct ColCand {
    int j;     // column
    int i;     // row
    double v;  // exact fp64 score
};

// column state of the fused sweep (all per call, in the workspace)
struct ColArgs {
    unsigned long long* gthr;   // per column: double_key of the largest (gthr[j]) and second largest (gthr[n + j])
                                // values inserted so far
    ColCand* buf;               // appended candidates (capacity cap)
    unsigned long long* count;  // reserved slots; above cap means the buffer overflowed
    int* ccount;                // per column: candidates stored in the buffer (n + 1, last 0)
    int* coff;                  // exclusive scan of ccount (n + 1)
    int* order;                 // buffer slots grouped by column
    const unsigned long long* xmaxima;  // [max ||x||_1, max |f|] of the row side (the column slack)
    const double* g;                    // column duals (fp64)
    int64_t cap;
    int64_t n;
};

// the running k-th value of column j (k <= 2): a lower bound of the column's k-th best score
__device__ inline double running_kth(const ColArgs& ca, int64_t j, int k) {
    return key_double(__hip_atomic_load(ca.gthr + (k == 1 ? j : ca.n + j), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

// insert v into column j's running top-2 values
__device__ inline void running_insert(const ColArgs& ca, int64_t j, double v) {
    const unsigned long long kv = double_key(v);
    const unsigned long long o1 = atomicMax(ca.gthr + j, kv);
    const unsigned long long lo = kv < o1 ? kv : o1;
    if (lo != double_key(-INFINITY)) atomicMax(ca.gthr + ca.n + j, lo);
}

// the fused sweep's candidate capacity: each column receives its first workgroup's k entries and, after that,
// the entries that beat its threshold when their workgroup reaches it
inline int64_t fused_cap(int64_t n, int k) { return 16 * n * k + 65536; }

// buffer slots a wave reserves at a time (one atomic on the shared count per CHUNK appends; a wave's unused slots
// are marked empty when it ends)
constexpr int CHUNK = 64;

// a wave's current run of reserved buffer slots (uniform over the wave)
struct SlotRun {
    int64_t base = -1;  // first slot; -1: none yet
    int used = 0;
};

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

// the fp32 entry threshold of a column whose running k-th value is kth: any pair whose fp32 score is at or below
// it has an exact score below kth (one ulp down keeps it strictly below kth - slack)
__device__ inline float column_threshold(double kth, float cslack) {
    return (kth == -INFINITY) ? -INFINITY : nextafterf((float)(kth - (double)cslack), -INFINITY);
}

// marks the unused slots of the wave's run empty (every lane of the wave calls it)
__device__ inline void slot_run_close(const ColArgs& ca, const SlotRun& run) {
    if (run.base < 0 || run.base + CHUNK > ca.cap) return;
    for (int e = run.used + (int)(threadIdx.x & 63); e < CHUNK; e += 64) ca.buf[run.base + e].j = -1;
}

// lanes with `app` append (j, row, v) to the buffer through the wave's run of slots (every lane calls it)
__device__ inline void column_append(const ColArgs& ca, SlotRun& run, bool app, int64_t j, int row, double v) {
    const unsigned long long am = __ballot(app);
    if (!am) return;
    const int na = __popcll(am);
    if (run.base < 0 || run.used + na > CHUNK) {
        slot_run_close(ca, run);
        unsigned long long b = 0;
        if ((threadIdx.x & 63) == 0) b = atomicAdd(ca.count, (unsigned long long)CHUNK);
        run.base = (int64_t)(((unsigned long long)(unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)(b >> 32)) << 32) |
                             (unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)b));
        run.used = 0;
    }
    if (app && run.base + CHUNK <= ca.cap) {  // a run past the capacity: the buffer overflowed
        const int rank = __popcll(am & ((1ull << (threadIdx.x & 63)) - 1ull));
        ColCand cc;
        cc.j = (int)j;
        cc.i = row;
        cc.v = v;
        ca.buf[run.base + run.used + rank] = cc;
    }
    run.used += na;
}

// Lanes in `mask` (uniform) beat column j's threshold: the wave's k best of them by exact score (tie rule) enter the
// column's running values and are appended when at or above the running k-th value. Every lane of the wave calls it.
__device__ void column_enter(const ColArgs& ca, SlotRun& run, unsigned long long mask, int64_t j, float c, double fi,
                             int row, int k) {
    const int lane = threadIdx.x & 63;
    const double sig = (ca.g[j] - (double)c) + fi;
    bool take = ((mask >> lane) & 1ull) && sig == sig;
    if (__popcll(__ballot(take)) > k) {
        bool rest = take;
        int win0 = -1, win1 = -1;
        for (int s = 0; s < k; ++s) {
            double bv = rest ? sig : -INFINITY;
            int bi = rest ? row : INT_MAX;
            for (int o = 32; o >= 1; o >>= 1) {
                const double ov = __shfl_xor(bv, o, 64);
                const int oi = __shfl_xor(bi, o, 64);
                if (ov > bv || (ov == bv && oi < bi)) {
                    bv = ov;
                    bi = oi;
                }
            }
            if (s == 0) win0 = bi;
            else win1 = bi;
            rest = rest && row != bi;
        }
        take = take && (row == win0 || row == win1);
    }
    if (take) running_insert(ca, j, sig);
    column_append(ca, run, take && sig >= running_kth(ca, j, k), j, row, sig);
}

// EXACT: d == DR (a multiple of 4), so Y rows in LDS are whole float4s.
// FUSED (K == 2, rows and columns): column lists as described at the top of this file; tiles start staggered.
// gate: the role-swapped column sweep of a fused call runs only when the fused buffer overflowed (*gate > cap).
// The fused sweep is held to 64 VGPRs (eight waves per SIMD): the slow path's temporaries then spill to scratch,
// which costs far less than the three waves per SIMD its registers would take from the pair loop.
template <int KIND, int K, int DR, bool EXACT, bool FUSED, bool ST>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(FUSED ? 8 : 1))) void norm_sweep(const float* __restrict__ X, const float* __restrict__ Y, int64_t m,
                                                  int64_t n, int d, const double* __restrict__ rb,
                                                  const double* __restrict__ cb,
                                                  const unsigned long long* __restrict__ ymaxima, int k,
                                                  int64_t seg_len, double* __restrict__ part_v, int* __restrict__ part_i,
                                                  double* __restrict__ blockstats, int STATS_, int TRANSPOSED, int ntile,
                                                  ColArgs ca, const unsigned long long* __restrict__ gate,
                                                  int64_t gate_cap) {
    static_assert(!FUSED || K == 2, "fused column lists hold two slots");
    // sweeps without the certificate (ST = false) drop its code, and with it a per-pair test of the runtime flag
    const int STATS = ST ? STATS_ : 0;
    if (gate != nullptr && *gate <= (unsigned long long)gate_cap) return;  // uniform: the fused lists are complete
    extern __shared__ float4 smem4[];
    float* smem = reinterpret_cast<float*>(smem4);
    float* sy = smem;                            // ntile * d
    float* scb = smem + (size_t)ntile * d;       // ntile (column duals as fp32)
    __shared__ double sRed[4][5];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
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
    // the same bound over every pair of a column (row side at its maxima)
    const float cslack = FUSED ? (float)((key_double(ca.xmaxima[0]) + ymax1 + gmax + key_double(ca.xmaxima[1])) * 4.0 *
                                         5.9604644775390625e-08 * (1.0 + 1e-6) + 1e-37)
                               : 0.0f;

    double v[K];
    int id[K];
#pragma unroll
    for (int s = 0; s < K; ++s) { v[s] = -INFINITY; id[s] = -1; }
    float thr = -INFINITY;
    double num64 = 0.0, den64 = 0.0, cnt64 = 0.0;
    float cmax = 0.0f;

    SlotRun run;  // fused: this wave's buffer slots
    // fused: the tiles in rotated order, starting along a Weyl sequence (stride about 0.618 of the tiles), so that the
    // workgroups resident at any time start spread over all tiles and each column is reached by one workgroup after
    // another; a column that many workgroups reach before its running values are set costs each of them slow paths
    int64_t shift = 0, span = 0;
    if constexpr (FUSED) {
        const int64_t ntiles = (y_end - y_begin + ntile - 1) / ntile;
        shift = (((int64_t)blockIdx.x * (((ntiles * 633) >> 10) | 1)) % ntiles) * ntile;
        span = ntiles * ntile;
    }
    for (int64_t th = y_begin; th < y_end; th += ntile) {
        int64_t t0 = th;
        if constexpr (FUSED) {
            t0 += shift;
            if (t0 >= y_begin + span) t0 -= span;
        }
        const int cnt = (int)((y_end - t0) < ntile ? (y_end - t0) : ntile);
        __syncthreads();
        for (int e = tid; e < cnt * d; e += 256) sy[e] = Y[t0 * d + e];
        for (int e = tid; e < cnt; e += 256) scb[e] = (float)cb[t0 + e];
        // fused: this lane's column thresholds, Y rows q * 64 + lane of the tile (any value of a column's monotone
        // running k-th value is a valid lower bound)
        float ct[FUSED ? 4 : 1];
        if constexpr (FUSED) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                ct[q] = INFINITY;
                if (q * 64 + lane < cnt) ct[q] = column_threshold(running_kth(ca, t0 + q * 64 + lane, k), cslack);
            }
        }
        __syncthreads();
        float tnum = 0.0f, tden = 0.0f;
        unsigned tc = 0;
        if (FUSED || row_ok) {  // fused: every lane takes part in the column ballots
#pragma unroll
          for (int q = 0; q < (FUSED ? 4 : 1); ++q) {
            const int jb = FUSED ? q * 64 : 0;
            const int je = FUSED ? (cnt < jb + 64 ? cnt : jb + 64) : cnt;
            for (int jj = jb; jj < je; ++jj) {
                const float* yj = sy + (size_t)jj * d;
                float c;
                if constexpr (EXACT) c = distance_exact<KIND, DR>(x, yj);
                else if (DR > 0) c = distance_reg<KIND, (DR > 0 ? DR : 1)>(x, yj, d);
                else c = distance_mem<KIND>(X + (row_ok ? row : 0) * d, yj, d);  // fused: lanes past m read row 0
                const float s32 = (scb[jj] - c) + fi32;
                if constexpr (FUSED) {
                    const float tcol = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ct[q]), jj - jb));
                    const unsigned long long mask = __ballot(row_ok && s32 > tcol);
                    if (mask) column_enter(ca, run, mask, t0 + jj, c, fi, (int)row, k);  // rare: the column visits once
                }
                if (row_ok && s32 > thr) {
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
                if (STATS && row_ok) {
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
        }
        if (STATS) {
            num64 += (double)tnum;
            den64 += (double)tden;
            cnt64 += (double)tc;
        }
    }
    if constexpr (FUSED) slot_run_close(ca, run);
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

// fp64 costs (HM_FP64, the reference's direct_norm_fp64: cost.cu:10-104 with CHAINS = 1 and a double accumulator):
// each feature difference is taken in fp64 from the fp32 inputs and the features combine one after another in
// feature order; l2 accumulates fma(z, z, acc) (nvcc contracts the multiply-add) and takes one fp64 sqrt.
template <int KIND>
__device__ inline double feature_op64(double part, double z) {
    if (KIND == HM_COST_L1) return part + fabs(z);
    if (KIND == HM_COST_LINF) return fmax(part, fabs(z));
    return fma(z, z, part);
}

// One thread per X row (its features in registers as fp64 when DR > 0, else read from memory), Y tiles in LDS as
// fp32 with their duals as fp64. Scores sigma = (g_j - c) + f_i, the row lists and the certificate are fp64; there
// is no fp32 filter. The lists are exact whatever the order of the pairs, the certificate sums fp64-grade.
template <int KIND, int K, int DR>
__global__ __launch_bounds__(256) void norm_sweep64(const float* __restrict__ X, const float* __restrict__ Y, int64_t m,
                                                    int64_t n, int d, const double* __restrict__ rb,
                                                    const double* __restrict__ cb, int k, int64_t seg_len,
                                                    double* __restrict__ part_v, int* __restrict__ part_i,
                                                    double* __restrict__ blockstats, int STATS, int TRANSPOSED,
                                                    int ntile) {
    extern __shared__ float4 smem4[];
    double* scb = reinterpret_cast<double*>(smem4);   // ntile column duals
    float* sy = reinterpret_cast<float*>(scb + ntile);  // ntile * d features
    __shared__ double sRed[4][5];
    const int tid = threadIdx.x;
    const int64_t row = (int64_t)blockIdx.x * NB_ROWS + tid;
    const bool row_ok = row < m;
    const int64_t y_begin = (int64_t)blockIdx.y * seg_len;
    const int64_t y_end = y_begin + seg_len < n ? y_begin + seg_len : n;

    double x[DR > 0 ? DR : 1];
    if (DR > 0) {
#pragma unroll
        for (int t = 0; t < (DR > 0 ? DR : 1); ++t) x[t] = (row_ok && t < d) ? (double)X[row * d + t] : 0.0;
    }
    const float* xr = X + (row_ok ? row : 0) * d;
    const double fi = row_ok ? rb[row] : 0.0;
    double v[K];
    int id[K];
#pragma unroll
    for (int s = 0; s < K; ++s) { v[s] = -INFINITY; id[s] = -1; }
    double num = 0.0, den = 0.0, cnt = 0.0, cmax = 0.0;
    for (int64_t t0 = y_begin; t0 < y_end; t0 += ntile) {
        const int tn = (int)((y_end - t0) < ntile ? (y_end - t0) : ntile);
        __syncthreads();
        for (int e = tid; e < tn * d; e += 256) sy[e] = Y[t0 * d + e];
        for (int e = tid; e < tn; e += 256) scb[e] = cb[t0 + e];
        __syncthreads();
        if (!row_ok) continue;
        for (int jj = 0; jj < tn; ++jj) {
            const float* yj = sy + (size_t)jj * d;
            double c = 0.0;
            if (DR > 0) {
#pragma unroll
                for (int t = 0; t < (DR > 0 ? DR : 1); ++t)
                    if (t < d) c = feature_op64<KIND>(c, x[t] - (double)yj[t]);
            } else {
                for (int t = 0; t < d; ++t) c = feature_op64<KIND>(c, (double)xr[t] - (double)yj[t]);
            }
            if (KIND == HM_COST_L2) c = sqrt(c);
            const double sig = TRANSPOSED ? (fi - c) + scb[jj] : (scb[jj] - c) + fi;
            const int j = (int)(t0 + jj);
            if (sig == sig && better(sig, j, v[k - 1], id[k - 1])) put_sorted<K>(v, id, k, sig, j);
            if (STATS) {
                den = fma(c, c, den);
                cmax = fmax(cmax, c);
                if (sig > 0.0) {
                    num = fma(sig, sig, num);
                    cnt += 1.0;
                }
            }
        }
    }
    if (row_ok) {
        double* ov = part_v + ((int64_t)blockIdx.y * m + row) * k;
        int* oi = part_i + ((int64_t)blockIdx.y * m + row) * k;
        for (int s = 0; s < k; ++s) { ov[s] = v[s]; oi[s] = id[s]; }
    }
    if (STATS) {
        const int lane = tid & 63, wave = tid >> 6;
        double r[5] = {num, den, cnt, 0.0, cmax};  // slot 3: exact row maximum later
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

// merge S exact segment lists per row (tie rule), one thread per row; gated like norm_sweep
template <int K>
__global__ void norm_merge(const double* __restrict__ part_v, const int* __restrict__ part_i, int64_t m, int S, int k,
                           double* __restrict__ out_v, int* __restrict__ out_i, const unsigned long long* gate,
                           int64_t gate_cap) {
    if (gate != nullptr && *gate <= (unsigned long long)gate_cap) return;
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

// fused column state: thresholds at double_key(-inf), counts at zero
__global__ void cols_clear(unsigned long long* __restrict__ gthr, int* __restrict__ ccount, int64_t n,
                           unsigned long long* __restrict__ count) {
    const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j < n) gthr[j] = gthr[n + j] = double_key(-INFINITY);
    if (j <= n) ccount[j] = 0;
    if (j == 0) *count = 0ull;
}

// candidates per column (empty slots skipped)
__global__ void cols_count(const ColCand* __restrict__ buf, const unsigned long long* __restrict__ count, int64_t cap,
                           int* __restrict__ ccount) {
    const unsigned long long c = *count;
    if (c > (unsigned long long)cap) return;
    for (int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; s < (int64_t)c; s += (int64_t)gridDim.x * blockDim.x) {
        const int j = buf[s].j;
        if (j >= 0) atomicAdd(ccount + j, 1);
    }
}

// buffer slots grouped by column: slot s of column j goes to coff[j] + (its rank among the column's arrivals);
// ccount counts back down to zero
__global__ void cols_group(const ColCand* __restrict__ buf, const unsigned long long* __restrict__ count, int64_t cap,
                           const int* __restrict__ coff, int* __restrict__ ccount, int* __restrict__ order) {
    const unsigned long long c = *count;
    if (c > (unsigned long long)cap) return;  // overflowed: the role-swapped sweep gives the columns
    for (int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; s < (int64_t)c; s += (int64_t)gridDim.x * blockDim.x) {
        const int j = buf[s].j;
        if (j >= 0) order[coff[j] + atomicSub(ccount + j, 1) - 1] = (int)s;
    }
}

// each column's k best among its candidates (tie rule), one thread per column
template <int K>
__global__ void cols_select(const ColCand* __restrict__ buf, const unsigned long long* __restrict__ count, int64_t cap,
                            const int* __restrict__ coff, const int* __restrict__ order, int64_t n, int k,
                            double* __restrict__ out_v, int* __restrict__ out_i) {
    if (*count > (unsigned long long)cap) return;
    const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= n) return;
    double v[K];
    int id[K];
#pragma unroll
    for (int s = 0; s < K; ++s) { v[s] = -INFINITY; id[s] = -1; }
    for (int e = coff[j]; e < coff[j + 1]; ++e) {
        const ColCand c = buf[order[e]];
        put_sorted<K>(v, id, k, c.v, c.i);
    }
    for (int s = 0; s < k; ++s) { out_v[j * k + s] = v[s]; out_i[j * k + s] = id[s]; }
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

// columns ride on the row sweep (k <= 2 with rows and columns requested; buffer slots in int32)
inline bool fusable(int64_t n, int k, uint32_t flags) {
    return k <= 2 && (flags & HM_ROWS) && (flags & HM_COLS) && !(flags & HM_FP64) && fused_cap(n, k) < INT32_MAX;
}

struct NormWork {
    double* pv;  // segment lists (rows, then the role-swapped columns)
    int* pi;
    double* bs;  // per-workgroup certificate partials
    unsigned long long* maxima;  // [0..1] Y side, [2..3] X side
    // fused columns
    unsigned long long* gthr;
    ColCand* buf;
    unsigned long long* count;
    int *ccount, *coff, *order;
    void* scan_tmp;
    size_t scan_bytes;
    int64_t cap;
};

inline size_t scan_tmp_bytes(int64_t n) {
    size_t bytes = 0;
    (void)hipcub::DeviceScan::ExclusiveSum(nullptr, bytes, (const int*)nullptr, (int*)nullptr, (int)(n + 1));
    return bytes;
}

// cap > 0: the fused path with a candidate buffer of cap entries
template <class A>
void norm_layout(A& a, int64_t m, int64_t n, int k, uint32_t flags, int64_t cap, NormWork& w) {
    const NormPlan pr = norm_plan(m, n), pc = norm_plan(n, m);
    size_t entries = 0;
    if (flags & (HM_ROWS | HM_STATS)) entries = (size_t)pr.S * m * k;
    if (flags & HM_COLS) {
        const size_t c = (size_t)pc.S * n * k;
        if (c > entries) entries = c;
    }
    w.pv = a.template take<double>(entries > 0 ? entries : 1);
    w.pi = a.template take<int>(entries > 0 ? entries : 1);
    const int64_t br = ((m + NB_ROWS - 1) / NB_ROWS) * pr.S, bc = ((n + NB_ROWS - 1) / NB_ROWS) * pc.S;
    w.bs = a.template take<double>((size_t)5 * (br > bc ? br : bc));
    w.maxima = a.template take<unsigned long long>(4);
    w.cap = cap;
    if (cap <= 0) return;
    w.gthr = a.template take<unsigned long long>(2 * n);
    w.count = a.template take<unsigned long long>(1);
    w.ccount = a.template take<int>(n + 1);
    w.coff = a.template take<int>(n + 1);
    w.order = a.template take<int>(w.cap);
    w.buf = a.template take<ColCand>(w.cap);
    w.scan_bytes = scan_tmp_bytes(n);
    w.scan_tmp = a.template take<char>(w.scan_bytes > 0 ? w.scan_bytes : 1);
}

// one sweep direction: rows of X against Y (TRANSPOSED: the roles swapped for the column lists)
struct Direction {
    const float *X, *Y;
    int64_t m, n;
    const double *rb, *cb;
    const unsigned long long* ymaxima;
    bool stats, transposed;
    NormPlan plan;
    double* out_v;
    int* out_i;
    ColArgs cols;                     // fused columns (cols.gthr == nullptr: none)
    const unsigned long long* gate;   // role-swapped column sweep of a fused call
    int64_t gate_cap;
};

template <int KIND, int K, int DR, bool EXACT, bool FUSED>
int norm_direction_t(hipStream_t st, const Direction& D, int d, int k, const NormWork& w, double* stats_out, int linf) {
    dim3 grid((unsigned)((D.m + NB_ROWS - 1) / NB_ROWS), (unsigned)D.plan.S);
    int ntile = NT;
    while (ntile > 1 && (size_t)ntile * (d + 1) > LDS_FLOATS) ntile >>= 1;
    if ((size_t)ntile * (d + 1) > LDS_FLOATS) return fail(HM_EINVAL, "norm pricing supports d <= %d", LDS_FLOATS - 1);
    const size_t shmem = ((size_t)ntile * d + ntile) * sizeof(float);
    prof_begin(st, D.gate != nullptr ? "norm_sweep_swapped" : "norm_sweep");
    if (D.stats)
        hipLaunchKernelGGL((norm_sweep<KIND, K, DR, EXACT, FUSED, true>), grid, dim3(256), shmem, st, D.X, D.Y, D.m, D.n,
                           d, D.rb, D.cb, D.ymaxima, k, D.plan.seg_len, w.pv, w.pi, w.bs, 1, (int)D.transposed, ntile,
                           D.cols, D.gate, D.gate_cap);
    else
        hipLaunchKernelGGL((norm_sweep<KIND, K, DR, EXACT, FUSED, false>), grid, dim3(256), shmem, st, D.X, D.Y, D.m,
                           D.n, d, D.rb, D.cb, D.ymaxima, k, D.plan.seg_len, w.pv, w.pi, w.bs, 0, (int)D.transposed,
                           ntile, D.cols, D.gate, D.gate_cap);
    prof_end(st);
    HM_LAUNCH_CHECK("norm_sweep");
    hipLaunchKernelGGL((norm_merge<K>), dim3((unsigned)((D.m + 255) / 256)), dim3(256), 0, st, w.pv, w.pi, D.m, D.plan.S,
                       k, D.out_v, D.out_i, D.gate, D.gate_cap);
    HM_LAUNCH_CHECK("norm_merge");
    if (D.stats) {
        hipLaunchKernelGGL(norm_reduce_stats, dim3(1), dim3(256), 0, st, w.bs, (int64_t)grid.x * grid.y, stats_out, linf);
        HM_LAUNCH_CHECK("norm_reduce_stats");
    }
    return HM_OK;
}

template <int KIND, int K, bool FUSED>
int norm_direction_d(hipStream_t st, const Direction& D, int d, int k, const NormWork& w, double* stats_out, int linf) {
    if (d == 8) return norm_direction_t<KIND, K, 8, true, FUSED>(st, D, d, k, w, stats_out, linf);
    if (d <= 8) return norm_direction_t<KIND, K, 8, false, FUSED>(st, D, d, k, w, stats_out, linf);
    if (d <= 64) return norm_direction_t<KIND, K, 64, false, FUSED>(st, D, d, k, w, stats_out, linf);
    return norm_direction_t<KIND, K, 0, false, FUSED>(st, D, d, k, w, stats_out, linf);
}

template <int KIND>
int norm_direction(hipStream_t st, const Direction& D, int d, int k, const NormWork& w, double* stats_out, int linf) {
    if (D.cols.gthr != nullptr) return norm_direction_d<KIND, 2, true>(st, D, d, k, w, stats_out, linf);
    switch (kbucket(k)) {
        case 2: return norm_direction_d<KIND, 2, false>(st, D, d, k, w, stats_out, linf);
        case 8: return norm_direction_d<KIND, 8, false>(st, D, d, k, w, stats_out, linf);
        case 32: return norm_direction_d<KIND, 32, false>(st, D, d, k, w, stats_out, linf);
    }
    return fail(HM_EINVAL, "unsupported k");
}

template <int KIND, int K, int DR>
int norm_direction64_t(hipStream_t st, const Direction& D, int d, int k, const NormWork& w, double* stats_out,
                       int linf) {
    dim3 grid((unsigned)((D.m + NB_ROWS - 1) / NB_ROWS), (unsigned)D.plan.S);
    const size_t budget = (size_t)LDS_FLOATS * sizeof(float);
    auto bytes = [d](int t) { return (size_t)t * sizeof(double) + (size_t)t * d * sizeof(float); };
    int ntile = NT;
    while (ntile > 1 && bytes(ntile) > budget) ntile >>= 1;
    if (bytes(ntile) > budget) return fail(HM_EINVAL, "fp64 norm pricing supports d <= %d", LDS_FLOATS - 2);
    prof_begin(st, D.transposed ? "norm_sweep64_swapped" : "norm_sweep64");
    hipLaunchKernelGGL((norm_sweep64<KIND, K, DR>), grid, dim3(256), bytes(ntile), st, D.X, D.Y, D.m, D.n, d, D.rb, D.cb,
                       k, D.plan.seg_len, w.pv, w.pi, w.bs, (int)D.stats, (int)D.transposed, ntile);
    prof_end(st);
    HM_LAUNCH_CHECK("norm_sweep64");
    hipLaunchKernelGGL((norm_merge<K>), dim3((unsigned)((D.m + 255) / 256)), dim3(256), 0, st, w.pv, w.pi, D.m, D.plan.S,
                       k, D.out_v, D.out_i, nullptr, (int64_t)0);
    HM_LAUNCH_CHECK("norm_merge");
    if (D.stats) {
        hipLaunchKernelGGL(norm_reduce_stats, dim3(1), dim3(256), 0, st, w.bs, (int64_t)grid.x * grid.y, stats_out, linf);
        HM_LAUNCH_CHECK("norm_reduce_stats");
    }
    return HM_OK;
}

template <int KIND, int K>
int norm_direction64_d(hipStream_t st, const Direction& D, int d, int k, const NormWork& w, double* stats_out, int linf) {
    if (d <= 8) return norm_direction64_t<KIND, K, 8>(st, D, d, k, w, stats_out, linf);
    if (d <= 32) return norm_direction64_t<KIND, K, 32>(st, D, d, k, w, stats_out, linf);
    if (d <= 64) return norm_direction64_t<KIND, K, 64>(st, D, d, k, w, stats_out, linf);
    return norm_direction64_t<KIND, K, 0>(st, D, d, k, w, stats_out, linf);
}

template <int KIND>
int norm_direction64(hipStream_t st, const Direction& D, int d, int k, const NormWork& w, double* stats_out, int linf) {
    switch (kbucket(k)) {
        case 2: return norm_direction64_d<KIND, 2>(st, D, d, k, w, stats_out, linf);
        case 8: return norm_direction64_d<KIND, 8>(st, D, d, k, w, stats_out, linf);
        case 32: return norm_direction64_d<KIND, 32>(st, D, d, k, w, stats_out, linf);
    }
    return fail(HM_EINVAL, "unsupported k");
}

inline size_t norm_workspace(int64_t m, int64_t n, int k, uint32_t flags, int64_t cap) {
    Sizer s;
    NormWork w;
    norm_layout(s, m, n, k, flags, cap, w);
    return s.used;
}

// the candidate capacity a workspace of `bytes` holds: the full capacity when it fits, else (with partial) what fits
// (the fused path stays exact with any capacity: an overflow hands the columns to the role-swapped sweep); 0: two
// sweeps
inline int64_t fused_capacity(int64_t m, int64_t n, int k, uint32_t flags, size_t bytes, bool partial) {
    if (!fusable(n, k, flags)) return 0;
    const int64_t full = fused_cap(n, k);
    if (norm_workspace(m, n, k, flags, full) <= bytes) return full;
    if (!partial) return 0;
    const size_t fixed = norm_workspace(m, n, k, flags, 1);
    const size_t per = sizeof(ColCand) + sizeof(int);
    if (bytes < fixed + 512 + per) return 0;
    int64_t cap = (int64_t)((bytes - fixed - 512) / per);  // 512: the two arrays' rounding to 256 bytes
    if (cap > full) cap = full;
    return norm_workspace(m, n, k, flags, cap) <= bytes ? cap : 0;
}

}  // namespace
}  // namespace hm

using namespace hm;

// the workspace of the fused path where it applies (a smaller workspace still runs the two-sweep path)
extern "C" size_t hm_pricing_norm_workspace_bytes(int64_t m, int64_t n, int32_t d, int32_t k, uint32_t flags) {
    (void)d;
    if (m < 1 || n < 1 || k < 1 || k > 32) return 0;
    return norm_workspace(m, n, k, flags, fusable(n, k, flags) ? fused_cap(n, k) : 0);
}

namespace {

// The scan with its scratch in `workspace` (caller memory, or the static scratch array of hm_pricing_norm_noalloc).
// Everything the scratch holds is written before it is read; maxima, thresholds and counts are cleared by kernels,
// not memsets.
int norm_scan_run(void* stream, const float* X, const float* Y, const double* f, const double* g, int64_t m,
                  int64_t n, int32_t d, int32_t k, int32_t kind, uint32_t flags, double* row_val, int32_t* row_idx,
                  double* col_val, int32_t* col_idx, double* stats, void* workspace, size_t workspace_bytes,
                  bool partial_buffer) {
    HM_CHECK_ARG(X && Y && f && g, "norm pricing: feature and dual pointers are required");
    HM_CHECK_ARG(m >= 1 && n >= 1 && d >= 1 && m < INT32_MAX && n < INT32_MAX,
                 "norm pricing requires nonempty inputs with int32 dimensions");
    HM_CHECK_ARG(k >= 1 && k <= 32, "norm pricing requires 1 <= k <= 32 (k=%d)", k);
    HM_CHECK_ARG(kind == HM_COST_L1 || kind == HM_COST_LINF || kind == HM_COST_L2, "unsupported norm cost %d", kind);
    HM_CHECK_ARG(!(flags & HM_ROWS) || (row_val && row_idx), "HM_ROWS requires row outputs");
    HM_CHECK_ARG(!(flags & HM_COLS) || (col_val && col_idx), "HM_COLS requires column outputs");
    HM_CHECK_ARG(!(flags & HM_STATS) || stats, "HM_STATS requires a stats output");
    HM_CHECK_ARG(!(flags & HM_STATS) || (flags & HM_ROWS), "norm pricing: HM_STATS requires HM_ROWS");
    HM_CHECK_ARG(workspace != nullptr, "workspace is required");
    const size_t need = norm_workspace(m, n, k, flags, 0);
    if (workspace_bytes < need)
        return fail(HM_ENOSPC, "norm pricing workspace too small: %zu < %zu bytes", workspace_bytes, need);
    const int64_t cap = fused_capacity(m, n, k, flags, workspace_bytes, partial_buffer);
    const bool fused = cap > 0;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    Arena a(workspace, workspace_bytes);
    NormWork w;
    norm_layout(a, m, n, k, flags, cap, w);
    hipLaunchKernelGGL(norm_zero, dim3(1), dim3(64), 0, st, w.maxima, 4);
    HM_LAUNCH_CHECK("norm_zero");
    hipLaunchKernelGGL(norm_prep, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, Y, n, d, g, w.maxima);
    HM_LAUNCH_CHECK("norm_prep");
    hipLaunchKernelGGL(norm_prep, dim3((unsigned)((m + 255) / 256)), dim3(256), 0, st, X, m, d, f, w.maxima + 2);
    HM_LAUNCH_CHECK("norm_prep");
    const int linf = (flags & HM_LINF) ? 1 : 0;
    const bool fp64 = (flags & HM_FP64) != 0;
    auto dispatch = [&](const Direction& D) {
        if (fp64) {
            if (kind == HM_COST_L1) return norm_direction64<HM_COST_L1>(st, D, d, k, w, stats, linf);
            if (kind == HM_COST_LINF) return norm_direction64<HM_COST_LINF>(st, D, d, k, w, stats, linf);
            return norm_direction64<HM_COST_L2>(st, D, d, k, w, stats, linf);
        }
        if (kind == HM_COST_L1) return norm_direction<HM_COST_L1>(st, D, d, k, w, stats, linf);
        if (kind == HM_COST_LINF) return norm_direction<HM_COST_LINF>(st, D, d, k, w, stats, linf);
        return norm_direction<HM_COST_L2>(st, D, d, k, w, stats, linf);
    };
    ColArgs none{};
    ColArgs cols{};
    if (fused) {
        cols.gthr = w.gthr;
        cols.buf = w.buf;
        cols.count = w.count;
        cols.ccount = w.ccount;
        cols.coff = w.coff;
        cols.order = w.order;
        cols.xmaxima = w.maxima + 2;
        cols.cap = w.cap;
        cols.n = n;
        cols.g = g;
        hipLaunchKernelGGL(cols_clear, dim3((unsigned)((n + 256) / 256)), dim3(256), 0, st, w.gthr, w.ccount, n, w.count);
        HM_LAUNCH_CHECK("cols_clear");
    }
    if (flags & HM_ROWS) {
        const Direction D{X, Y, m, n, f, g, w.maxima, (flags & HM_STATS) != 0, false, norm_plan(m, n), row_val, row_idx,
                          fused ? cols : none, nullptr, 0};
        if (int rc = dispatch(D)) return rc;
        if (flags & HM_STATS) {
            hipLaunchKernelGGL(norm_exact_max, dim3(1), dim3(256), 0, st, row_val, m, k, stats);
            HM_LAUNCH_CHECK("norm_exact_max");
        }
    }
    if (fused) {
        prof_begin(st, "norm_cols");
        hipLaunchKernelGGL(cols_count, dim3(2048), dim3(256), 0, st, w.buf, w.count, w.cap, w.ccount);
        HM_LAUNCH_CHECK("cols_count");
        HM_HIP(hipcub::DeviceScan::ExclusiveSum(w.scan_tmp, w.scan_bytes, w.ccount, w.coff, (int)(n + 1), st));
        hipLaunchKernelGGL(cols_group, dim3(2048), dim3(256), 0, st, w.buf, w.count, w.cap, w.coff, w.ccount, w.order);
        HM_LAUNCH_CHECK("cols_group");
        hipLaunchKernelGGL((cols_select<2>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, w.buf, w.count, w.cap,
                           w.coff, w.order, n, k, col_val, col_idx);
        HM_LAUNCH_CHECK("cols_select");
        prof_end(st);
        if (profiling()) {  // candidates appended (a count above the capacity means the buffer overflowed)
            unsigned long long c = 0;
            HM_HIP(hipMemcpyAsync(&c, w.count, sizeof(c), hipMemcpyDeviceToHost, st));
            HM_HIP(hipStreamSynchronize(st));
            prof_count("norm_cols_candidates", (int64_t)c);
            prof_count(c > (unsigned long long)w.cap ? "norm_cols_overflow" : "norm_cols_fused", 1);
        }
    }
    if (flags & HM_COLS) {
        // the role-swapped sweep; in a fused call it runs only if the candidate buffer overflowed
        const Direction D{Y, X, n, m, g, f, w.maxima + 2, false, true, norm_plan(n, m), col_val, col_idx, none,
                          fused ? w.count : nullptr, w.cap};
        if (int rc = dispatch(D)) return rc;
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
                         workspace, workspace_bytes, true);
}

extern "C" size_t hm_pricing_norm_noalloc_max_bytes(void) { return NORM_SCRATCH_BYTES; }

extern "C" int hm_pricing_norm_noalloc(void* stream, const float* X, const float* Y, const double* f,
                                       const double* g, int64_t m, int64_t n, int32_t d, int32_t k, int32_t kind,
                                       uint32_t flags, double* row_val, int32_t* row_idx, double* col_val,
                                       int32_t* col_idx, double* stats) {
    HM_CHECK_ARG(m >= 1 && n >= 1 && k >= 1 && k <= 32, "norm pricing requires nonempty inputs and 1 <= k <= 32");
    // the two-sweep path's scratch; the fused path runs when its larger scratch fits as well
    const size_t need = norm_workspace(m, n, k, flags, 0);
    if (need > NORM_SCRATCH_BYTES)
        return fail(HM_ENOSPC, "norm pricing (no-alloc): this call needs %zu bytes of scratch, above the %zu-byte static "
                               "scratch array; call hm_pricing_norm with a workspace instead",
                    need, NORM_SCRATCH_BYTES);
    void* scratch_ptr = nullptr;
    if (int rc = scratch_for_current_device(&scratch_ptr)) return rc;
    const ProfileOff no_events;  // timing events would be created on demand
    // the fused path only with its full candidate buffer: a partial one that overflows would cost both sweeps
    return norm_scan_run(stream, X, Y, f, g, m, n, d, k, kind, flags, row_val, row_idx, col_val, col_idx, stats,
                         scratch_ptr, NORM_SCRATCH_BYTES, false);
}
