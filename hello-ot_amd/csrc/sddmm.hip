// SDDMM cost evaluation on the active support (gfx950).
//
// l2^2: out[e] = (p_i + q_j) - scale*dot64(x_i, y_j)  (costs/pairs.py:394-407 association; gpu_resident/cost.py:59-71)
// norms: fp64 l1 / linf / l2 of (x_i - y_j)           (norm_cost_scan_kernel.cu:233-245, without perturbation)
//
// dot64 / norm partials use the fixed 64-lane order: lane l accumulates features l, l+64, ... sequentially
// and the lanes are combined by a halving-stride tree. For d <= G (G a power of two <= 64) a group of G
// lanes per pair produces the same bits: the missing lanes only ever add +0.0.
#include "common.h"

namespace hm {
namespace {

// CSR rows: one wave per row, x_i cached in registers when d <= 64*XR.
template <int XR>
__global__ __launch_bounds__(256) void sddmm_l2sq_csr_kernel(const float* __restrict__ X, const float* __restrict__ Y,
                                                             const double* __restrict__ p, const double* __restrict__ q,
                                                             const int32_t* __restrict__ rowptr,
                                                             const int32_t* __restrict__ col, int64_t m, int d,
                                                             double scale, double* __restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int64_t waves = (int64_t)gridDim.x * (blockDim.x >> 6);
    for (int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); row < m; row += waves) {
        const float* xr = X + row * (int64_t)d;
        const int32_t e0 = rowptr[row], e1 = rowptr[row + 1];
        if (e0 >= e1) continue;
        const double pi = p[row];
        if (XR > 0) {
            float xv[XR > 0 ? XR : 1];
#pragma unroll
            for (int t = 0; t < XR; ++t) xv[t] = (lane + 64 * t < d) ? xr[lane + 64 * t] : 0.0f;
            // U gathered Y rows in flight per step; each pair keeps the fixed lane order
            constexpr int U = 4;
            int32_t e = e0;
            for (; e + U <= e1; e += U) {
                const float* yp[U];
                double a[U];
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    yp[u] = Y + (int64_t)col[e + u] * d;
                    a[u] = 0.0;
                }
#pragma unroll
                for (int t = 0; t < XR; ++t) {
                    const int k = lane + 64 * t;
                    if (k < d) {
#pragma unroll
                        for (int u = 0; u < U; ++u) a[u] = a[u] + (double)xv[t] * (double)yp[u][k];
                    }
                }
#pragma unroll
                for (int u = 0; u < U; ++u) a[u] = wave_tree_sum(a[u]);
                if (lane < U) {
                    double mine = a[0];
#pragma unroll
                    for (int u = 1; u < U; ++u)
                        if (lane == u) mine = a[u];
                    const int64_t j = col[e + lane];
                    out[e + lane] = (pi + q[j]) - scale * mine;
                }
            }
            for (; e < e1; ++e) {
                const int64_t j0 = col[e];
                const float* y0 = Y + j0 * d;
                double a0 = 0.0;
#pragma unroll
                for (int t = 0; t < XR; ++t) {
                    const int k = lane + 64 * t;
                    if (k < d) a0 = a0 + (double)xv[t] * (double)y0[k];
                }
                a0 = wave_tree_sum(a0);
                if (lane == 0) out[e] = (pi + q[j0]) - scale * a0;
            }
        } else {
            for (int32_t e = e0; e < e1; ++e) {
                const int64_t j = col[e];
                const double dot = wave_dot64(xr, Y + j * d, d, lane);
                if (lane == 0) out[e] = (pi + q[j]) - scale * dot;
            }
        }
    }
}

template <int G>
__device__ inline double group_tree_sum(double v) {
#pragma unroll
    for (int s = G / 2; s >= 1; s >>= 1) v = v + __shfl_down(v, s, G);
    return v;
}
template <int G>
__device__ inline double group_tree_max(double v) {
#pragma unroll
    for (int s = G / 2; s >= 1; s >>= 1) v = fmax(v, __shfl_down(v, s, G));
    return v;
}

// COO pairs: groups of G lanes per pair (G = 64 handles any d; smaller G only when d <= G).
template <int G>
__global__ __launch_bounds__(256) void pair_costs_l2sq_kernel(const float* __restrict__ X, const float* __restrict__ Y,
                                                              const double* __restrict__ p, const double* __restrict__ q,
                                                              const int64_t* __restrict__ rows,
                                                              const int64_t* __restrict__ cols, int64_t count, int d,
                                                              double scale, double* __restrict__ out) {
    const int g = threadIdx.x % G;
    const int64_t groups = (int64_t)gridDim.x * (blockDim.x / G);
    for (int64_t e = (int64_t)blockIdx.x * (blockDim.x / G) + threadIdx.x / G; e < count; e += groups) {
        const int64_t i = rows[e], j = cols[e];
        const float* x = X + i * d;
        const float* y = Y + j * d;
        double a = 0.0;
        for (int k = g; k < d; k += 64) a = a + (double)x[k] * (double)y[k];
        a = group_tree_sum<G>(a);
        if (g == 0) out[e] = (p[i] + q[j]) - scale * a;
    }
}

template <int G, int KIND>
__global__ __launch_bounds__(256) void pair_costs_norm_kernel(const float* __restrict__ X, const float* __restrict__ Y,
                                                              const int64_t* __restrict__ rows,
                                                              const int64_t* __restrict__ cols, int64_t count, int d,
                                                              double* __restrict__ out) {
    const int g = threadIdx.x % G;
    const int64_t groups = (int64_t)gridDim.x * (blockDim.x / G);
    for (int64_t e = (int64_t)blockIdx.x * (blockDim.x / G) + threadIdx.x / G; e < count; e += groups) {
        const float* x = X + rows[e] * d;
        const float* y = Y + cols[e] * d;
        double a = 0.0;
        for (int k = g; k < d; k += 64) {
            const double z = (double)x[k] - (double)y[k];
            if (KIND == HM_COST_L1) a = a + fabs(z);
            else if (KIND == HM_COST_LINF) a = fmax(a, fabs(z));
            else a = a + z * z;
        }
        a = (KIND == HM_COST_LINF) ? group_tree_max<G>(a) : group_tree_sum<G>(a);
        if (g == 0) out[e] = (KIND == HM_COST_L2) ? sqrt(a) : a;
    }
}

// fp32 norm costs exactly as the pricing scan forms them: 32-feature chunks accumulated sequentially in fp32,
// chunk results combined in order, l2 = sqrt in fp64 of the fp32 sum, rounded once to fp32.
template <int KIND>
__global__ __launch_bounds__(256) void pair_costs_norm32_kernel(const float* __restrict__ X, const float* __restrict__ Y,
                                                                const int64_t* __restrict__ rows,
                                                                const int64_t* __restrict__ cols, int64_t count, int d,
                                                                double* __restrict__ out) {
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < count; e += (int64_t)gridDim.x * blockDim.x) {
        const float* x = X + rows[e] * d;
        const float* y = Y + cols[e] * d;
        float acc = 0.0f;
        for (int base = 0; base < d; base += 32) {
            float part = 0.0f;
            const int end = base + 32 < d ? base + 32 : d;
            for (int k = base; k < end; ++k) {
                const float z = x[k] - y[k];
                if (KIND == HM_COST_L1) part = part + fabsf(z);
                else if (KIND == HM_COST_LINF) part = fmaxf(part, fabsf(z));
                else part = fmaf(z, z, part);
            }
            acc = (KIND == HM_COST_LINF) ? fmaxf(acc, part) : acc + part;
        }
        out[e] = (KIND == HM_COST_L2) ? (double)(float)sqrt((double)acc) : (double)acc;
    }
}

inline int group_for(int d) { return d <= 8 ? 8 : (d <= 16 ? 16 : (d <= 32 ? 32 : 64)); }

inline unsigned grid_for(int64_t items, int per_block) {
    int64_t b = (items + per_block - 1) / per_block;
    if (b > 65536) b = 65536;
    if (b < 1) b = 1;
    return (unsigned)b;
}

}  // namespace
}  // namespace hm

using namespace hm;

extern "C" int hm_sddmm_l2sq_csr(void* stream, const float* X, const float* Y, const double* p, const double* q,
                                 const int32_t* rowptr, const int32_t* col, int64_t m, int64_t nnz, int32_t d,
                                 double scale, double* out) {
    HM_CHECK_ARG(m >= 0 && nnz >= 0 && d >= 1, "SDDMM requires m >= 0, nnz >= 0, d >= 1");
    HM_CHECK_ARG(scale == 1.0 || scale == 2.0, "dot_scale must be exactly 1 or 2");
    if (m == 0 || nnz == 0) return HM_OK;
    HM_CHECK_ARG(X && Y && p && q && rowptr && col && out, "SDDMM: null pointer argument");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const unsigned grid = grid_for(m, 4);
#define HM_SDDMM(XR) \
    hipLaunchKernelGGL((sddmm_l2sq_csr_kernel<XR>), dim3(grid), dim3(256), 0, st, X, Y, p, q, rowptr, col, m, d, scale, out)
    prof_begin(st, "sddmm_l2sq_csr");
    if (d <= 64) HM_SDDMM(1);
    else if (d <= 128) HM_SDDMM(2);
    else if (d <= 256) HM_SDDMM(4);
    else if (d <= 512) HM_SDDMM(8);
    else HM_SDDMM(0);
    prof_end(st);
#undef HM_SDDMM
    HM_LAUNCH_CHECK("sddmm_l2sq_csr");
    return HM_OK;
}

extern "C" int hm_pair_costs_l2sq(void* stream, const float* X, const float* Y, const double* p, const double* q,
                                  const int64_t* rows, const int64_t* cols, int64_t count, int32_t d, double scale,
                                  double* out) {
    HM_CHECK_ARG(count >= 0 && d >= 1, "pair costs require count >= 0 and d >= 1");
    HM_CHECK_ARG(scale == 1.0 || scale == 2.0, "dot_scale must be exactly 1 or 2");
    if (count == 0) return HM_OK;
    HM_CHECK_ARG(X && Y && p && q && rows && cols && out, "pair costs: null pointer argument");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int G = group_for(d);
#define HM_PAIRS(GG)                                                                                            \
    hipLaunchKernelGGL((pair_costs_l2sq_kernel<GG>), dim3(grid_for(count, 256 / GG)), dim3(256), 0, st, X, Y, p, q, \
                       rows, cols, count, d, scale, out)
    if (G == 8) HM_PAIRS(8);
    else if (G == 16) HM_PAIRS(16);
    else if (G == 32) HM_PAIRS(32);
    else HM_PAIRS(64);
#undef HM_PAIRS
    HM_LAUNCH_CHECK("pair_costs_l2sq");
    return HM_OK;
}

extern "C" int hm_pair_costs_norm(void* stream, const float* X, const float* Y, const int64_t* rows,
                                  const int64_t* cols, int64_t count, int32_t d, int32_t kind, double* out) {
    HM_CHECK_ARG(count >= 0 && d >= 1, "pair costs require count >= 0 and d >= 1");
    HM_CHECK_ARG(kind == HM_COST_L1 || kind == HM_COST_LINF || kind == HM_COST_L2, "unsupported norm cost %d", kind);
    if (count == 0) return HM_OK;
    HM_CHECK_ARG(X && Y && rows && cols && out, "pair costs: null pointer argument");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int G = group_for(d);
#define HM_NORM(GG, KK)                                                                                           \
    hipLaunchKernelGGL((pair_costs_norm_kernel<GG, KK>), dim3(grid_for(count, 256 / GG)), dim3(256), 0, st, X, Y, rows, \
                       cols, count, d, out)
#define HM_NORM_K(GG)                                   \
    do {                                                \
        if (kind == HM_COST_L1) HM_NORM(GG, HM_COST_L1);     \
        else if (kind == HM_COST_LINF) HM_NORM(GG, HM_COST_LINF); \
        else HM_NORM(GG, HM_COST_L2);                        \
    } while (0)
    if (G == 8) HM_NORM_K(8);
    else if (G == 16) HM_NORM_K(16);
    else if (G == 32) HM_NORM_K(32);
    else HM_NORM_K(64);
#undef HM_NORM_K
#undef HM_NORM
    HM_LAUNCH_CHECK("pair_costs_norm");
    return HM_OK;
}

extern "C" int hm_pair_costs_norm_fp32(void* stream, const float* X, const float* Y, const int64_t* rows,
                                       const int64_t* cols, int64_t count, int32_t d, int32_t kind, double* out) {
    HM_CHECK_ARG(count >= 0 && d >= 1, "pair costs require count >= 0 and d >= 1");
    HM_CHECK_ARG(kind == HM_COST_L1 || kind == HM_COST_LINF || kind == HM_COST_L2, "unsupported norm cost %d", kind);
    if (count == 0) return HM_OK;
    HM_CHECK_ARG(X && Y && rows && cols && out, "pair costs: null pointer argument");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const unsigned grid = grid_for(count, 256);
    if (kind == HM_COST_L1)
        hipLaunchKernelGGL((pair_costs_norm32_kernel<HM_COST_L1>), dim3(grid), dim3(256), 0, st, X, Y, rows, cols, count, d,
                           out);
    else if (kind == HM_COST_LINF)
        hipLaunchKernelGGL((pair_costs_norm32_kernel<HM_COST_LINF>), dim3(grid), dim3(256), 0, st, X, Y, rows, cols, count,
                           d, out);
    else
        hipLaunchKernelGGL((pair_costs_norm32_kernel<HM_COST_L2>), dim3(grid), dim3(256), 0, st, X, Y, rows, cols, count, d,
                           out);
    HM_LAUNCH_CHECK("pair_costs_norm_fp32");
    return HM_OK;
}
