// l2^2 ("raw lowrank") pricing scan for gfx950 -- kernels and per-K1 driver (included by pricing_l2sq*.hip): fp32 MFMA sweep + exact fp64 re-check.
//
// Semantics (reference: generic_scan.py:577-597 -> pricing_small.cu:230-304 / pricing.cu:185-229 with
// matrix_selection.cuh:20-74):
//   sigma_ij = (scale*<x_i,y_j> + qb_i) + db_j,   c_ij = (p_i + q_j) - scale*<x_i,y_j>.
// Per X row (and, in a second sweep with the roles swapped, per Y row) the k best sigma with lowest-index
// ties; certificate sums over all pairs.
//
// Pipeline per direction:
//   1. prep:     fp64 row norms ||x_i||, ||y_j||, their maxima, max|bias|; fp32 copies of the biases.
//   2. sweep:    MFMA 32x32x2 fp32 tiles of Y * X^T (a lane owns one X row of a 32-row block and 16 Y
//                columns per 32x32 block). Each lane keeps its best K1 = k + slack values of the fp32
//                score w = scale*dot32 + db32_j (w + qb_i ranks like sigma) in registers; certificate sums
//                are accumulated in fp32 per tile and flushed to fp64.
//   3. finalize: one wave per row merges the lane lists, checks that the K1-th approximate value is below
//                the k-th minus twice the rigorous error bound (otherwise the row is queued for step 4),
//                and re-evaluates the K1 survivors with the fixed-order fp64 dot (dot64) -> exact top-k.
//   4. rescan:   queued rows are scanned exactly (one wave per row, one lane per column).
#pragma once

#include "common.h"

namespace hm {

struct Entry {
    float w;
    int j;
};

struct DirPlan {
    int64_t rows, cols;
    int S;
    int64_t seg_len;
};

namespace {

typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int BX = 128;            // X rows per workgroup (4 waves x 32)
constexpr int NB = 4;              // 32-wide Y blocks per wave
constexpr int BY = 32 * NB;        // Y rows per tile
constexpr int KC = 32;             // features per LDS chunk
constexpr int STR = KC + 4;        // LDS row stride (floats)
constexpr int FLUSH_CHUNKS = 8;    // fp32 block length 256 features before folding into the outer sum


// fp32 unit roundoff doubled (covers truncating accumulation) and the classic gamma_n bound.
inline double gamma_fp32(double n) {
    const double u2 = 2.0 * std::ldexp(1.0, -24);
    return n * u2 / (1.0 - n * u2);
}

// -------------------------------------------------------------------------------------------------
// prep: norms, maxima and fp32 bias copies
// -------------------------------------------------------------------------------------------------
__global__ void l2sq_prep_rows(const float* __restrict__ X, int64_t m, int d, const double* __restrict__ p,
                               const double* __restrict__ qb, const double* __restrict__ db_for_ge,
                               double* __restrict__ norm, float* __restrict__ qb32, float* __restrict__ p32,
                               unsigned long long* __restrict__ maxima /*[norm, |qb|]*/) {
    // one wave per row
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
    if (row >= m) return;
    const float* x = X + row * (int64_t)d;
    double s = 0.0;
    for (int k = lane; k < d; k += 64) s += (double)x[k] * (double)x[k];
    for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
    if (lane == 0) {
        const double nrm = std::sqrt(s) * (1.0 + 1e-12);
        norm[row] = nrm;
        qb32[row] = (float)qb[row];
        // "ge" = q + db for the cost of the certificate, "p" = p for the row side
        p32[row] = db_for_ge ? (float)(p[row] + db_for_ge[row]) : (float)p[row];
        atomicMax(&maxima[0], double_key(nrm));
        atomicMax(&maxima[1], double_key(std::fabs(qb[row])));
    }
}

// -------------------------------------------------------------------------------------------------
// sweep
// -------------------------------------------------------------------------------------------------
template <int K1, bool TWO_LEVEL>
__global__ __launch_bounds__(256) void l2sq_sweep(
    const float* __restrict__ X, const float* __restrict__ Y, int64_t m, int64_t n, int d,
    const float* __restrict__ qb32, const float* __restrict__ db32, const float* __restrict__ p32,
    const float* __restrict__ ge32, float scale, int64_t seg_len, Entry* __restrict__ part,
    double* __restrict__ blockstats, int VEC4, int STATS) {
    __shared__ float sX[BX * STR];
    __shared__ float sY[BY * STR];
    __shared__ float sDB[BY];
    __shared__ float sGE[BY];
    __shared__ double sRed[4][5];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int h = lane >> 5;    // which half of the 2-wide MFMA k slot
    const int r = lane & 31;    // X row within the wave's 32-row block
    const int64_t x0 = (int64_t)blockIdx.x * BX;
    const int64_t seg = blockIdx.y;
    const int64_t y_begin = seg * seg_len;
    const int64_t y_end = (y_begin + seg_len < n) ? (y_begin + seg_len) : n;
    const int64_t my_row = x0 + wave * 32 + r;
    const bool row_ok = my_row < m;

    float lv[K1];
    int li[K1];
#pragma unroll
    for (int s = 0; s < K1; ++s) { lv[s] = -INFINITY; li[s] = -1; }

    const float qbi = row_ok ? qb32[my_row] : 0.0f;
    const float pi = (STATS && row_ok) ? p32[my_row] : 0.0f;
    double num64 = 0.0, den64 = 0.0, cnt64 = 0.0;
    float mx = 0.0f, cmax = 0.0f;

    const int nchunks = (d + KC - 1) / KC;

    // global -> register staging for one chunk: 4 float4 of X and 4 of Y per thread
    float4 gx[4], gy[4];
    auto load_chunk = [&](int c, int64_t ytile) {
        const int k0 = c * KC;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int lin = tid + 256 * i;
            const int row = lin >> 3, c4 = lin & 7;
            const int k = k0 + 4 * c4;
            const int64_t xr = x0 + row, yr = ytile + row;
            if (VEC4) {
                gx[i] = (xr < m && k < d) ? *reinterpret_cast<const float4*>(X + xr * d + k) : make_float4(0, 0, 0, 0);
                gy[i] = (yr < y_end && k < d) ? *reinterpret_cast<const float4*>(Y + yr * d + k) : make_float4(0, 0, 0, 0);
            } else {
                float a[4], b[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    a[e] = (xr < m && k + e < d) ? X[xr * d + k + e] : 0.0f;
                    b[e] = (yr < y_end && k + e < d) ? Y[yr * d + k + e] : 0.0f;
                }
                gx[i] = make_float4(a[0], a[1], a[2], a[3]);
                gy[i] = make_float4(b[0], b[1], b[2], b[3]);
            }
        }
    };
    auto store_chunk = [&]() {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int lin = tid + 256 * i;
            const int row = lin >> 3, c4 = lin & 7;
            *reinterpret_cast<float4*>(&sX[row * STR + 4 * c4]) = gx[i];
            *reinterpret_cast<float4*>(&sY[row * STR + 4 * c4]) = gy[i];
        }
    };

    for (int64_t ytile = y_begin; ytile < y_end; ytile += BY) {
        v16f acc[NB];
        float outer[NB][16];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
#pragma unroll
            for (int q = 0; q < 16; ++q) { acc[b][q] = 0.0f; outer[b][q] = 0.0f; }
        }
        // biases of this tile's Y rows
        if (tid < BY) {
            const int64_t j = ytile + tid;
            sDB[tid] = j < y_end ? db32[j] : 0.0f;
            sGE[tid] = (STATS && j < y_end) ? ge32[j] : 0.0f;
        }
        load_chunk(0, ytile);
        store_chunk();
        __syncthreads();
        for (int c = 0; c < nchunks; ++c) {
            if (c + 1 < nchunks) load_chunk(c + 1, ytile);
            // B operand: this lane's X row, features h*16 .. h*16+15 of the chunk
            const float* bx = &sX[(wave * 32 + r) * STR + h * 16];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float4 bv = *reinterpret_cast<const float4*>(bx + 4 * g);
                float4 av[NB];
#pragma unroll
                for (int b = 0; b < NB; ++b)
                    av[b] = *reinterpret_cast<const float4*>(&sY[(b * 32 + r) * STR + h * 16 + 4 * g]);
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[b].x, bv.x, acc[b], 0, 0, 0);
                    acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[b].y, bv.y, acc[b], 0, 0, 0);
                    acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[b].z, bv.z, acc[b], 0, 0, 0);
                    acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[b].w, bv.w, acc[b], 0, 0, 0);
                }
            }
            if (TWO_LEVEL && ((c + 1) % FLUSH_CHUNKS == 0)) {
#pragma unroll
                for (int b = 0; b < NB; ++b) {
#pragma unroll
                    for (int q = 0; q < 16; ++q) { outer[b][q] += acc[b][q]; acc[b][q] = 0.0f; }
                }
            }
            __syncthreads();
            if (c + 1 < nchunks) {
                store_chunk();
                __syncthreads();
            }
        }
        // epilogue: lane (h, r) holds D[m][n] for n = r (X row) and m = b*32 + 8*(q/4) + 4*h + q%4 (Y row)
        float tnum = 0.0f, tden = 0.0f;
        unsigned int tcnt = 0;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const int jl0 = b * 32 + 8 * a + 4 * h;
                const float4 dbv = *reinterpret_cast<const float4*>(&sDB[jl0]);
                float4 gev = make_float4(0, 0, 0, 0);
                if (STATS) gev = *reinterpret_cast<const float4*>(&sGE[jl0]);
                const float dbs[4] = {dbv.x, dbv.y, dbv.z, dbv.w};
                const float ges[4] = {gev.x, gev.y, gev.z, gev.w};
#pragma unroll
                for (int cc = 0; cc < 4; ++cc) {
                    const int q = 4 * a + cc;
                    const float tot = TWO_LEVEL ? (outer[b][q] + acc[b][q]) : acc[b][q];
                    const float w = fmaf(scale, tot, dbs[cc]);
                    const int64_t j = ytile + jl0 + cc;
                    const bool ok = row_ok && j < y_end;
                    if (ok && w > lv[K1 - 1]) {
                        float cv = w;
                        int ci = (int)j;
#pragma unroll
                        for (int s = 0; s < K1; ++s) {
                            if (cv > lv[s]) {
                                const float tv = lv[s];
                                const int ti = li[s];
                                lv[s] = cv;
                                li[s] = ci;
                                cv = tv;
                                ci = ti;
                            }
                        }
                    }
                    if (STATS && ok) {
                        const float sg = w + qbi;
                        const float cost = (pi + ges[cc]) - w;
                        tden = fmaf(cost, cost, tden);
                        cmax = fmaxf(cmax, fabsf(cost));
                        if (sg > 0.0f) {
                            tnum = fmaf(sg, sg, tnum);
                            mx = fmaxf(mx, sg);
                            ++tcnt;
                        }
                    }
                }
            }
        }
        if (STATS) {
            num64 += (double)tnum;
            den64 += (double)tden;
            cnt64 += (double)tcnt;
        }
        __syncthreads();  // all epilogue reads of sDB/sGE finish before the next tile rewrites them
    }

    // lane lists -> part[(seg*m + row)*2 + h][K1]
    if (row_ok) {
        Entry* out = part + ((seg * m + my_row) * 2 + h) * K1;
#pragma unroll
        for (int s = 0; s < K1; ++s) out[s] = Entry{lv[s], li[s]};
    }
    if (STATS) {
        double v[5] = {num64, den64, cnt64, (double)mx, (double)cmax};
#pragma unroll
        for (int e = 0; e < 5; ++e) {
            for (int o = 32; o >= 1; o >>= 1) {
                const double t = __shfl_xor(v[e], o, 64);
                v[e] = (e >= 3) ? fmax(v[e], t) : v[e] + t;
            }
        }
        if (lane == 0) {
#pragma unroll
            for (int e = 0; e < 5; ++e) sRed[wave][e] = v[e];
        }
        __syncthreads();
        if (tid == 0) {
            double o[5];
            for (int e = 0; e < 5; ++e) {
                o[e] = sRed[0][e];
                for (int w = 1; w < 4; ++w) o[e] = (e >= 3) ? fmax(o[e], sRed[w][e]) : o[e] + sRed[w][e];
            }
            double* dst = blockstats + ((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * 5;
            for (int e = 0; e < 5; ++e) dst[e] = o[e];
        }
    }
}

// deterministic reduction of per-block certificate partials (single block)
__global__ void l2sq_reduce_stats(const double* __restrict__ blockstats, int64_t blocks, double* __restrict__ stats,
                                  int linf) {
    __shared__ double s[256][5];
    const int t = threadIdx.x;
    double v[5] = {0, 0, 0, 0, 0};
    for (int64_t b = t; b < blocks; b += 256) {
        for (int e = 0; e < 5; ++e) v[e] = (e >= 3) ? fmax(v[e], blockstats[b * 5 + e]) : v[e] + blockstats[b * 5 + e];
    }
    for (int e = 0; e < 5; ++e) s[t][e] = v[e];
    __syncthreads();
    for (int w = 128; w >= 1; w >>= 1) {
        if (t < w)
            for (int e = 0; e < 5; ++e) s[t][e] = (e >= 3) ? fmax(s[t][e], s[t + w][e]) : s[t][e] + s[t + w][e];
        __syncthreads();
    }
    if (t == 0) {
        stats[0] = s[0][0];
        stats[1] = s[0][1];
        stats[2] = s[0][2];
        stats[3] = s[0][3];  // replaced by the exact row maximum when rows are computed
        stats[4] = linf ? s[0][4] : 0.0;
    }
}

// -------------------------------------------------------------------------------------------------
// finalize: one wave per row
// -------------------------------------------------------------------------------------------------
struct BoundArgs {
    double acc_rel;   // relative bound on |dot32 - dot| in units of ||x||*||y||, plus fp64 slack
    double db_rel;    // relative bound contribution of fp32 bias rounding, in units of max|db|
    double abs_slack; // absolute slack (flushed denormals)
};

constexpr int FIN_MAX = 512;   // entries one finalize wave can rank (2 * S * K1 <= FIN_MAX)

template <int K1>
__global__ __launch_bounds__(256) void l2sq_finalize(
    const float* __restrict__ X, const float* __restrict__ Y, int64_t m, int d, int S,
    const Entry* __restrict__ part, const double* __restrict__ qb, const double* __restrict__ db,
    const double* __restrict__ xnorm, const unsigned long long* __restrict__ ymaxima, double scale, int k,
    BoundArgs bnd, double* __restrict__ out_val, int* __restrict__ out_idx, int* __restrict__ redo,
    int* __restrict__ redo_count, int TRANSPOSED) {
    __shared__ Entry sE[4][FIN_MAX];
    __shared__ Entry sS[4][64];
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int64_t row = (int64_t)blockIdx.x * 4 + wv;
    const bool valid = row < m;
    const int N = 2 * S * K1;
    // gather this row's lane lists; empty slots become (-inf, -1)
    int nreal = 0;
    for (int e = lane; e < N; e += 64) {
        Entry en{-INFINITY, -1};
        if (valid) {
            const int list = e / K1, slot = e % K1;
            en = part[(((int64_t)(list >> 1) * m + row) * 2 + (list & 1)) * K1 + slot];
            if (en.j < 0) en.w = -INFINITY;
        }
        sE[wv][e] = en;
        nreal += en.j >= 0 ? 1 : 0;
    }
    for (int o = 32; o >= 1; o >>= 1) nreal += __shfl_xor(nreal, o, 64);
    __syncthreads();
    // rank of each real entry by (w desc, j asc); j is unique within a row
    for (int e = lane; e < N; e += 64) {
        const Entry me = sE[wv][e];
        if (me.j < 0) continue;
        int rank = 0;
        for (int f = 0; f < N; ++f) {
            const Entry o = sE[wv][f];
            if (o.j >= 0 && (o.w > me.w || (o.w == me.w && o.j < me.j))) ++rank;
        }
        if (rank < K1) sS[wv][rank] = me;
    }
    __syncthreads();
    if (!valid) return;
    const int kept = nreal < K1 ? nreal : K1;
    const float wk = nreal >= k ? sS[wv][k - 1].w : -INFINITY;
    const float wK1 = nreal >= K1 ? sS[wv][K1 - 1].w : -INFINITY;
    const double ymax = key_double(ymaxima[0]);
    const double dmax = key_double(ymaxima[1]);
    const double nxy = scale * xnorm[row] * ymax;
    const double b = (nxy * bnd.acc_rel + dmax * bnd.db_rel + fabs(qb[row]) * 1e-15 + bnd.abs_slack) * (1.0 + 1e-6);
    // pairs outside the kept list have w <= wK1; they cannot reach the exact top-k when wK1 < wk - 2b
    const bool unsafe = (nreal > K1) && ((double)wK1 >= (double)wk - 2.0 * b);
    if (unsafe) {
        if (lane == 0) {
            const int slot = atomicAdd(redo_count, 1);
            redo[slot] = (int)row;
        }
        return;
    }
    // exact re-evaluation of the kept entries; lane e owns kept entry e
    double sv = -INFINITY;
    int sj = -1;
    const float* xr = X + row * (int64_t)d;
    for (int e = 0; e < kept; ++e) {
        const int jj = sS[wv][e].j;
        const double dot = wave_dot64(xr, Y + (int64_t)jj * d, d, lane);
        const double sdot = scale * dot;
        const double sig = TRANSPOSED ? (sdot + db[jj]) + qb[row] : (sdot + qb[row]) + db[jj];
        if (lane == e) { sv = sig; sj = jj; }
    }
    int er = 0;
    for (int src = 0; src < kept; ++src) {
        const double v2 = __shfl(sv, src, 64);
        const int j2 = __shfl(sj, src, 64);
        if (lane < kept && src != lane && better(v2, j2, sv, sj)) ++er;
    }
    if (lane < kept && er < k) {
        out_val[row * k + er] = sv;
        out_idx[row * k + er] = sj;
    }
    if (lane >= kept && lane < k) {
        out_val[row * k + lane] = -INFINITY;
        out_idx[row * k + lane] = -1;
    }
}

// -------------------------------------------------------------------------------------------------
// exact rescan of queued rows: one wave per row; each lane scores one column per step with the register
// form of dot64, and the wave inserts the few winners into one replicated list (ballot loop)
// -------------------------------------------------------------------------------------------------
template <int K>
__global__ __launch_bounds__(64) void l2sq_rescan(const float* __restrict__ X, const float* __restrict__ Y,
                                                  int64_t n, int d, const double* __restrict__ qb,
                                                  const double* __restrict__ db, double scale, int k,
                                                  const int* __restrict__ redo, const int* __restrict__ redo_count,
                                                  double* __restrict__ out_val, int* __restrict__ out_idx,
                                                  int TRANSPOSED) {
    const int lane = threadIdx.x;
    const int count = *redo_count;
    for (int slot = blockIdx.x; slot < count; slot += gridDim.x) {
        const int64_t row = redo[slot];
        const float* xr = X + row * (int64_t)d;
        double v[K];
        int id[K];
#pragma unroll
        for (int s = 0; s < K; ++s) { v[s] = -INFINITY; id[s] = -1; }
        for (int64_t j0 = 0; j0 < n; j0 += 64) {
            const int64_t j = j0 + lane;
            double sig = -INFINITY;
            if (j < n) {
                const double sdot = scale * lane_dot64(xr, Y + j * d, d);
                sig = TRANSPOSED ? (sdot + db[j]) + qb[row] : (sdot + qb[row]) + db[j];
            }
            const bool cand = j < n && sig == sig && better(sig, (int)j, v[k - 1], id[k - 1]);
            unsigned long long mask = __ballot(cand);
            while (mask) {
                const int src = __ffsll((long long)mask) - 1;
                mask &= mask - 1;
                const double sv = __shfl(sig, src, 64);
                const int sjv = (int)(j0 + src);
                put_sorted<K>(v, id, k, sv, sjv);
            }
        }
        if (lane < k) {
            double ov = -INFINITY;
            int oi = -1;
#pragma unroll
            for (int s = 0; s < K; ++s)
                if (s == lane) { ov = v[s]; oi = id[s]; }
            out_val[row * k + lane] = ov;
            out_idx[row * k + lane] = oi;
        }
    }
}

__global__ void exact_row_max(const double* __restrict__ row_val, int64_t m, int k, double* __restrict__ stats) {
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

__global__ void zero_words(unsigned long long* p, int count) {
    if ((int)threadIdx.x < count) p[threadIdx.x] = 0ull;
}

// -------------------------------------------------------------------------------------------------
// host orchestration
// -------------------------------------------------------------------------------------------------
inline int bucket_k1(int k) { return k <= 2 ? 8 : (k <= 8 ? 16 : 40); }

inline int choose_segments(int64_t m, int64_t n, int k) {
    const int64_t panels = (m + BX - 1) / BX;
    const int64_t tiles = (n + BY - 1) / BY;
    int64_t s = (2048 + panels - 1) / panels;
    const int64_t max_s = tiles / 4 > 0 ? tiles / 4 : 1;
    if (s > max_s) s = max_s;
    const int64_t cap = 256 / bucket_k1(k);  // finalize ranks at most 2 * S * K1 <= 512 entries
    if (s > cap) s = cap;
    if (s < 1) s = 1;
    return (int)s;
}


inline DirPlan plan_dir(int64_t rows, int64_t cols, int k) {
    DirPlan p;
    p.rows = rows;
    p.cols = cols;
    p.S = choose_segments(rows, cols, k);
    const int64_t tiles = (cols + BY - 1) / BY;
    const int64_t tiles_per = (tiles + p.S - 1) / p.S;
    p.seg_len = tiles_per * BY;
    p.S = (int)((cols + p.seg_len - 1) / p.seg_len);
    return p;
}

template <class A>
void layout(A& a, int64_t m, int64_t n, int k, uint32_t flags, DirPlan pr, DirPlan pc, double** xnorm,
            double** ynorm, float** qb32, float** p32, float** db32, float** ge32,
            unsigned long long** maxima, Entry** part, double** blockstats, int** redo, int** redo_count) {
    const int K1 = bucket_k1(k);
    *xnorm = a.template take<double>(m);
    *ynorm = a.template take<double>(n);
    *qb32 = a.template take<float>(m);
    *p32 = a.template take<float>(m);
    *db32 = a.template take<float>(n);
    *ge32 = a.template take<float>(n);
    *maxima = a.template take<unsigned long long>(4);
    size_t part_entries = 0;
    if (flags & (HM_ROWS | HM_STATS)) part_entries = (size_t)pr.S * m * 2 * K1;
    if (flags & HM_COLS) {
        const size_t c = (size_t)pc.S * n * 2 * K1;
        if (c > part_entries) part_entries = c;
    }
    *part = a.template take<Entry>(part_entries > 0 ? part_entries : 1);
    const int64_t blocks_r = (int64_t)((m + BX - 1) / BX) * pr.S;
    const int64_t blocks_c = (int64_t)((n + BX - 1) / BX) * pc.S;
    *blockstats = a.template take<double>((size_t)5 * (blocks_r > blocks_c ? blocks_r : blocks_c));
    *redo = a.template take<int>((size_t)(m > n ? m : n));
    *redo_count = a.template take<int>(2);
}

template <int K1>
int run_direction(hipStream_t st, const float* X, const float* Y, int64_t m, int64_t n, int d, int k,
                  double scale, bool stats, bool transposed, const double* qb, const double* db,
                  const double* xnorm, const unsigned long long* ymaxima, const float* qb32, const float* db32,
                  const float* p32, const float* ge32, DirPlan plan, Entry* part, double* blockstats,
                  int* redo, int* redo_count, double* out_val, int* out_idx, double* stats_out, int linf,
                  bool want_rows) {
    const bool two_level = d > KC * FLUSH_CHUNKS;
    const bool vec4 = (d % 4) == 0;
    dim3 grid((unsigned)((m + BX - 1) / BX), (unsigned)plan.S);
#define HM_SWEEP(TL)                                                                                       \
    hipLaunchKernelGGL((l2sq_sweep<K1, TL>), grid, dim3(256), 0, st, X, Y, m, n, d, qb32, db32, p32, ge32,       \
                       (float)scale, plan.seg_len, part, blockstats, (int)vec4, (int)stats)
    prof_begin(st, "l2sq_sweep");
    if (two_level) HM_SWEEP(true);
    else HM_SWEEP(false);
    prof_end(st);
#undef HM_SWEEP
    HM_LAUNCH_CHECK("l2sq_sweep");
    if (stats) {
        hipLaunchKernelGGL(l2sq_reduce_stats, dim3(1), dim3(256), 0, st, blockstats, (int64_t)grid.x * grid.y,
                           stats_out, linf);
        HM_LAUNCH_CHECK("l2sq_reduce_stats");
    }
    if (!want_rows) return HM_OK;
    // rigorous bound constants
    const double kb = two_level ? (double)(KC * FLUSH_CHUNKS) : (double)d;
    const double nblk = two_level ? std::ceil((double)d / (KC * FLUSH_CHUNKS)) : 1.0;
    const double ea = gamma_fp32(kb) + gamma_fp32(nblk) + gamma_fp32(kb) * gamma_fp32(nblk);
    const double u = std::ldexp(1.0, -24);
    BoundArgs bnd;
    bnd.acc_rel = ea + u * (1.0 + ea) + 4e-15 * (d / 64.0 + 8.0);
    bnd.db_rel = 2.0 * u + 1e-15;
    bnd.abs_slack = 1e-30 * (double)d;
    hipLaunchKernelGGL(zero_words, dim3(1), dim3(64), 0, st, reinterpret_cast<unsigned long long*>(redo_count), 1);
    HM_LAUNCH_CHECK("zero_words");
    const unsigned fin_blocks = (unsigned)((m + 3) / 4);
    prof_begin(st, "l2sq_finalize");
    hipLaunchKernelGGL((l2sq_finalize<K1>), dim3(fin_blocks), dim3(256), 0, st, X, Y, m, d, plan.S, part, qb, db, xnorm,
                       ymaxima, scale, k, bnd, out_val, out_idx, redo, redo_count, (int)transposed);
    prof_end(st);
    HM_LAUNCH_CHECK("l2sq_finalize");
    const unsigned rescan_blocks = (unsigned)(m < 1024 ? m : 1024);
#define HM_RESCAN(KK)                                                                                        \
    hipLaunchKernelGGL((l2sq_rescan<KK>), dim3(rescan_blocks), dim3(64), 0, st, X, Y, n, d, qb, db, scale, k, redo, \
                       redo_count, out_val, out_idx, (int)transposed)
    prof_begin(st, "l2sq_rescan");
    if (k <= 2) HM_RESCAN(2);
    else if (k <= 8) HM_RESCAN(8);
    else HM_RESCAN(32);
    prof_end(st);
#undef HM_RESCAN
    HM_LAUNCH_CHECK("l2sq_rescan");
    return HM_OK;
}

}  // namespace
}  // namespace hm

// driver signature shared by the per-K1 translation units
#define L2SQ_RUN_ARGS                                                                                             \
    hipStream_t st, const float *X, const float *Y, int64_t m, int64_t n, int d, int k, double scale, bool stats,      \
        bool transposed, const double *qb, const double *db, const double *xnorm, const unsigned long long *ymaxima,  \
        const float *qb32, const float *db32, const float *p32, const float *ge32, ::hm::DirPlan plan,             \
        ::hm::Entry *part, double *blockstats, int *redo, int *redo_count, double *out_val, int *out_idx,           \
        double *stats_out, int linf, bool want_rows
#define L2SQ_RUN_PASS                                                                                              \
    st, X, Y, m, n, d, k, scale, stats, transposed, qb, db, xnorm, ymaxima, qb32, db32, p32, ge32, plan, part,         \
        blockstats, redo, redo_count, out_val, out_idx, stats_out, linf, want_rows
