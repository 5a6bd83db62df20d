// l2^2 ("raw lowrank") pricing scan for gfx950 -- kernels and the driver (instantiated by pricing_l2sq_l*_m*.hip):
// one MFMA sweep feeds both the row and the column candidate lists, then an exact fp64 re-check.
//
// Semantics (reference: generic_scan.py:577-597 -> pricing_small.cu:230-304 / pricing.cu:185-229 with
// matrix_selection.cuh:20-74):
//   sigma_ij = (scale*<x_i,y_j> + qb_i) + db_j,   c_ij = (p_i + q_j) - scale*<x_i,y_j>.
// Per X row and per Y row the k best sigma with lowest-index ties; certificate sums over all pairs.
//
// Pipeline, per internal chunk of at most CHUNK_MAX X rows (the column lists of a chunk stay bounded):
//   1. prep (once): fp64 row norms ||x_i||, ||y_j||, their maxima, max|bias|; fp32 copies of the biases; with
//                HM_BF16X3 the split-bf16 copies of X and Y.
//   2. sweep:    MFMA tiles of Y * X^T, fp32 32x32x2 or split-bf16 32x32x16 (a workgroup owns a panel of 128 X
//                rows, 256 in the split sweep for d > 128, and walks one segment of Y in 128-row tiles; lane (h, r)
//                of a wave owns X row r of the wave's 32 and 16 Y rows of each 32-row block). From the same
//                accumulators:
//                  rows:    each lane keeps its best K1 of w = scale*dot32 + db32_j (ranks like sigma in j);
//                  columns: the tile's scores scale*dot32 + qb32_i go through LDS and each Y row keeps its
//                           best K1 over the panel's X rows (one list per X panel);
//                  certificate sums in fp32 per tile, flushed to fp64.
//   3. finalize: one wave per row (or column) merges the partial lists into the best KM, checks that every
//                dropped value is below the k-th minus twice the rigorous error bound (otherwise the row is
//                queued for step 4), and re-evaluates the survivors that can still reach the top k with the
//                fixed-order fp64 dot (dot64).
//   4. rescan:   queued rows / columns are scanned exactly (sliced over waves, then merged).
//   5. columns:  each chunk's exact column lists are merged into the output (tie rule kept).
#pragma once

#include <type_traits>

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
typedef int v16i __attribute__((ext_vector_type(16)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int BX = 128;            // X rows per workgroup of the fp32 and short split sweeps (4 waves x 32)
constexpr int NB = 4;              // 32-wide Y blocks per wave
constexpr int BY = 32 * NB;        // Y rows per tile
constexpr int KC = 32;             // features per LDS chunk
constexpr int STR = KC + 4;        // LDS row stride (floats)
constexpr int STAGE = (BX + BY) * STR;  // floats per LDS stage of the sweep (X tile, then Y tile)
constexpr int CST = BX + 1;        // LDS row stride of the column-score tile (floats)
constexpr int QN = 12;             // queued row candidates per lane and tile (128-row sweeps; one spare slot more)
constexpr int FLUSH_CHUNKS = 8;    // fp32 block length 256 features before folding into the outer sum
constexpr int FLUSH_SPLIT = 4;     // split-bf16 block length 128 features (3 product terms per feature)
constexpr int64_t CHUNK_MAX = 65536;          // X rows per internal chunk
// Y rows per chunk of the role-swapped pass against a resident Y side (whose sweep copy is whole, so a chunk costs
// only its partial lists): fewer, longer launches with one finalize each
constexpr int64_t CHUNK_MAX_RESIDENT = 4 * CHUNK_MAX;
constexpr int FUSE_MIN_D = 256;               // columns ride on the row sweep from this d on (below it the
                                              // per-tile column epilogue outweighs the MFMA work: two sweeps)
constexpr int64_t SWEEP_WGS = 1024;           // target workgroups per sweep launch (sets the Y segments)
constexpr int64_t SWEEP_CUS = 256;            // CUs of an MI355X: one sweep workgroup each at a time
constexpr int64_t RESCAN_SLICE = 512;         // candidates per exact-rescan item (one wave)
constexpr int64_t RESCAN_ITEMS = 65536;       // (row, slice) items whose partial lists fit the rescan scratch
constexpr size_t COLPART_CAP = size_t(12) << 30;  // bytes of per-chunk column partial lists
constexpr int64_t WIDE_BUF = int64_t(1) << 22;  // candidate ids per wide-pass batch (rows x capacity)
constexpr int WIDE_ROWS = 8192;               // queued rows per batch of the first wide round (capacity 512)
constexpr int WIDE_CAP1 = 512;                // candidates a row may collect in the first wide round
constexpr int WIDE_CAP2 = 16384;              // ... in the second round (rows that overflowed the first)
constexpr int WIDE_SLICE = 128;               // collected candidates per exact-evaluation item (one wave)

// fp32 unit roundoff doubled (covers truncating accumulation) and the classic gamma_n bound.
inline double gamma_fp32(double n) {
    const double u2 = 2.0 * std::ldexp(1.0, -24);
    return n * u2 / (1.0 - n * u2);
}

// better() on fp32 list entries (lowest index wins ties; missing entries lose)
__device__ inline bool better_e(float av, int ai, float bv, int bi) {
    return av > bv || (av == bv && ai >= 0 && (bi < 0 || ai < bi));
}

template <int K>
__device__ inline void insert_e(float (&w)[K], int (&id)[K], float v, int i) {
    float cv = v;
    int ci = i;
#pragma unroll
    for (int s = 0; s < K; ++s) {
        if (better_e(cv, ci, w[s], id[s])) {
            const float tv = w[s];
            const int ti = id[s];
            w[s] = cv;
            id[s] = ci;
            cv = tv;
            ci = ti;
        }
    }
}

// Certificate inputs of a sweep: the fp64 biases (staged in LDS per panel and per tile) and the device maxima of
// the swept-against side (ymax[1] = max|db|), so that pairs near zero get their score in fp64.
struct CertArgs {
    const double* qb;
    const double* db;
    const unsigned long long* ymax;  // [max ||y||, max |db|] of the swept-against side
    const double* xnorm;             // ||x_i|| of the swept rows (global row index)
};

// 2.5 fp32 units: the slack below bounds four fp32 roundings (db_j and qb_i to fp32, the fma giving w, the add
// giving sg) with room for the rounding of the slack itself
constexpr float CERT_REL = 1.4901161e-07f;
// LDS entries of a certificate bias array (the wide pass, which has no certificate, compiles them to one entry)
#define STATS_LDS(n) (APPEND ? 1 : (n))

// Certificate terms of one pair from its fp32 dot t and fp32 score w = fl(scale*t + db32_j). The fp64 score
// sigma' = (scale*t + qb_i) + db_j (the reference's arithmetic: fp32 dot, fp64 epilogue) differs from the fp32 score
// sg = fl(w + qb32_i) by at most CERT_REL * (|w| + |qb32_i| + max|db|), and |w| <= scale ||x_i|| max||y|| (1 + 1e-2)
// + max|db| bounds every |w| of row i, so the row's slack (row_cert_slack) covers all its pairs. Pairs beyond the
// slack are decided in fp32 (a positive one adds sg^2 to the tile's fp32 sum); pairs within it get sigma' in fp64,
// which decides the count and adds sigma'^2 to the lane's fp64 sum.
//
// cert_fast is the per-pair part, without branches: the cost terms, the fp32 decision, and `near` set for a pair
// within the slack. A tile with a near pair on some lane runs cert_near over its pairs afterwards (rare: the slack is
// a few fp32 units of the row's largest score).
__device__ __forceinline__ void cert_fast(bool ok, float w, float ge, float pi, float qbi, float slack, float& tden,
                                          float& cmax, float& tnum, unsigned int& tcnt, bool& near) {
    const float cost = (pi + ge) - w;
    const float cm = ok ? cost : 0.0f;
    tden = fmaf(cm, cm, tden);
    cmax = fmaxf(cmax, fabsf(cm));
    const float sg = w + qbi;
    const bool pos = ok && sg > slack;
    const float sp = pos ? sg : 0.0f;
    tnum = fmaf(sp, sp, tnum);
    tcnt += pos ? 1u : 0u;
    near = near || (ok && fabsf(sg) <= slack);
}

__device__ __forceinline__ void cert_near(bool ok, float t, float w, float qbi, float slack, float scale, double qb64,
                                          double db64, unsigned int& tcnt, double& num64) {
    const float sg = w + qbi;
    if (ok && fabsf(sg) <= slack) {
        const double sig = ((double)scale * (double)t + qb64) + db64;
        if (sig > 0.0) {
            num64 = fma(sig, sig, num64);
            ++tcnt;
        }
    }
}

// slack of row `row` (0 without a certificate or past the chunk)
__device__ __forceinline__ float row_cert_slack(int STATS, const CertArgs& c, int64_t row, bool ok, float scale) {
    if (!STATS || !ok) return 0.0f;
    const double ymax = key_double(c.ymax[0]), dmax = key_double(c.ymax[1]);
    const double wmax = 1.01 * (double)scale * c.xnorm[row] * ymax + dmax;
    return (float)(CERT_REL * (wmax + fabs(c.qb[row]) + dmax) * (1.0 + 1e-3));
}

// int8 split (HM_INT8X3): the rows of a block of 32 are quantized to v_k = rint(x_k / s) with one scale
// s = max |x_k| / I8_Q over the block, so |v_k| <= I8_Q, and v = 256 h + l splits into int8 limbs
// h = (v + 128) >> 8 in [-127, 127] and l in [-128, 127]. A scale per block keeps the scales of a sweep tile's Y
// blocks uniform over the wave.
constexpr int I8_Q = 32639;  // 256 * 127 + 127
// the scale of a block with largest magnitude amax; 1 for a zero block or one so small that 1 / s would overflow
// (all its v are then 0, and the quantization error |x_k| < s / 2 still holds)
__device__ __forceinline__ float i8_scale(float amax) {
    const float s = amax / (float)I8_Q;
    return (s >= 1e-37f && s < INFINITY) ? s : 1.0f;
}

// -------------------------------------------------------------------------------------------------
// prep: norms, maxima and fp32 bias copies
// -------------------------------------------------------------------------------------------------
// one wave per row (grid-stride); the maxima are reduced per workgroup before one atomic each
__global__ __launch_bounds__(256) void l2sq_prep_rows(const float* __restrict__ X, int64_t m, int d,
                                                      const double* __restrict__ p, const double* __restrict__ qb,
                                                      const double* __restrict__ db_for_ge, double* __restrict__ norm,
                                                      float* __restrict__ qb32, float* __restrict__ p32,
                                                      unsigned long long* __restrict__ maxima /*[norm, |qb|]*/,
                                                      float* __restrict__ qscale = nullptr,
                                                      double* __restrict__ l1 = nullptr) {
    __shared__ double sM[4][2];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    double mx_norm = 0.0, mx_bias = 0.0;
    for (int64_t row = (int64_t)blockIdx.x * 4 + wave; row < m; row += (int64_t)gridDim.x * 4) {
        const float* x = X + row * (int64_t)d;
        // the norms only bound errors (they are inflated by 1e-12 below), so any summation order will do: float4
        // loads and four independent sums when rows are whole float4s
        double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0, a1 = 0.0;
        float amax = 0.0f;
        int k0 = 0;
        if ((d & 3) == 0) {
            const float4* x4 = reinterpret_cast<const float4*>(x);
            for (int k = lane; k < d / 4; k += 64) {
                const float4 v = x4[k];
                s0 += (double)v.x * (double)v.x;
                s1 += (double)v.y * (double)v.y;
                s2 += (double)v.z * (double)v.z;
                s3 += (double)v.w * (double)v.w;
                a1 += ((double)fabsf(v.x) + (double)fabsf(v.y)) + ((double)fabsf(v.z) + (double)fabsf(v.w));
                amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
            }
            k0 = d;
        }
        for (int k = k0 + lane; k < d; k += 64) {
            s0 += (double)x[k] * (double)x[k];
            a1 += (double)fabsf(x[k]);
            amax = fmaxf(amax, fabsf(x[k]));
        }
        double s = (s0 + s1) + (s2 + s3);
        for (int o = 32; o >= 1; o >>= 1) {
            s += __shfl_xor(s, o, 64);
            a1 += __shfl_xor(a1, o, 64);
            amax = fmaxf(amax, __shfl_xor(amax, o, 64));
        }
        const double nrm = std::sqrt(s) * (1.0 + 1e-12);
        mx_norm = fmax(mx_norm, nrm);
        if (qb) mx_bias = fmax(mx_bias, std::fabs(qb[row]));
        if (lane == 0) {
            norm[row] = nrm;
            if (qb) {  // (a resident side's preparation has no biases)
                qb32[row] = (float)qb[row];
                // "ge" = q + db for the cost of the certificate, "p" = p for the row side
                p32[row] = db_for_ge ? (float)(p[row] + db_for_ge[row]) : (float)p[row];
            }
            if (qscale) {
                qscale[row] = amax;  // the int8 copy turns it into its block's scale
                l1[row] = a1 * (1.0 + 1e-12);
            }
        }
    }
    if (lane == 0) {
        sM[wave][0] = mx_norm;
        sM[wave][1] = mx_bias;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; ++w) {
            mx_norm = fmax(mx_norm, sM[w][0]);
            mx_bias = fmax(mx_bias, sM[w][1]);
        }
        atomicMax(&maxima[0], double_key(mx_norm));
        atomicMax(&maxima[1], double_key(mx_bias));
    }
}

// The Y side's biases for a call against a resident side (whose norms were computed once): db32, ge32 = q + db,
// and the maxima max ||y|| (copied from the resident side) and max |db|.
__global__ __launch_bounds__(256) void l2sq_prep_bias(int64_t n, const double* __restrict__ q,
                                                      const double* __restrict__ db,
                                                      const unsigned long long* __restrict__ ynorm_max,
                                                      float* __restrict__ db32, float* __restrict__ ge32,
                                                      unsigned long long* __restrict__ maxima /*[norm, |db|]*/) {
    __shared__ double sM[4];
    double mx = 0.0;
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < n; j += (int64_t)gridDim.x * blockDim.x) {
        db32[j] = (float)db[j];
        ge32[j] = (float)(q[j] + db[j]);
        mx = fmax(mx, std::fabs(db[j]));
    }
    for (int o = 32; o >= 1; o >>= 1) mx = fmax(mx, __shfl_xor(mx, o, 64));
    if ((threadIdx.x & 63) == 0) sM[threadIdx.x >> 6] = mx;
    __syncthreads();
    if (threadIdx.x == 0) {
        mx = fmax(fmax(sM[0], sM[1]), fmax(sM[2], sM[3]));
        atomicMax(&maxima[1], double_key(mx));
        if (blockIdx.x == 0) atomicMax(&maxima[0], *ynorm_max);
    }
}

inline unsigned prep_grid(int64_t rows) {
    const int64_t b = (rows + 3) / 4;
    return (unsigned)(b < 2048 ? b : 2048);
}

// -------------------------------------------------------------------------------------------------
// split-bf16 copy: x = hi + lo + e with hi = bf16(x), lo = bf16(x - hi) (round to nearest even), |e| <= 2^-16|x|.
// The copy is stored in the operand order of v_mfma_f32_32x32x16_bf16. Rows form blocks of 32 (block stride
// 32 * ld words, ld = split_ld). A block is a run of 4 KiB chunks of 32 features. A chunk holds four 1 KiB operand
// tiles: K-step s (16 features) and part p (hi / lo) at (2s + p) KiB. Within a tile, the 16 bytes at lane
// 32h + r are features 8h .. 8h+7 of the K-step for row r, as 8 bf16. Padding features (to split_features) and
// padding rows (to a whole 128-row panel) are zero.
//
// With this layout a lane's operand of one K-step is one coalesced 16-byte load. A Y tile's chunk is four
// contiguous 4 KiB runs that go to LDS unchanged: conflict-free reads, no padding.
// -------------------------------------------------------------------------------------------------
__device__ inline unsigned short bf16_rne(float x) {
    const unsigned int u = __float_as_uint(x);
    return (unsigned short)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// 16-byte unit (hi part) of row `row`, chunk c, group g4 = 2s + h of a split copy with ld words per row; the lo
// part follows 64 units later
__host__ __device__ inline int64_t split_unit(int64_t row, int c, int g4, int ld) {
    return ((row >> 5) * 32 * (int64_t)ld + (int64_t)c * 1024) / 4 + (g4 >> 1) * 128 + (g4 & 1) * 32 + (row & 31);
}

// Item (32-row block, pair of chunks): the workgroup reads the block's 64 features per row into LDS (consecutive
// threads on consecutive features of a row), then writes the 512 operand-order units of the two chunks
// (consecutive threads on consecutive rows of a unit group): reads and writes both coalesced.
__global__ __launch_bounds__(256) void l2sq_split_bf16(const float* __restrict__ X, int64_t rows, int64_t padded_rows,
                                                       int d, int sd, int ld, unsigned short* __restrict__ out) {
    __shared__ float tile[32][65];  // 32 rows x 64 features (one pad column: conflict-free row-wise reads)
    const int nch = sd / KC;
    const int npair = (nch + 1) / 2;
    const int64_t items = (padded_rows >> 5) * npair;
    uint4* out4 = reinterpret_cast<uint4*>(out);
    const int t = threadIdx.x;
    for (int64_t it = blockIdx.x; it < items; it += gridDim.x) {
        const int64_t blk = it / npair;
        const int c0 = (int)(it % npair) * 2;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int e = t + 256 * i;
            const int rr = e >> 6, f = e & 63;
            const int64_t row = blk * 32 + rr;
            const int k = c0 * KC + f;
            tile[rr][f] = (row < rows && k < d) ? X[row * d + k] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int u = t + 256 * i;  // (part, chunk of the pair, group g4, row r), r fastest
            const int r = u & 31, g4 = (u >> 5) & 3, cc = (u >> 7) & 1, part = u >> 8;
            if (c0 + cc < nch) {
                const float* src = &tile[r][cc * KC + g4 * 8];
                unsigned short v[8];
#pragma unroll
                for (int e2 = 0; e2 < 8; ++e2) {
                    const float x = src[e2];
                    const unsigned short hi = bf16_rne(x);
                    v[e2] = part ? bf16_rne(x - __uint_as_float((unsigned int)hi << 16)) : hi;
                }
                uint4 w;
                w.x = v[0] | ((unsigned int)v[1] << 16);
                w.y = v[2] | ((unsigned int)v[3] << 16);
                w.z = v[4] | ((unsigned int)v[5] << 16);
                w.w = v[6] | ((unsigned int)v[7] << 16);
                out4[split_unit(blk * 32 + r, c0 + cc, g4, ld) + (part ? 64 : 0)] = w;
            }
        }
        __syncthreads();  // the tile is rewritten by the next item
    }
}

// -------------------------------------------------------------------------------------------------
// int8 split copy (HM_INT8X3) in the operand order of v_mfma_i32_32x32x32_i8, with the split-bf16 copy's geometry
// counted in 4-byte words: a block of 32 rows is a run of 4 KiB chunks, here of 64 features (two bytes per feature,
// ld = i8_ld(d) words per row); a chunk holds four 1 KiB tiles, K-step s (32 features) and limb p (h, then l) at
// (2s + p) KiB; within a tile the 16 bytes at lane 32h + r are features 16h .. 16h+15 of the K-step for row r.
// Padding features and rows are zero. The sweeps' unit arithmetic (split_unit, the LDS ring) is unchanged.
//
// Error terms of a pair (x, y), in dot units. With xq = s v and e = x - xq, |e_k| <= 0.51 s (v is rint of the fp32
// product x * fl(1/s), within 0.504 of x / s):
//   |x.y - xq.yq| <= sum |e_x||y| + sum |xq||e_y| <= alpha_x beta_y + alpha_y beta_x,
//       alpha = 0.51 s,  beta = ||x||_1 + 0.51 s d (at least ||x||_1 and ||xq||_1);
//   the sweep drops the limb product: s_x s_y |sum l_x l_y| <= gamma_x gamma_y,  gamma = s ||l||_2;
//   the fp32 conversion of the two int32 sums (four roundings of values at most sum (|v_x| + 256)(|v_y| + 256) s_x s_y
//       in magnitude) <= 5 u rho_x rho_y,  rho = ||x||_2 + 257 s sqrt(d).
// Terms per row (alpha, beta, gamma, rho) go to qterm; their maxima over the side to qmax (ordered keys).
// -------------------------------------------------------------------------------------------------
inline int i8_features(int d) { return (d + 255) / 256 * 256; }  // whole groups of 4 chunks (the sweep's unroll)
inline int i8_words(int d) { return i8_features(d) / 2; }
inline int i8_ld(int d) { return i8_words(d) + (i8_words(d) % 512 == 0 ? KC : 0); }

// One workgroup per 32-row block (grid-stride): the block's scale from its rows' maxima (which `qscale` holds on
// entry and receives the block scale in their place), then per chunk the block's 32 x 64 features pass through LDS
// (coalesced reads) and thread t quantizes and writes unit t of the chunk (coalesced writes); ||l||_2^2 is summed
// exactly.
__global__ __launch_bounds__(256) void l2sq_split_i8(const float* __restrict__ X, int64_t rows, int64_t padded_rows,
                                                     int d, int sd, int ld, float* __restrict__ qscale,
                                                     const double* __restrict__ l1, const double* __restrict__ norm,
                                                     unsigned int* __restrict__ out, double* __restrict__ qterm,
                                                     unsigned long long* __restrict__ qmax) {
    __shared__ float tile[32][65];
    __shared__ unsigned int sl[4][32];
    __shared__ float sScale;
    const int nch = sd / KC;  // 64-feature chunks
    const int t = threadIdx.x;
    const int s = t >> 7, p = (t >> 6) & 1, h = (t >> 5) & 1, r = t & 31;  // unit t: tile 2s + p, lane 32h + r
    const int64_t blocks = padded_rows >> 5;
    double mq[4] = {0.0, 0.0, 0.0, 0.0};
    uint4* out4 = reinterpret_cast<uint4*>(out);
    for (int64_t blk = blockIdx.x; blk < blocks; blk += gridDim.x) {
        const int64_t row = blk * 32 + r;
        if (t < 64) {
            float a = (t < 32 && row < rows) ? qscale[row] : 0.0f;
            for (int o = 16; o >= 1; o >>= 1) a = fmaxf(a, __shfl_xor(a, o, 64));
            if (t == 0) sScale = i8_scale(a);
        }
        __syncthreads();
        const float sb = sScale;
        if (t < 32 && row < rows) qscale[row] = sb;
        const float inv = 1.0f / sb;
        unsigned int lsq = 0u;
        for (int c = 0; c < nch; ++c) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int e = t + 256 * i;
                const int rr = e >> 6, f = e & 63;
                const int64_t xr = blk * 32 + rr;
                const int k = c * 64 + f;
                tile[rr][f] = (xr < rows && k < d) ? X[xr * d + k] : 0.0f;
            }
            __syncthreads();
            const float* src = &tile[r][s * 32 + h * 16];
            unsigned int wv[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                unsigned int word = 0u;
#pragma unroll
                for (int e2 = 0; e2 < 4; ++e2) {
                    const int v = (int)rintf(src[4 * g + e2] * inv);
                    const int hi = (v + 128) >> 8;
                    const int lo = v - hi * 256;
                    lsq += (unsigned int)(lo * lo);
                    word |= (unsigned int)((p ? lo : hi) & 0xff) << (8 * e2);
                }
                wv[g] = word;
            }
            out4[(blk * 32 * (int64_t)ld + (int64_t)c * 1024) / 4 + t] = make_uint4(wv[0], wv[1], wv[2], wv[3]);
            __syncthreads();  // the tile is rewritten by the next chunk
        }
        if (p == 0) sl[2 * s + h][r] = lsq;  // the p = 1 threads summed the same values
        __syncthreads();
        if (t < 32 && row < rows) {
            const unsigned long long l2 = (unsigned long long)sl[0][t] + sl[1][t] + sl[2][t] + sl[3][t];
            const double sc = (double)sb;
            const double q[4] = {0.51 * sc, l1[row] + 0.51 * sc * d, sc * std::sqrt((double)l2) * (1.0 + 1e-12),
                                 norm[row] + 257.0 * sc * std::sqrt((double)d) * (1.0 + 1e-12)};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                qterm[row * 4 + e] = q[e];
                mq[e] = fmax(mq[e], q[e]);
            }
        }
        __syncthreads();  // sl and sScale are rewritten by the next block
    }
    if (t < 64) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            for (int o = 32; o >= 1; o >>= 1) mq[e] = fmax(mq[e], __shfl_xor(mq[e], o, 64));
        }
        if (t == 0) {
#pragma unroll
            for (int e = 0; e < 4; ++e) atomicMax(&qmax[e], double_key(mq[e]));
        }
    }
}

// -------------------------------------------------------------------------------------------------
// sweep over X rows [xb, xe) of one chunk
// -------------------------------------------------------------------------------------------------
// Workgroup -> (X panel, Y segment). Workgroups reach the 8 XCDs round-robin in launch order, so XCD x runs
// workgroups x, x + 8, x + 16, .... Up to 64 panels the order is panel-major (workgroup L = panel + P * seg): with
// all panels in flight each panel stays on one XCD and the segments in flight are few. With more panels, the 32
// workgroups an XCD runs at a time (one per CU) form a block of 8 panels x 4 segments and the 8 XCDs' blocks
// step through the segment groups of the same panel groups, so the panels in flight stay few and their features
// stay in the last-level cache across Y tiles (measured at d = 8192: 15% faster for 500 panels, 8% slower for
// 64). Grid: sweep_grid(P, S) workgroups; the padding ones exit at once.
constexpr int MAP_PANELS = 64;  // panel-major order up to this many panels
constexpr int MAP_BP = 8, MAP_BS = 4;  // block of one XCD's 32 concurrent workgroups
__host__ __device__ inline void sweep_block(int64_t L, int P, int S, int64_t& panel, int64_t& seg) {
    if (P <= MAP_PANELS) {
        panel = L % P;
        seg = L / P;
        return;
    }
    const int64_t x = L & 7, t = L >> 3;
    const int64_t B = (t >> 5) * 8 + x, i = t & 31;
    const int64_t SG = (S + MAP_BS - 1) / MAP_BS;
    panel = (B / SG) * MAP_BP + (i % MAP_BP);
    seg = (B % SG) * MAP_BS + (i / MAP_BP);
}

inline unsigned sweep_grid(int64_t P, int64_t S) {
    if (P <= MAP_PANELS) return (unsigned)(P * S);
    const int64_t blocks = ((P + MAP_BP - 1) / MAP_BP) * ((S + MAP_BS - 1) / MAP_BS);
    return (unsigned)((blocks + 7) / 8 * 8 * 32);
}

// Shared row thresholds (per local row of a sweep launch; all keys start at float_key(-inf)): a lane whose partial
// list of a row is full publishes its last entry, so the key is the K1-th value of some full list of that row.
// Scores at or below it are not inserted into any of the row's lists: they are at most the largest last entry of
// the row's full lists, which the finalize already takes as the bound of what the lists dropped. With no buffer
// (nullptr) nothing is filtered.
__device__ __forceinline__ float row_threshold_get(const unsigned int* rowthr, int64_t local) {
    return rowthr ? key_float(rowthr[local]) : -INFINITY;
}
__device__ __forceinline__ void row_threshold_raise(unsigned int* rowthr, int64_t local, float last) {
    if (rowthr) atomicMax(&rowthr[local], float_key(last));
}

// Lane state of a sweep: the row's partial top-K1 list, its per-row constants and certificate partial sums.
template <int K1>
struct SweepRow {
    float lv[K1];
    int li[K1];
    int64_t row;   // global X row of this lane
    bool ok;       // row < xe
    float qbi;     // row bias (scores of the column lists)
    float wt;      // wide-pass threshold
    float pi;      // certificate row term
    double num64, den64;
    unsigned int cnt;  // violated pairs of this lane (at most its share of one segment: fits 32 bits)
    float cmax;
};

template <int K1, bool APPEND>
__device__ __forceinline__ void sweep_row_init(SweepRow<K1>& s, int64_t row, int64_t xe, int STATS,
                                               const float* __restrict__ qb32, const float* __restrict__ p32,
                                               const float* __restrict__ wthr) {
#pragma unroll
    for (int i = 0; i < K1; ++i) { s.lv[i] = -INFINITY; s.li[i] = -1; }
    s.row = row;
    s.ok = row < xe;
    s.qbi = (s.ok && !APPEND) ? qb32[row] : 0.0f;
    s.wt = (APPEND && s.ok) ? wthr[row] : INFINITY;
    s.pi = (STATS && s.ok) ? p32[row] : 0.0f;
    s.num64 = s.den64 = 0.0;
    s.cnt = 0u;
    s.cmax = 0.0f;
}

// Per-tile epilogue of both sweeps. tot[b][q] is the fp32 dot of this lane's X row with Y row
// ytile + b*32 + 8*(q/4) + 4*h + q%4 (the lane (h, r) layout of the 32x32 MFMA accumulators). It ranks
// w = scale*dot + db into the row list (or appends for the wide pass), adds the certificate terms and, with COLS,
// passes the tile's scores scale*dot + qb through LDS so that each Y row keeps its best K1 over the workgroup's
// 128 X rows, CPASS Y rows at a time (sC holds CPASS * CST floats; 256 / CPASS threads scan each row and merge
// their lists). Ends with a barrier: the next tile may rewrite sDB / sGE / sC.
template <int K1, bool COLS, bool APPEND, int CPASS, bool FULL, bool ST, bool SRT = false>
__device__ __forceinline__ void sweep_epilogue(const v16f (&tot)[NB], SweepRow<K1>& s, int tid, int wave, int h,
                                               int r, int64_t ytile, int64_t y_end, int64_t x0, int64_t panel,
                                               int64_t n, float scale, int STATS_, float slack, const double* sQB64,
                                               const double* sDB64, const float* sDB, const float* sGE,
                                               float* sC, Entry* __restrict__ colpart,
                                               unsigned int* __restrict__ colthr, int* __restrict__ wcnt,
                                               int* __restrict__ wbuf, int wcap, unsigned int* __restrict__ rowthr,
                                               int64_t xb, Entry* sQ, const unsigned int* sRT = nullptr) {
    // ST = false (sweeps without the certificate) drops the certificate code, and with it a per-score test of the
    // runtime flag (a scalar branch per score). With ST = true the flag stays a runtime test: as a compile-time
    // constant the certificate terms get scheduled across scores and the sweeps spill.
    const int STATS = ST ? STATS_ : 0;
    float tnum = 0.0f, tden = 0.0f;
    unsigned int tcnt = 0;
    bool near = false;  // a pair of this tile within the certificate slack (cert_fast)
    // Y rows of the tile inside the segment; pair (lane half h, offset c) is inside when 4h < ylim - c, a compare
    // against a wave-uniform bound
    // (FULL: the whole tile lies inside the segment and the whole panel inside the chunk, so every pair is inside)
    const int ylim = FULL ? NB * 32 : (int)(y_end - ytile < (int64_t)(NB * 32) ? y_end - ytile : (int64_t)(NB * 32));
    const bool rok = FULL || s.ok;
    // the row's shared threshold: scores at or below it cannot enter the row's merged lists (row_threshold_*);
    // with SRT, sRT holds the panel's thresholds as read at the start of the tile
    float rthr = -INFINITY;
    if (!APPEND && rok && rowthr) {
        if constexpr (SRT) rthr = key_float(sRT[wave * 32 + r]);
        else rthr = row_threshold_get(rowthr, s.row - xb);
    }
    const float last0 = APPEND ? 0.0f : s.lv[K1 - 1];
    // Row candidates of the tile: every score above the lane's threshold at the start of the tile is queued in the
    // lane's LDS slots, without branches (a full queue writes its spare slot), and inserted after the tile in pair
    // order. A lane with more than QN candidates (a segment's first tiles) inserts the tile directly instead.
    const float qthr = fmaxf(s.lv[K1 - 1], rthr);
    Entry* myq = sQ + tid * (QN + 1);
    int qn = 0;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
        for (int a = 0; a < 4; ++a) {
            // the lane's largest score among its 4 pairs of the group (pairs outside the tile excluded): the group's
            // scores are queued only when some lane of the wave has one above its threshold
            float amax = -INFINITY;
            const int jl0 = b * 32 + 8 * a + 4 * h;
            const float4 dbv = *reinterpret_cast<const float4*>(&sDB[jl0]);
            float4 gev = make_float4(0, 0, 0, 0);
            if (STATS) gev = *reinterpret_cast<const float4*>(&sGE[jl0]);
            const float dbs[4] = {dbv.x, dbv.y, dbv.z, dbv.w};
            const float ges[4] = {gev.x, gev.y, gev.z, gev.w};
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
                const int q = 4 * a + cc;
                const float t = tot[b][q];
                const float w = fmaf(scale, t, dbs[cc]);
                const int64_t j = ytile + jl0 + cc;
                const bool ok = rok && (FULL || 4 * h < ylim - (b * 32 + 8 * a + cc));
                if (APPEND) {
                    if (ok && w >= s.wt) {
                        const int pos = atomicAdd(&wcnt[s.row], 1);
                        if (pos < wcap) wbuf[s.row * (int64_t)wcap + pos] = (int)j;
                    }
                } else {
                    amax = fmaxf(amax, ok ? w : -INFINITY);
                }
                if (STATS) cert_fast(ok, w, ges[cc], s.pi, s.qbi, slack, tden, s.cmax, tnum, tcnt, near);
            }
            if (!APPEND && __any(amax > qthr)) {
                // every score above the threshold, in pair order, as if each had been tested
#pragma unroll
                for (int cc = 0; cc < 4; ++cc) {
                    const float w = fmaf(scale, tot[b][4 * a + cc], dbs[cc]);
                    const bool ok = rok && (FULL || 4 * h < ylim - (b * 32 + 8 * a + cc));
                    const bool cand = ok && w > qthr;
                    myq[qn < QN ? qn : QN] = Entry{w, (int)(ytile + jl0 + cc)};
                    qn += cand ? 1 : 0;
                }
            }
        }
    }
    if (!APPEND) {
        if (qn > QN) {
            // direct insertion of the whole tile (the queue overflowed)
            asm volatile("" ::: "memory");
#pragma unroll
            for (int b = 0; b < NB; ++b) {
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    const int jl = b * 32 + 8 * (q / 4) + 4 * h + (q % 4);
                    const float w = fmaf(scale, tot[b][q], sDB[jl]);
                    const bool ok = rok && (FULL || 4 * h < ylim - (jl - 4 * h));
                    if (ok && w > s.lv[K1 - 1] && w > rthr) insert_e<K1>(s.lv, s.li, w, (int)(ytile + jl));
                }
            }
        } else {
            // the queue, in pair order; the loop runs as often as the wave's longest queue
            for (int e = 0; e < QN; ++e) {
                if (!__any(e < qn)) break;
                if (e < qn) {
                    const Entry c = myq[e];
                    if (c.w > s.lv[K1 - 1]) insert_e<K1>(s.lv, s.li, c.w, c.j);
                }
            }
        }
    }
    if (STATS && near) {
        // reload the biases rather than keep the fast path's values alive in registers through the tile
        asm volatile("" ::: "memory");
        const double qb64 = sQB64[wave * 32 + r];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int jl = b * 32 + 8 * (q / 4) + 4 * h + (q % 4);
                const float t = tot[b][q];
                cert_near(rok && (FULL || 4 * h < ylim - (jl - 4 * h)), t, fmaf(scale, t, sDB[jl]), s.qbi, slack, scale, qb64,
                          sDB64[jl], tcnt, s.num64);
            }
        }
    }
    if (!APPEND && s.ok && s.li[K1 - 1] >= 0 && s.lv[K1 - 1] != last0)
        row_threshold_raise(rowthr, s.row - xb, s.lv[K1 - 1]);
    if (STATS) {
        s.num64 += (double)tnum;
        s.den64 += (double)tden;
        s.cnt += tcnt;
    }
    if (COLS) {
        __syncthreads();  // every lane's queue (in sC's space) is read before the column scores overwrite it
        // each Y row of the tile: its best K1 over this workgroup's 128 X rows (TPR threads per row, merged by
        // shuffles). colthr[j] is the K1-th value of some full list of this chunk, a lower bound of the chunk's
        // K1-th value: scores at or below it cannot enter the merged top-K1 and are skipped.
        static_assert(BY % CPASS == 0 && 256 % CPASS == 0 && CPASS % 32 == 0, "column pass shape");
        constexpr int TPR = 256 / CPASS;  // threads per Y row
        constexpr int XPT = BX / TPR;     // X rows each of them scans
#pragma unroll
        for (int pass = 0; pass < BY / CPASS; ++pass) {
            if (pass > 0) __syncthreads();  // the previous pass's reads of sC are done
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                if (b * 32 < pass * CPASS || b * 32 >= (pass + 1) * CPASS) continue;
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    const int jl = b * 32 + 8 * (q / 4) + 4 * h + (q % 4) - pass * CPASS;
                    sC[jl * CST + wave * 32 + r] = s.ok ? fmaf(scale, tot[b][q], s.qbi) : -INFINITY;
                }
            }
            __syncthreads();
            const int jl = tid / TPR, part = tid % TPR;
            const int64_t j = ytile + pass * CPASS + jl;
            const float thr = j < y_end ? key_float(colthr[j]) : INFINITY;
            float cw[K1];
            int cidx[K1];
#pragma unroll
            for (int i = 0; i < K1; ++i) { cw[i] = -INFINITY; cidx[i] = -1; }
            const float* src = &sC[jl * CST + part * XPT];
            const int base = (int)(x0 + part * XPT);
            for (int xx = 0; xx < XPT; ++xx) {
                const float v = src[xx];
                if (v > thr && v > cw[K1 - 1]) insert_e<K1>(cw, cidx, v, base + xx);
            }
#pragma unroll
            for (int m = 1; m < TPR; m <<= 1) {
                float pv[K1];
                int pi2[K1];
#pragma unroll
                for (int i = 0; i < K1; ++i) {
                    pv[i] = __shfl_xor(cw[i], m, 64);
                    pi2[i] = __shfl_xor(cidx[i], m, 64);
                }
#pragma unroll
                for (int i = 0; i < K1; ++i)
                    if (pi2[i] >= 0 && better_e(pv[i], pi2[i], cw[K1 - 1], cidx[K1 - 1])) insert_e<K1>(cw, cidx, pv[i], pi2[i]);
            }
            if (part == 0 && j < y_end) {
                Entry* dst = colpart + (panel * n + j) * K1;
#pragma unroll
                for (int i = 0; i < K1; ++i) dst[i] = Entry{cw[i], cidx[i]};
                if (cidx[K1 - 1] >= 0) atomicMax(&colthr[j], float_key(cw[K1 - 1]));
            }
        }
    }
    __syncthreads();  // all epilogue reads of sDB/sGE/sC finish before the next tile rewrites them
}

// End of a sweep workgroup: lane lists -> part[(seg*rows + local row)*2 + h][K1], certificate partials reduced
// over the workgroup into blockstats[(seg*P + panel)*5 ...].
template <int K1, bool APPEND>
__device__ __forceinline__ void sweep_finish(SweepRow<K1>& s, int tid, int lane, int wave, int h, int64_t seg,
                                             int64_t rows, int64_t xb, int P, int64_t panel, int STATS,
                                             Entry* __restrict__ part, double* __restrict__ blockstats,
                                             double (*sRed)[5]) {
    if (s.ok && !APPEND) {
        Entry* out = part + ((seg * rows + (s.row - xb)) * 2 + h) * K1;
#pragma unroll
        for (int i = 0; i < K1; ++i) out[i] = Entry{s.lv[i], s.li[i]};
    }
    if (STATS) {
        // the maximum violation (slot 3) is taken exactly from the fp64 row lists after the sweep
        double v[5] = {s.num64, s.den64, (double)s.cnt, 0.0, (double)s.cmax};
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
            double* dst = blockstats + (seg * P + panel) * 5;
            for (int e = 0; e < 5; ++e) dst[e] = o[e];
        }
    }
}

// fp32 sweep: X / Y are the fp32 features (row stride ld = d), products on v_mfma_f32_32x32x2f32.
// APPEND (the wide pass of queued rows): no lists, columns or certificate; every candidate j of row r with
// w >= wthr[r] is appended to wbuf[r * wcap + ...] (wcnt[r] counts all of them, also past the capacity).
template <int K1, bool TWO_LEVEL, bool COLS, bool APPEND = false, bool ST = false>
__global__ __launch_bounds__(256) void l2sq_sweep(
    const float* __restrict__ X, const float* __restrict__ Y, int64_t xb, int64_t xe, int64_t n, int d, int ld,
    const float* __restrict__ qb32, const float* __restrict__ db32, const float* __restrict__ p32,
    const float* __restrict__ ge32, float scale, int64_t seg_len, int P, int S, Entry* __restrict__ part,
    Entry* __restrict__ colpart, unsigned int* __restrict__ colthr, double* __restrict__ blockstats, int VEC4,
    int STATS, CertArgs cert, const float* __restrict__ wthr = nullptr, int* __restrict__ wcnt = nullptr,
    int* __restrict__ wbuf = nullptr, int wcap = 0, unsigned int* __restrict__ rowthr = nullptr) {
    static_assert(!(APPEND && COLS), "the wide pass keeps no column lists");
    int64_t panel, seg;
    sweep_block(blockIdx.x, P, S, panel, seg);
    if (panel >= P || seg >= S) return;  // grid padding (uniform per workgroup, before any barrier)
    __shared__ float sT[2 * STAGE];  // two LDS stages of (X tile, Y tile), 32 features each
    __shared__ double sQB64[STATS_LDS(BX)], sDB64[STATS_LDS(BY)];  // fp64 biases for the certificate's near pairs
    __shared__ float sDB[BY];
    __shared__ float sGE[BY];
    __shared__ __align__(16) float sC[COLS ? BY * CST : 1];
    // queued row candidates (sweep_epilogue); with column lists they use the column-score tile's space
    __shared__ Entry sQ[(APPEND || COLS) ? 1 : 256 * (QN + 1)];
    __shared__ double sRed[4][5];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int h = lane >> 5;    // which half of the 2-wide MFMA k slot
    const int r = lane & 31;    // X row within the wave's 32-row block
    const int64_t rows = xe - xb;
    const int64_t x0 = xb + panel * BX;
    const int64_t y_begin = seg * seg_len;
    const int64_t y_end = (y_begin + seg_len < n) ? (y_begin + seg_len) : n;
    SweepRow<K1> s;
    sweep_row_init<K1, APPEND>(s, x0 + wave * 32 + r, xe, STATS, qb32, p32, wthr);
    const float slack = row_cert_slack(STATS, cert, s.row, s.ok, scale);
    if (!APPEND && tid < BX) sQB64[tid] = (STATS && x0 + tid < xe) ? cert.qb[x0 + tid] : 0.0;

    const int nchunks = (d + KC - 1) / KC;

    // global -> register staging for one chunk: 4 float4 of X and 4 of Y per thread (named registers: an array
    // indexed before unrolling would be moved to LDS or scratch)
    float4 gx0, gx1, gx2, gx3, gy0, gy1, gy2, gy3;  // set A: the chunk after the one being multiplied
    float4 hx0, hx1, hx2, hx3, hy0, hy1, hy2, hy3;  // set B: the chunk after that
    auto load_one = [&](int i, int k0, int64_t ytile, float4& ox, float4& oy) {
        const int lin = tid + 256 * i;
        const int row = lin >> 3, c4 = lin & 7;
        const int k = k0 + 4 * c4;
        const int64_t xr = x0 + row, yr = ytile + row;
        if (VEC4) {
            ox = (xr < xe && k < d) ? *reinterpret_cast<const float4*>(X + xr * ld + k) : make_float4(0, 0, 0, 0);
            oy = (yr < y_end && k < d) ? *reinterpret_cast<const float4*>(Y + yr * ld + k) : make_float4(0, 0, 0, 0);
        } else {
            ox.x = (xr < xe && k < d) ? X[xr * ld + k] : 0.0f;
            ox.y = (xr < xe && k + 1 < d) ? X[xr * ld + k + 1] : 0.0f;
            ox.z = (xr < xe && k + 2 < d) ? X[xr * ld + k + 2] : 0.0f;
            ox.w = (xr < xe && k + 3 < d) ? X[xr * ld + k + 3] : 0.0f;
            oy.x = (yr < y_end && k < d) ? Y[yr * ld + k] : 0.0f;
            oy.y = (yr < y_end && k + 1 < d) ? Y[yr * ld + k + 1] : 0.0f;
            oy.z = (yr < y_end && k + 2 < d) ? Y[yr * ld + k + 2] : 0.0f;
            oy.w = (yr < y_end && k + 3 < d) ? Y[yr * ld + k + 3] : 0.0f;
        }
    };
    auto load_a = [&](int c, int64_t ytile) {
        load_one(0, c * KC, ytile, gx0, gy0);
        load_one(1, c * KC, ytile, gx1, gy1);
        load_one(2, c * KC, ytile, gx2, gy2);
        load_one(3, c * KC, ytile, gx3, gy3);
    };
    auto load_b = [&](int c, int64_t ytile) {
        load_one(0, c * KC, ytile, hx0, hy0);
        load_one(1, c * KC, ytile, hx1, hy1);
        load_one(2, c * KC, ytile, hx2, hy2);
        load_one(3, c * KC, ytile, hx3, hy3);
    };
    auto rotate = [&]() {
        gx0 = hx0; gx1 = hx1; gx2 = hx2; gx3 = hx3;
        gy0 = hy0; gy1 = hy1; gy2 = hy2; gy3 = hy3;
    };
    // chunk f of the tile sequence starting at `tile` (f may run past the tile's chunks into the next tiles); past
    // the segment's end any in-bounds chunk will do, its data is never multiplied
    auto locate = [&](int64_t tile, int f, int64_t& t, int& cc) {
        t = tile;
        cc = f;
        while (cc >= nchunks) {
            cc -= nchunks;
            t += BY;
        }
        if (t >= y_end) {
            t = tile;
            cc = 0;
        }
    };
    auto store_one = [&](float* stage, int i, const float4& vx, const float4& vy) {
        const int lin = tid + 256 * i;
        const int row = lin >> 3, c4 = lin & 7;
        *reinterpret_cast<float4*>(&stage[row * STR + 4 * c4]) = vx;
        *reinterpret_cast<float4*>(&stage[BX * STR + row * STR + 4 * c4]) = vy;
    };
    auto store_chunk = [&](float* stage) {
        store_one(stage, 0, gx0, gy0);
        store_one(stage, 1, gx1, gy1);
        store_one(stage, 2, gx2, gy2);
        store_one(stage, 3, gx3, gy3);
    };

    v16f acc[NB];
    float outer[NB][16];
    // products of one 32-feature chunk held in an LDS stage
    auto compute = [&](const float* sx, const float* sy) {
        // B operand: this lane's X row, features h*16 .. h*16+15 of the chunk
        const float* bx = &sx[(wave * 32 + r) * STR + h * 16];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const float4 bv = *reinterpret_cast<const float4*>(bx + 4 * g);
            float4 av[NB];
#pragma unroll
            for (int b = 0; b < NB; ++b)
                av[b] = *reinterpret_cast<const float4*>(&sy[(b * 32 + r) * STR + h * 16 + 4 * g]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    const float ae = e == 0 ? av[b].x : e == 1 ? av[b].y : e == 2 ? av[b].z : av[b].w;
                    const float be = e == 0 ? bv.x : e == 1 ? bv.y : e == 2 ? bv.z : bv.w;
                    acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(ae, be, acc[b], 0, 0, 0);
                }
            }
        }
    };

    // Software pipeline with two LDS stages, two register sets and one barrier per chunk: while the chunk in stage
    // g&1 is multiplied, the chunk two ahead in the tile sequence is loaded into set B, and set A (the next chunk,
    // loaded one step earlier) is stored to the other stage. The barrier ending a chunk both publishes the next
    // stage and retires all reads of the current one.
    unsigned g = 0;
    {
        int64_t t1;
        int c1;
        load_a(0, y_begin);
        store_chunk(sT);
        locate(y_begin, 1, t1, c1);
        load_a(c1, t1);
        __syncthreads();
    }
    for (int64_t ytile = y_begin; ytile < y_end; ytile += BY) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
#pragma unroll
            for (int q = 0; q < 16; ++q) { acc[b][q] = 0.0f; outer[b][q] = 0.0f; }
        }
        // biases of this tile's Y rows (read in the epilogue, after at least one chunk barrier)
        if (tid < BY) {
            const int64_t j = ytile + tid;
            sDB[tid] = j < y_end ? db32[j] : 0.0f;
            sGE[tid] = (STATS && j < y_end) ? ge32[j] : 0.0f;
            if (!APPEND) sDB64[tid] = (STATS && j < y_end) ? cert.db[j] : 0.0;
        }
        auto step = [&](int c) {
            int64_t t2;
            int c2;
            locate(ytile, c + 2, t2, c2);
            load_b(c2, t2);
            // keep the order loads -> products -> stores: stores hoisted above the products would wait for the
            // loads at once and expose their latency
            asm volatile("" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
            const float* cur = sT + (g & 1u) * STAGE;
            compute(cur, cur + BX * STR);
            asm volatile("" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
            store_chunk(sT + ((g + 1u) & 1u) * STAGE);
            __syncthreads();
            rotate();
            ++g;
        };
        int c = 0;
        if (TWO_LEVEL) {
            // fp32 blocks of FLUSH_CHUNKS chunks folded into the outer sums (the error bound assumes this blocking)
            for (; c + FLUSH_CHUNKS <= nchunks; c += FLUSH_CHUNKS) {
#pragma unroll
                for (int u = 0; u < FLUSH_CHUNKS; ++u) step(c + u);
#pragma unroll
                for (int b = 0; b < NB; ++b) {
#pragma unroll
                    for (int q = 0; q < 16; ++q) { outer[b][q] += acc[b][q]; acc[b][q] = 0.0f; }
                }
            }
        }
        for (; c < nchunks; ++c) step(c);
        if (TWO_LEVEL) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
#pragma unroll
                for (int q = 0; q < 16; ++q) acc[b][q] = outer[b][q] + acc[b][q];
            }
        }
#define HM_EPILOGUE(FULL_TILE)                                                                                  \
    sweep_epilogue<K1, COLS, APPEND, BY, FULL_TILE, ST>(acc, s, tid, wave, h, r, ytile, y_end, x0, panel, n, scale,  \
                                                   STATS, slack, sQB64, sDB64, sDB, sGE, sC, colpart, colthr,    \
                                                   wcnt, wbuf, wcap, rowthr, xb,                                 \
                                                   COLS ? reinterpret_cast<Entry*>(sC) : sQ)
        if (y_end - ytile >= (int64_t)(NB * 32) && x0 + BX <= xe) HM_EPILOGUE(true);
        else HM_EPILOGUE(false);
#undef HM_EPILOGUE
    }
    sweep_finish<K1, APPEND>(s, tid, lane, wave, h, seg, rows, xb, P, panel, STATS, part, blockstats, sRed);
}

// -------------------------------------------------------------------------------------------------
// split-bf16 sweep for d <= 128 (X / Y: split copies in operand order, see l2sq_split_bf16; d = split_features,
// which is 1, 2 or 4 chunks; ld = split_ld). dot = hi*hi + hi*lo + lo*hi on v_mfma_f32_32x32x16_bf16 in one fp32
// block; longer rows take l2sq_sweep_split_w.
//
// Data flow per chunk of 32 features:
//   X: the panel's operands (at most 4 chunks) are loaded once into registers and stay for the whole segment (a
//      wave is the only reader of its 32 rows).
//   Y: the tile's chunk (4 blocks x 4 KiB) goes straight from global memory to a ring of LDS stages
//      (global_load_lds_dwordx4: each wave instruction writes 1 KiB), one stage fewer chunks ahead of the one
//      multiplied than the ring has stages; no staging registers, no LDS stores.
// One barrier per chunk, between its two K-steps. Before it, the products of K-step 0 run while the operands of
// K-step 1 are read from LDS and the loads ahead are issued into the stage the previous chunk used (all its reads
// retired at the previous barrier); each wave then waits for its own loads of the next chunk, so the barrier
// publishes that stage. After it, the products of K-step 1 run while the next chunk's K-step-0 operands are read.
// -------------------------------------------------------------------------------------------------
constexpr int SPLIT_STAGES = 3;  // LDS ring of Y chunks (16 KiB each): 49 KiB of LDS, two workgroups per CU

struct XOps { float4 h0, l0, h1, l1; };                  // this lane's X operands of one chunk (K-steps 0 and 1)
struct YOps { float4 h0, h1, h2, h3, l0, l1, l2, l3; };  // A operands of one K-step for the Y blocks 0..3

__device__ __forceinline__ float4 ld16(const float* base, unsigned byte_off) {
    return *reinterpret_cast<const float4*>(reinterpret_cast<const char*>(base) + byte_off);
}
__device__ __forceinline__ bf16x8 as_bf16x8(const float4& v) { return __builtin_bit_cast(bf16x8, v); }

// one K-step: acc[b] += Y_hi*X_hi, then Y_hi*X_lo, then Y_lo*X_hi; with ZERO the first products start from 0
// (the accumulators' first K-step of a tile: the MFMA takes 0 as its addend, so no clearing is needed)
template <bool ZERO = false>
__device__ __forceinline__ void split_kstep(v16f (&acc)[NB], const YOps& a, const float4& xh4, const float4& xl4) {
    const bf16x8 xh = as_bf16x8(xh4), xl = as_bf16x8(xl4);
    const v16f zero = {};
    acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a.h0), xh, ZERO ? zero : acc[0], 0, 0, 0);
    acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a.h1), xh, ZERO ? zero : acc[1], 0, 0, 0);
    acc[2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a.h2), xh, ZERO ? zero : acc[2], 0, 0, 0);
    acc[3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a.h3), xh, ZERO ? zero : acc[3], 0, 0, 0);
    acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a.h0), xl, acc[0], 0, 0, 0);
    acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a.h1), xl, acc[1], 0, 0, 0);
    acc[2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a.h2), xl, acc[2], 0, 0, 0);
    acc[3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a.h3), xl, acc[3], 0, 0, 0);
    acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a.l0), xh, acc[0], 0, 0, 0);
    acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a.l1), xh, acc[1], 0, 0, 0);
    acc[2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a.l2), xh, acc[2], 0, 0, 0);
    acc[3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a.l3), xh, acc[3], 0, 0, 0);
}

template <int U>
__device__ __forceinline__ float4* xset_stage(float4* a, float4* b, float4* c, float4* d) {
    if constexpr (U == 0) return a;
    else if constexpr (U == 1) return b;
    else if constexpr (U == 2) return c;
    else return d;
}

template <int U>
__device__ __forceinline__ XOps& xset(XOps& a, XOps& b, XOps& c, XOps& d) {
    if constexpr (U == 0) return a;
    else if constexpr (U == 1) return b;
    else if constexpr (U == 2) return c;
    else return d;
}

// Four loads of 16 bytes per lane from global memory straight to LDS: lane l reads b_i + off (b_i wave-uniform, a
// 32-bit byte offset per lane) and writes lds_i + 16 l (M0 holds the wave-uniform LDS address; it is saved once and
// restored, so the compiler's use of it, if any, is untouched). Issued from assembly: the compiler would otherwise
// treat every later LDS read as a possible alias of these writes and wait for all outstanding loads before it. The
// caller waits (wait_vmcnt) before the data is read, and before the workgroup ends.
__device__ __forceinline__ void load_lds16x4(const char* b0, const char* b1, const char* b2, const char* b3,
                                             unsigned off, unsigned l0, unsigned l1, unsigned l2, unsigned l3) {
    unsigned saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %6\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2\n\ts_nop 0\n\t"
        "s_mov_b32 m0, %7\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %3\n\ts_nop 0\n\t"
        "s_mov_b32 m0, %8\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %4\n\ts_nop 0\n\t"
        "s_mov_b32 m0, %9\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %5\n\ts_nop 0\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(off), "s"(b0), "s"(b1), "s"(b2), "s"(b3), "s"(l0), "s"(l1), "s"(l2), "s"(l3));
}

// the wave-uniform LDS byte address of a shared-memory pointer (for M0)
__device__ __forceinline__ unsigned lds_addr(const void* p) {
    return __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)p);
}

// the lane's index, computed where it is used: the compiler cannot hoist it out of a loop and keep it (or what is
// derived from it) live across the loop, where it would spill
__device__ __forceinline__ unsigned lane_here() {
    unsigned l;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
    return l;
}

// 4 bytes per lane from global memory straight to LDS: lane l reads base + off (a wave-uniform base, a 32-bit
// byte offset per lane) and writes lds_byte + 4 l. As load_lds16x4.
__device__ __forceinline__ void load_lds4(const void* base, unsigned off, unsigned lds_byte) {
    unsigned saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2\n\ts_nop 0\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(off), "s"(base), "s"(lds_byte));
}

// s_waitcnt that waits for the vector-memory counter only (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt
// and lgkmcnt at their maxima)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Barrier of the split sweep's chunk loop: this wave's loads older than the last N have landed (the stage the
// barrier publishes) and its LDS reads are done (the stage refilled after the barrier). No release fence: the
// fence of __syncthreads would also wait for the loads still in flight to the other stages. The empty asm
// statements keep the compiler from moving memory accesses across the barrier.
template <int N>
__device__ __forceinline__ void ring_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// scheduling groups (masks of __builtin_amdgcn_sched_group_barrier)
constexpr int SG_VALU = 0x002, SG_MFMA = 0x008, SG_VMEM_READ = 0x020, SG_DS_READ = 0x100;

template <int K1, bool COLS, bool APPEND = false, bool ST = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(COLS ? 1 : 2))) void l2sq_sweep_split(
    const float* __restrict__ X, const float* __restrict__ Y, int64_t xb, int64_t xe, int64_t n, int d, int ld,
    const float* __restrict__ qb32, const float* __restrict__ db32, const float* __restrict__ p32,
    const float* __restrict__ ge32, float scale, int64_t seg_len, int P, int S, Entry* __restrict__ part,
    Entry* __restrict__ colpart, unsigned int* __restrict__ colthr, double* __restrict__ blockstats, int STATS,
    CertArgs cert, const float* __restrict__ wthr = nullptr, int* __restrict__ wcnt = nullptr,
    int* __restrict__ wbuf = nullptr,
    int wcap = 0, unsigned int* __restrict__ rowthr = nullptr) {
    static_assert(!(APPEND && COLS), "the wide pass keeps no column lists");
    // Ring of Y chunks: the stage index is dynamic, so the loads are issued from assembly (there are no other
    // loads in the chunk loop to count)
    constexpr int NS = SPLIT_STAGES;
    constexpr int AHEAD = NS - 1;  // Y chunks in flight ahead of the one multiplied
    constexpr int VMEM_STEP = 4;   // vector-memory instructions a chunk issues
    int64_t panel, seg;
    sweep_block(blockIdx.x, P, S, panel, seg);
    if (panel >= P || seg >= S) return;  // grid padding (uniform per workgroup, before any barrier)
    __shared__ float4 sY0[1024], sY1[1024], sY2[1024];  // LDS ring (Y chunk: 4 blocks x 4 KiB)
    __shared__ double sQB64[STATS_LDS(BX)], sDB64[STATS_LDS(BY)];  // fp64 biases for the certificate's near pairs
    __shared__ float sDB[BY];
    __shared__ float sGE[BY];
    __shared__ __align__(16) float sC[COLS ? BY * CST : 1];
    // queued row candidates (sweep_epilogue); with column lists they use the column-score tile's space
    __shared__ Entry sQ[(APPEND || COLS) ? 1 : 256 * (QN + 1)];
    __shared__ double sRed[4][5];
    __shared__ unsigned int sRT[APPEND ? 1 : BX];  // the panel's shared row thresholds, read per tile

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5;
    const int r = lane & 31;
    const int64_t rows = xe - xb;
    const int64_t x0 = xb + panel * BX;
    const int64_t y_begin = seg * seg_len;
    const int64_t y_end = (y_begin + seg_len < n) ? (y_begin + seg_len) : n;
    SweepRow<K1> s;
    sweep_row_init<K1, APPEND>(s, x0 + wave * 32 + r, xe, STATS, qb32, p32, wthr);
    const float slack = row_cert_slack(STATS, cert, s.row, s.ok, scale);
    if (!APPEND && tid < BX) sQB64[tid] = (STATS && x0 + tid < xe) ? cert.qb[x0 + tid] : 0.0;
    const bool stats = ST && STATS != 0;  // the certificate's biases are loaded per tile

    const int nchunks = d / KC;
    const int64_t bstride = (int64_t)ld * 32;          // words per 32-row block
    const float* Xw = X + (((x0 - xb) >> 5) + wave) * bstride;  // this wave's X block (X starts at row xb)
    const unsigned lane16 = (unsigned)lane * 16u;
    const unsigned tid16 = (unsigned)tid * 16u;
    const unsigned ystep = (unsigned)(bstride * 4);     // bytes between consecutive Y blocks

    auto load_x = [&](XOps& o, int cc) {
        const float* b = Xw + cc * 1024;
        o.h0 = ld16(b, lane16);
        o.l0 = ld16(b, 1024u + lane16);
        o.h1 = ld16(b, 2048u + lane16);
        o.l1 = ld16(b, 3072u + lane16);
    };
    // Y chunk position AHEAD chunks past the one multiplied (ta, ca) and its address ya (chunk ca of the tile at
    // row ta: Y + ta*ld + ca*1024 words), advanced chunk by chunk; past the segment any in-bounds chunk will do, its
    // data is never multiplied. Branch-free, so that a chunk step stays one scheduling region.
    int64_t ta = y_begin;
    int ca = 0;
    const char* const yfirst = reinterpret_cast<const char*>(Y + (y_begin >> 5) * bstride);
    const char* ya = yfirst;
    const int64_t wrap_bytes = (4 * bstride - (int64_t)(nchunks - 1) * 1024) * 4;  // last chunk -> next tile's first
    auto load_ahead = [&](float4* stage) {
        const char* b = ta < y_end ? ya : yfirst;
        // thread t's 16 bytes of block i go to stage + i*4 KiB + t*16; one wave instruction fills 1 KiB
        const unsigned dst = lds_addr(stage + wave * 64);
        load_lds16x4(b, b + ystep, b + 2 * ystep, b + 3 * ystep, tid16, dst, dst + 4096u, dst + 8192u, dst + 12288u);
        ++ca;
        const bool wrap = ca == nchunks;
        ca = wrap ? 0 : ca;
        ta = wrap ? ta + BY : ta;
        ya += wrap ? wrap_bytes : 4096;
    };
    auto read_ops = [&](YOps& o, const float4* stage, int ks) {
        const float4* src = stage + ks * 128 + lane;
        o.h0 = src[0];
        o.l0 = src[64];
        o.h1 = src[256];
        o.l1 = src[320];
        o.h2 = src[512];
        o.l2 = src[576];
        o.h3 = src[768];
        o.l3 = src[832];
    };

    XOps xs0, xs1, xs2, xs3;  // X operands of chunks 0..3
    YOps o0, o1;              // Y operands of K-steps 0 and 1
    // LDS stages of the chunk being multiplied, the next one, and the one refilled (with the chunk AHEAD further)
    float4 *cur = sY0, *nxt = sY1, *fill = sY2;
    static_assert(NS == 3, "three stages rotate");

    static_assert(AHEAD == 2, "initial ring fill");
    load_ahead(sY0);
    load_ahead(sY1);
    load_x(xs0, 0);
    if (nchunks > 1) load_x(xs1, 1);
    if (nchunks > 2) {
        load_x(xs2, 2);
        load_x(xs3, 3);
    }
    wait_vmcnt<0>();
    __syncthreads();
    read_ops(o0, sY0, 0);

    v16f acc[NB];

    // chunk c = U of the tile
    auto step = [&](auto uc) {
        constexpr int U = decltype(uc)::value;
        XOps& xs = xset<U>(xs0, xs1, xs2, xs3);
        // K-step 0, then the Y chunk AHEAD further into the stage chunk - 1 used
        read_ops(o1, cur, 1);
        split_kstep<U == 0>(acc, o0, xs.h0, xs.l0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
            __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(SG_MFMA, 8, 0);
        __builtin_amdgcn_sched_barrier(0);
        // this wave's loads of the next chunk were issued AHEAD - 1 chunks back, so at most the later chunks'
        // instructions may still be in flight
        load_ahead(fill);
        ring_barrier<(AHEAD - 1) * VMEM_STEP>();
        // K-step 1; the next chunk's K-step-0 operands
        read_ops(o0, nxt, 0);
        split_kstep(acc, o1, xs.h1, xs.l1);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
            __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(SG_MFMA, 8, 0);
        __builtin_amdgcn_sched_barrier(0);
        float4* const used = cur;
        cur = nxt;
        nxt = fill;
        fill = used;
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;

    for (int64_t ytile = y_begin; ytile < y_end; ytile += BY) {
        // (the tile's first K-step starts the accumulators from 0)
        // biases of this tile's Y rows and the panel's shared row thresholds, straight to LDS; the epilogue reads
        // them after the first chunk's ring barrier, which waits for them as for any load older than the chunk's
        // (loads into registers would need a wait of their own, and with it for the Y chunks in flight). Columns
        // past the segment read the last one in it; the epilogue skips their pairs.
        {
            // offsets within the tile, the last column of the segment for those past it (wave-uniform bases)
            const unsigned ln = lane_here();
            const unsigned jlim = (unsigned)(y_end - 1 - ytile);
            auto col = [&](unsigned t) { return t < jlim ? t : jlim; };
            if (wave < 2) {
                load_lds4(db32 + ytile, col(wave * 64 + ln) * 4u, lds_addr(sDB + wave * 64));
                if (!APPEND && rowthr) {
                    const unsigned xlim = (unsigned)(xe - 1 - x0);
                    const unsigned t = wave * 64 + ln;
                    load_lds4(rowthr + (x0 - xb), (t < xlim ? t : xlim) * 4u, lds_addr(sRT + wave * 64));
                }
            } else if (stats) {
                load_lds4(ge32 + ytile, col((wave - 2) * 64 + ln) * 4u, lds_addr(sGE + (wave - 2) * 64));
            }
            if (stats && !APPEND)  // the fp64 biases as 256 dwords, 64 per wave
                load_lds4(cert.db + ytile, col(wave * 32 + (ln >> 1)) * 8u + (ln & 1) * 4u,
                          lds_addr(sDB64 + wave * 32));
        }
        step(I0{});
        if (nchunks > 1) step(I1{});
        if (nchunks > 2) {
            step(I2{});
            step(I3{});
        }
#define HM_EPILOGUE(FULL_TILE)                                                                                  \
    sweep_epilogue<K1, COLS, APPEND, BY, FULL_TILE, ST, true>(acc, s, tid, wave, h, r, ytile, y_end, x0, panel, n,   \
                                                   scale, STATS, slack, sQB64, sDB64, sDB, sGE, sC, colpart,     \
                                                   colthr, wcnt, wbuf, wcap, rowthr, xb,                         \
                                                   COLS ? reinterpret_cast<Entry*>(sC) : sQ, sRT)
        if (y_end - ytile >= (int64_t)(NB * 32) && x0 + BX <= xe) HM_EPILOGUE(true);
        else HM_EPILOGUE(false);
#undef HM_EPILOGUE
    }
    wait_vmcnt<0>();  // the loads ahead into LDS land before the workgroup can end
    sweep_finish<K1, APPEND>(s, tid, lane, wave, h, seg, rows, xb, P, panel, STATS, part, blockstats, sRed);
}

// -------------------------------------------------------------------------------------------------
// split-bf16 sweep over 256-row X panels, for d > 128 (outer sums; d a multiple of 4 chunks). Same copies,
// products and Y ring as l2sq_sweep_split, with 8 waves (two per SIMD), each owning 32 X rows against the tile's
// 128 Y rows: per chunk a CU fetches 48 KiB for twice the products of the 128-row panel's 32 KiB, and the 8
// concurrent panels of an XCD hit its L2 far more often (83% against 53% of requests at d = 8192).
//   X: each wave's operands come straight to registers, two sets, chunk c in set c % 2, loaded one chunk ahead.
//   Y operands: read from LDS right before their pass (the other wave of the SIMD multiplies meanwhile), so that at
//      most two halves of a K-step are live; every read of a chunk's stage precedes the barrier after which the
//      stage may be refilled.
//   Accumulators: one set of 4 blocks (32 Y rows x 32 X rows each) and their outer sums, all in the 256 registers
//      a wave has at two waves per SIMD. Block y restarts at the chunks c = y (mod 4): its accumulator is folded
//      into the outer sums (outer += acc) and its first product of the chunk starts from zero. So every fp32 block
//      spans at most 4 chunks (128 features), a dot is the ordered fp32 sum of at most d / 128 + 1 blocks, and one
//      block is folded per chunk.
//   Row lists: lane (h, r) of wave w holds X row 32w + r; its partial list lives in `part` between tiles (each
//      epilogue reads it, merges the tile and writes it back), so the chunk loop carries no lists.
//   Columns: the tile's scores pass through LDS 64 Y rows at a time; 8 threads per Y row scan 32 X rows each
//      (panel rows t, t + 8, ...: a stride that spreads the reads over the LDS banks) into lists of 64-bit keys
//      (score order, then lower index), merged across the 8 by bitonic merges.
// -------------------------------------------------------------------------------------------------
constexpr int BXW = 256;                // X rows per workgroup of the 256-row split sweep
constexpr int WAVES_W = BXW / 32;       // waves per workgroup (32 X rows each)
constexpr int THREADS_W = 64 * WAVES_W;
constexpr int CSTW = BXW + 8;           // LDS row stride of its column-score pass (floats)
constexpr int CROWS_W = 64;             // Y rows per column-score pass

template <int U>
__device__ __forceinline__ XOps& xset2(XOps& a, XOps& b) {
    if constexpr ((U & 1) == 0) return a;
    else return b;
}

// Y operands of one K-step in two halves: the hi parts of the 4 Y blocks, and the lo parts
struct YHalf { float4 b0, b1, b2, b3; };

template <int Y>
__device__ __forceinline__ const float4& yhalf_at(const YHalf& a) {
    if constexpr (Y == 0) return a.b0;
    else if constexpr (Y == 1) return a.b1;
    else if constexpr (Y == 2) return a.b2;
    else return a.b3;
}

// Products of one pass over the 4 Y blocks: acc[y] += Y_part(y) * X_part. With R >= 0 the pass takes the blocks
// from R + 1 on, R last; with FOLD, block R is first folded into outer (outer += acc) and its product starts from
// zero (the block restarts).
template <int R, bool FOLD, int I>
__device__ __forceinline__ void pass_one(v16f (&acc)[NB], float (&outer)[NB][16], const YHalf& yp, const bf16x8& xv) {
    constexpr int y = R < 0 ? I : (R + 1 + I) % NB;
    const bf16x8 yv = as_bf16x8(yhalf_at<y>(yp));
    if constexpr (FOLD && y == R) {
#pragma unroll
        for (int q = 0; q < 16; ++q) outer[y][q] += acc[y][q];
        const v16f zero = {};
        acc[y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(yv, xv, zero, 0, 0, 0);
    } else {
        acc[y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(yv, xv, acc[y], 0, 0, 0);
    }
}

template <int R, bool FOLD>
__device__ __forceinline__ void split_pass(v16f (&acc)[NB], float (&outer)[NB][16], const YHalf& yp, const float4& x4) {
    const bf16x8 xv = as_bf16x8(x4);
    pass_one<R, FOLD, 0>(acc, outer, yp, xv);
    pass_one<R, FOLD, 1>(acc, outer, yp, xv);
    pass_one<R, FOLD, 2>(acc, outer, yp, xv);
    pass_one<R, FOLD, 3>(acc, outer, yp, xv);
}

// Column candidates of the 256-row sweep as 64-bit keys: float_key of the score (with -0 taken as +0, so that
// equal scores compare equal) above the complement of the X index, so that a larger key is a better entry (higher
// score, then lower index: the order of better_e); the empty entry (-inf, -1) is the smallest key of all.
constexpr unsigned long long CAND_EMPTY = (unsigned long long)0x007fffffu << 32;  // float_key(-inf), index -1
__device__ __forceinline__ unsigned long long cand_key(float v, int i) {
    return ((unsigned long long)float_key(v + 0.0f) << 32) | (unsigned int)~i;
}
__device__ __forceinline__ float cand_value(unsigned long long k) { return key_float((unsigned int)(k >> 32)); }
__device__ __forceinline__ int cand_index(unsigned long long k) { return (int)~(unsigned int)k; }

// insert kv into the descending list k[0..K) (the smallest entry drops out)
template <int K>
__device__ __forceinline__ void cand_insert(unsigned long long (&k)[K], unsigned long long kv) {
#pragma unroll
    for (int i = 0; i < K; ++i) {
        const bool c = kv > k[i];
        const unsigned long long t = k[i];
        k[i] = c ? kv : t;
        kv = c ? t : kv;
    }
}

// k := the best K of k and the descending list of the lane `m` apart (xor): the elementwise maximum of k and the
// other list reversed is a bitonic sequence holding the best K of both, which a bitonic sorter puts in order
template <int K>
__device__ __forceinline__ void cand_merge(unsigned long long (&k)[K], int m) {
    static_assert((K & (K - 1)) == 0, "power-of-two list");
    unsigned long long o[K];
#pragma unroll
    for (int i = 0; i < K; ++i) {
        const unsigned long long v = k[K - 1 - i];
        const unsigned int lo = __shfl_xor((unsigned int)v, m, 64);
        const unsigned int hi = __shfl_xor((unsigned int)(v >> 32), m, 64);
        o[i] = ((unsigned long long)hi << 32) | lo;
    }
#pragma unroll
    for (int i = 0; i < K; ++i) k[i] = k[i] > o[i] ? k[i] : o[i];
#pragma unroll
    for (int s = K / 2; s >= 1; s >>= 1) {
#pragma unroll
        for (int i = 0; i < K; ++i) {
            if ((i & s) == 0) {
                const unsigned long long a = k[i], b = k[i + s];
                const bool c = a > b;
                k[i] = c ? a : b;
                k[i + s] = c ? b : a;
            }
        }
    }
}

// Epilogue of the 256-row split sweep for one tile. tot[y][q] is the fp32 dot of the lane's X row with Y row
// ytile + 32y + 8(q/4) + 4h + q%4. Rows: the lane's list (half h of segment seg) is read from `part` (or starts
// empty at the segment's first tile), takes w = scale*dot + db in increasing j and is written back; APPEND
// queues candidates instead. Columns as in sweep_epilogue, over the panel's 256 X rows.
template <int K1, bool COLS, bool APPEND, bool ST>
__device__ __forceinline__ void sweep_epilogue_w(const float (&tot)[NB][16], int64_t row, bool ok, float qbi,
                                                 float pi, float wt, bool first, int tid, int wave, int h, int r,
                                                 int64_t ytile, int64_t y_end, int64_t x0, int64_t xb, int64_t rows,
                                                 int64_t seg, int64_t panel, int64_t n, float scale, int STATS_,
                                                 float slack, const double* sQB64, const double* sDB64,
                                                 const float* sDB, const float* sGE, float* sC,
                                                 Entry* __restrict__ part, Entry* __restrict__ colpart,
                                                 unsigned int* __restrict__ colthr, int* __restrict__ wcnt,
                                                 int* __restrict__ wbuf, int wcap, double& num64, double& den64,
                                                 unsigned int& cnt, float& cmax,
                                                 unsigned int* __restrict__ rowthr) {
    const int STATS = ST ? STATS_ : 0;  // as in sweep_epilogue
    float tnum = 0.0f, tden = 0.0f;
    unsigned int tcnt = 0;
    bool near = false;  // a pair of this tile within the certificate slack (cert_fast)
    // Y rows of the tile inside the segment; pair (lane half h, offset c) is inside when 4h < ylim - c, a compare
    // against a wave-uniform bound
    const int ylim = (int)(y_end - ytile < (int64_t)(NB * 32) ? y_end - ytile : (int64_t)(NB * 32));
    float lv[APPEND ? 1 : K1];
    int li[APPEND ? 1 : K1];
    Entry* lp = APPEND ? nullptr : part + ((seg * rows + (row - xb)) * 2 + h) * K1;
    if (!APPEND) {
#pragma unroll
        for (int i = 0; i < K1; ++i) {
            Entry e{-INFINITY, -1};
            if (ok && !first) e = lp[i];
            lv[i] = e.w;
            li[i] = e.j;
        }
    }
    // the row's shared threshold: scores at or below it cannot enter the row's merged lists (row_threshold_*)
    const float rthr = (!APPEND && ok) ? row_threshold_get(rowthr, row - xb) : -INFINITY;
    const float last0 = APPEND ? 0.0f : lv[K1 - 1];
#pragma unroll
    for (int y = 0; y < NB; ++y) {
#pragma unroll
        for (int a = 0; a < 4; ++a) {
            const int jl0 = y * 32 + 8 * a + 4 * h;
            const float4 dbv = *reinterpret_cast<const float4*>(&sDB[jl0]);
            float4 gev = make_float4(0, 0, 0, 0);
            if (STATS) gev = *reinterpret_cast<const float4*>(&sGE[jl0]);
            const float dbs[4] = {dbv.x, dbv.y, dbv.z, dbv.w};
            const float ges[4] = {gev.x, gev.y, gev.z, gev.w};
            // the lane's largest score of the group: its scores are tested for the list only when some lane of
            // the wave has one above its list's last entry and the shared threshold
            float amax = -INFINITY;
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
                const float t = tot[y][4 * a + cc];
                const float w = fmaf(scale, t, dbs[cc]);
                const int64_t j = ytile + jl0 + cc;
                const bool okj = ok && 4 * h < ylim - (y * 32 + 8 * a + cc);
                if constexpr (APPEND) {
                    if (okj && w >= wt) {
                        const int pos = atomicAdd(&wcnt[row], 1);
                        if (pos < wcap) wbuf[row * (int64_t)wcap + pos] = (int)j;
                    }
                } else {
                    amax = fmaxf(amax, okj ? w : -INFINITY);
                }
                if (STATS) cert_fast(okj, w, ges[cc], pi, qbi, slack, tden, cmax, tnum, tcnt, near);
            }
            if (!APPEND && __any(amax > fmaxf(lv[K1 - 1], rthr))) {
                // the group's scores in pair order, each inserted when it beats the list's last entry (as if
                // every score had been tested)
#pragma unroll
                for (int cc = 0; cc < 4; ++cc) {
                    const float w = fmaf(scale, tot[y][4 * a + cc], dbs[cc]);
                    const bool okj = ok && 4 * h < ylim - (y * 32 + 8 * a + cc);
                    if (okj && w > lv[K1 - 1] && w > rthr) {
                        float cv = w;
                        int ci = (int)(ytile + jl0 + cc);
#pragma unroll
                        for (int i = 0; i < K1; ++i) {
                            if (cv > lv[i]) {
                                const float tv = lv[i];
                                const int ti = li[i];
                                lv[i] = cv;
                                li[i] = ci;
                                cv = tv;
                                ci = ti;
                            }
                        }
                    }
                }
            }
            // one group of pairs at a time: the scheduler would otherwise hoist every group's LDS reads to the
            // top of the epilogue and spill them
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    if (STATS && near) {
        // reload the biases rather than keep the fast path's values alive in registers through the tile
        asm volatile("" ::: "memory");
        const double qb64 = sQB64[wave * 32 + r];
#pragma unroll
        for (int y = 0; y < NB; ++y) {
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int jl = y * 32 + 8 * (q / 4) + 4 * h + (q % 4);
                const float t = tot[y][q];
                cert_near(ok && 4 * h < ylim - (jl - 4 * h), t, fmaf(scale, t, sDB[jl]), qbi, slack, scale, qb64, sDB64[jl],
                          tcnt, num64);
            }
        }
    }
    if (!APPEND && ok) {
#pragma unroll
        for (int i = 0; i < K1; ++i) lp[i] = Entry{lv[i], li[i]};
        if (li[K1 - 1] >= 0 && lv[K1 - 1] != last0) row_threshold_raise(rowthr, row - xb, lv[K1 - 1]);
    }
    if (STATS) {
        num64 += (double)tnum;
        den64 += (double)tden;
        cnt += tcnt;
    }
    if (COLS) {
        // each Y row of the tile: its best K1 over the panel's 256 X rows, 64 Y rows per pass (8 threads per row
        // scanning 32 X rows each, then merged across the 8); colthr[j] bounds the chunk's K1-th value from below,
        // as in sweep_epilogue
        constexpr int TPR = THREADS_W / CROWS_W;  // threads per Y row
        constexpr int XPT = BXW / TPR;            // X rows each of them scans (panel rows t, t + TPR, ...)
#pragma unroll
        for (int pass = 0; pass < NB * 32 / CROWS_W; ++pass) {
            if (pass > 0) __syncthreads();  // the previous pass's reads of sC are done
#pragma unroll
            for (int bb = 0; bb < CROWS_W / 32; ++bb) {
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    const int jl = bb * 32 + 8 * (q / 4) + 4 * h + (q % 4);
                    sC[jl * CSTW + wave * 32 + r] =
                        ok ? fmaf(scale, tot[pass * (CROWS_W / 32) + bb][q], qbi) : -INFINITY;
                }
            }
            __syncthreads();
            const int jl = tid / TPR, part8 = tid % TPR;
            const int64_t j = ytile + pass * CROWS_W + jl;
            const float thr = j < y_end ? key_float(colthr[j]) : INFINITY;
            const float* src = &sC[jl * CSTW + part8];
            const int base = (int)(x0 + part8);
            Entry* dst = colpart + (panel * n + j) * K1;
            if constexpr ((K1 & (K1 - 1)) == 0) {
                // candidates as 64-bit keys (value order, then lower index): insertion while scanning, bitonic
                // merges across the row's threads
                unsigned long long key[K1];
#pragma unroll
                for (int i = 0; i < K1; ++i) key[i] = CAND_EMPTY;
                for (int xx = 0; xx < XPT; ++xx) {
                    const float v = src[TPR * xx];
                    if (v > thr) {
                        const unsigned long long kv = cand_key(v, base + TPR * xx);
                        if (kv > key[K1 - 1]) cand_insert<K1>(key, kv);
                    }
                }
#pragma unroll
                for (int m = 1; m < TPR; m <<= 1) cand_merge<K1>(key, m);
                if (part8 == 0 && j < y_end) {
#pragma unroll
                    for (int i = 0; i < K1; ++i) dst[i] = Entry{cand_value(key[i]), cand_index(key[i])};
                    if (cand_index(key[K1 - 1]) >= 0) atomicMax(&colthr[j], (unsigned int)(key[K1 - 1] >> 32));
                }
            } else {
                float cw[K1];
                int cidx[K1];
#pragma unroll
                for (int i = 0; i < K1; ++i) { cw[i] = -INFINITY; cidx[i] = -1; }
                for (int xx = 0; xx < XPT; ++xx) {
                    const float v = src[TPR * xx];
                    if (v > thr && v > cw[K1 - 1]) insert_e<K1>(cw, cidx, v, base + TPR * xx);
                }
#pragma unroll
                for (int m = 1; m < TPR; m <<= 1) {
                    float pv[K1];
                    int pi2[K1];
#pragma unroll
                    for (int i = 0; i < K1; ++i) {
                        pv[i] = __shfl_xor(cw[i], m, 64);
                        pi2[i] = __shfl_xor(cidx[i], m, 64);
                    }
#pragma unroll
                    for (int i = 0; i < K1; ++i)
                        if (pi2[i] >= 0 && better_e(pv[i], pi2[i], cw[K1 - 1], cidx[K1 - 1]))
                            insert_e<K1>(cw, cidx, pv[i], pi2[i]);
                }
                if (part8 == 0 && j < y_end) {
#pragma unroll
                    for (int i = 0; i < K1; ++i) dst[i] = Entry{cw[i], cidx[i]};
                    if (cidx[K1 - 1] >= 0) atomicMax(&colthr[j], float_key(cw[K1 - 1]));
                }
            }
        }
    }
    __syncthreads();  // all epilogue reads of sDB/sGE/sC finish before the next tile rewrites them
}

template <int K1, bool COLS, bool APPEND = false, bool ST = false>
__global__ __launch_bounds__(THREADS_W) void l2sq_sweep_split_w(
    const float* __restrict__ X, const float* __restrict__ Y, int64_t xb, int64_t xe, int64_t n, int d, int ld,
    const float* __restrict__ qb32, const float* __restrict__ db32, const float* __restrict__ p32,
    const float* __restrict__ ge32, float scale, int64_t seg_len, int P, int S, Entry* __restrict__ part,
    Entry* __restrict__ colpart, unsigned int* __restrict__ colthr, double* __restrict__ blockstats, int STATS,
    CertArgs cert, const float* __restrict__ wthr = nullptr, int* __restrict__ wcnt = nullptr,
    int* __restrict__ wbuf = nullptr,
    int wcap = 0, unsigned int* __restrict__ rowthr = nullptr) {
    static_assert(!(APPEND && COLS), "the wide pass keeps no column lists");
    constexpr int AHEAD = 3;      // Y chunks in flight ahead of the one multiplied (4-stage ring)
    constexpr int VMEM_STEP = 6;  // vector-memory instructions a chunk issues (4 X, then 2 Y)
    int64_t panel, seg;
    sweep_block(blockIdx.x, P, S, panel, seg);
    if (panel >= P || seg >= S) return;  // grid padding (uniform per workgroup, before any barrier)
    __shared__ float4 sY0[1024], sY1[1024], sY2[1024], sY3[1024];  // LDS ring (Y chunk: 4 blocks x 4 KiB)
    __shared__ double sQB64[STATS_LDS(BXW)], sDB64[STATS_LDS(BY)];  // fp64 biases for the certificate's near pairs
    __shared__ float sDB[BY];
    __shared__ float sGE[BY];
    __shared__ float sC[COLS ? CROWS_W * CSTW : 1];
    __shared__ double sRed[WAVES_W][5];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5;
    const int r = lane & 31;
    const int64_t rows = xe - xb;
    const int64_t x0 = xb + panel * BXW;
    const int64_t y_begin = seg * seg_len;
    const int64_t y_end = (y_begin + seg_len < n) ? (y_begin + seg_len) : n;
    const int64_t row = x0 + wave * 32 + r;
    const bool ok = row < xe;
    const float qbi = (ok && !APPEND) ? qb32[row] : 0.0f;
    const float pi = (STATS && ok) ? p32[row] : 0.0f;
    const float wt = (APPEND && ok) ? wthr[row] : INFINITY;
    double num64 = 0.0, den64 = 0.0;
    unsigned int cnt = 0u;
    float cmax = 0.0f;
    const float slack = row_cert_slack(STATS, cert, row, ok, scale);
    if (!APPEND && tid < BXW) sQB64[tid] = (STATS && x0 + tid < xe) ? cert.qb[x0 + tid] : 0.0;

    const int nchunks = d / KC;
    const int64_t bstride = (int64_t)ld * 32;          // words per 32-row block
    const float* Xw = X + (((x0 - xb) >> 5) + wave) * bstride;  // this wave's X block (X starts at row xb)
    const unsigned lane16 = (unsigned)lane * 16u;
    const unsigned t16 = (unsigned)(tid & 255) * 16u;
    const unsigned bstep = (unsigned)(bstride * 4);     // bytes between consecutive 32-row blocks
    const int bsel = tid >> 8;                          // Y blocks 0 and 2 (waves 0-3) or 1 and 3 (waves 4-7)

    auto load_x = [&](XOps& o, int cc) {
        const float* b = Xw + cc * 1024;
        o.h0 = ld16(b, lane16);
        o.l0 = ld16(b, 1024u + lane16);
        o.h1 = ld16(b, 2048u + lane16);
        o.l1 = ld16(b, 3072u + lane16);
    };
    // Y chunk AHEAD chunks past the one multiplied (ta, ca); past the segment any in-bounds chunk will do, its
    // data is never multiplied. Thread t's 16 bytes of block 2i + bsel go to stage + (2i + bsel)*4 KiB +
    // (t % 256)*16: one wave instruction fills 1 KiB.
    int64_t ta = y_begin;
    int ca = 0;
    auto load_ahead = [&](float4* stage) {
        const bool past = ta >= y_end;
        const char* b = reinterpret_cast<const char*>(Y + ((past ? y_begin : ta) >> 5) * bstride + (past ? 0 : ca) * 1024);
        float4* dst = stage + bsel * 256 + (wave & 3) * 64;
#pragma unroll
        for (int i = 0; i < 2; ++i)
            __builtin_amdgcn_global_load_lds(b + (2 * i + bsel) * bstep + t16,
                                             (__attribute__((address_space(3))) void*)(dst + i * 512), 16, 0, 0);
        ++ca;
        const bool wrap = ca == nchunks;
        ca = wrap ? 0 : ca;
        ta = wrap ? ta + BY : ta;
    };
    // half p (0: hi, 1: lo) of the operands of K-step ks of the Y chunk in `stage`
    auto read_half = [&](YHalf& o, const float4* stage, int ks, int p) {
        const float4* src = stage + ks * 128 + p * 64 + lane;
        o.b0 = src[0];
        o.b1 = src[256];
        o.b2 = src[512];
        o.b3 = src[768];
    };

    XOps xs0, xs1;  // X operands: chunk c in set c % 2
    YHalf yh, yl;   // Y operands of the pass in flight (hi and lo halves of one K-step)
    load_ahead(sY0);
    load_ahead(sY1);
    load_ahead(sY2);
    load_x(xs0, 0);
    wait_vmcnt<0>();
    __syncthreads();

    v16f acc[NB];
    float outer[NB][16];
#pragma unroll
    for (int y = 0; y < NB; ++y) {
#pragma unroll
        for (int q = 0; q < 16; ++q) { acc[y][q] = 0.0f; outer[y][q] = 0.0f; }
    }

    // chunk c (U = c % 4: Y stage U, X set U % 2, restarting accumulator block U)
    auto step = [&](auto uc, int c) {
        constexpr int U = decltype(uc)::value;
        XOps& xs = xset2<U>(xs0, xs1);
        float4* cur = xset_stage<U>(sY0, sY1, sY2, sY3);
        float4* fill = xset_stage<(U + 3) % 4>(sY0, sY1, sY2, sY3);
        // the next chunk's X into the other set (last used by chunk c - 1)
        load_x(xset2<U + 1>(xs0, xs1), c + 1 == nchunks ? 0 : c + 1);
        // K-step 0 (block U restarts), then K-step 1's operands, all read before the barrier
        read_half(yh, cur, 0, 0);
        read_half(yl, cur, 0, 1);
        split_pass<U, true>(acc, outer, yh, xs.h0);
        split_pass<U, false>(acc, outer, yh, xs.l0);
        __builtin_amdgcn_sched_barrier(0);
        read_half(yh, cur, 1, 0);
        split_pass<U, false>(acc, outer, yl, xs.h0);
        __builtin_amdgcn_sched_barrier(0);
        read_half(yl, cur, 1, 1);
        // the Y chunk AHEAD further into the stage chunk - 1 used (all its reads retired at the previous barrier);
        // this wave's loads of the next chunk's Y were issued AHEAD - 1 chunks back, so at most the later chunks'
        // instructions may still be in flight at the barrier
        load_ahead(fill);
        ring_barrier<(AHEAD - 1) * VMEM_STEP>();
        split_pass<-1, false>(acc, outer, yh, xs.h1);
        split_pass<-1, false>(acc, outer, yh, xs.l1);
        split_pass<-1, false>(acc, outer, yl, xs.h1);
        __builtin_amdgcn_sched_barrier(0);
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;

    for (int64_t ytile = y_begin; ytile < y_end; ytile += BY) {
        // biases of this tile's Y rows (read in the epilogue, after at least one chunk barrier)
        if (tid < BY) {
            const int64_t j = ytile + tid;
            sDB[tid] = j < y_end ? db32[j] : 0.0f;
            sGE[tid] = (STATS && j < y_end) ? ge32[j] : 0.0f;
            if (!APPEND) sDB64[tid] = (STATS && j < y_end) ? cert.db[j] : 0.0;
        }
        for (int c = 0; c < nchunks; c += 4) {
            step(I0{}, c);
            step(I1{}, c + 1);
            step(I2{}, c + 2);
            step(I3{}, c + 3);
        }
        // the blocks' last parts into the outer sums; the accumulators restart from zero for the next tile
#pragma unroll
        for (int y = 0; y < NB; ++y) {
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                outer[y][q] += acc[y][q];
                acc[y][q] = 0.0f;
            }
        }
        sweep_epilogue_w<K1, COLS, APPEND, ST>(outer, row, ok, qbi, pi, wt, ytile == y_begin, tid, wave, h, r, ytile,
                                           y_end, x0, xb, rows, seg, panel, n, scale, STATS, slack, sQB64, sDB64, sDB,
                                           sGE, sC,
                                           part,
                                           colpart, colthr, wcnt, wbuf, wcap, num64, den64, cnt, cmax, rowthr);
#pragma unroll
        for (int y = 0; y < NB; ++y) {
#pragma unroll
            for (int q = 0; q < 16; ++q) outer[y][q] = 0.0f;
        }
    }
    wait_vmcnt<0>();  // the loads ahead into LDS land before the workgroup can end
    if (STATS) {
        // the maximum violation (slot 3) is taken exactly from the fp64 row lists after the sweep
        double v[5] = {num64, den64, (double)cnt, 0.0, (double)cmax};
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
                for (int w = 1; w < WAVES_W; ++w) o[e] = (e >= 3) ? fmax(o[e], sRed[w][e]) : o[e] + sRed[w][e];
            }
            double* dst = blockstats + (seg * P + panel) * 5;
            for (int e = 0; e < 5; ++e) dst[e] = o[e];
        }
    }
}

// int8 sweep over 256-row X panels (HM_INT8X3): the panels, Y ring, X operand sets and epilogue of
// l2sq_sweep_split_w on the int8 copies (64 features per 4 KiB chunk) and v_mfma_i32_32x32x32_i8. Per K-step of
// 32 features: A[y] += Yh*Xh, B[y] += Yh*Xl, B[y] += Yl*Xh, exact in int32 (|A|, |B| <= 32512 d < 2^31 for
// d <= 65536), so the dot needs no blocking: after the tile's last chunk t = ((65536 A + 256 B) s_y) s_x in fp32.
__device__ __forceinline__ void i8_pass(v16i (&acc)[NB], const YHalf& yp, const float4& x4) {
    const v4i xv = __builtin_bit_cast(v4i, x4);
    acc[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(v4i, yp.b0), xv, acc[0], 0, 0, 0);
    acc[1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(v4i, yp.b1), xv, acc[1], 0, 0, 0);
    acc[2] = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(v4i, yp.b2), xv, acc[2], 0, 0, 0);
    acc[3] = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(v4i, yp.b3), xv, acc[3], 0, 0, 0);
}

template <int K1, bool COLS, bool APPEND = false, bool ST = false>
__global__ __launch_bounds__(THREADS_W) void l2sq_sweep_i8_w(
    const float* __restrict__ X, const float* __restrict__ Y, int64_t xb, int64_t xe, int64_t n, int d, int ld,
    const float* __restrict__ qb32, const float* __restrict__ db32, const float* __restrict__ p32,
    const float* __restrict__ ge32, float scale, int64_t seg_len, int P, int S, Entry* __restrict__ part,
    Entry* __restrict__ colpart, unsigned int* __restrict__ colthr, double* __restrict__ blockstats, int STATS,
    CertArgs cert, const float* __restrict__ xqs, const float* __restrict__ yqs, const float* __restrict__ wthr = nullptr, int* __restrict__ wcnt = nullptr,
    int* __restrict__ wbuf = nullptr,
    int wcap = 0, unsigned int* __restrict__ rowthr = nullptr) {
    static_assert(!(APPEND && COLS), "the wide pass keeps no column lists");
    constexpr int AHEAD = 3;      // Y chunks in flight ahead of the one multiplied (4-stage ring)
    constexpr int VMEM_STEP = 6;  // vector-memory instructions a chunk issues (4 X, then 2 Y)
    int64_t panel, seg;
    sweep_block(blockIdx.x, P, S, panel, seg);
    if (panel >= P || seg >= S) return;  // grid padding (uniform per workgroup, before any barrier)
    __shared__ float4 sY0[1024], sY1[1024], sY2[1024], sY3[1024];  // LDS ring (Y chunk: 4 blocks x 4 KiB)
    __shared__ double sQB64[STATS_LDS(BXW)], sDB64[STATS_LDS(BY)];  // fp64 biases for the certificate's near pairs
    __shared__ float sDB[BY];
    __shared__ float sGE[BY];
    __shared__ float sC[COLS ? CROWS_W * CSTW : 1];
    __shared__ double sRed[WAVES_W][5];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5;
    const int r = lane & 31;
    const int64_t rows = xe - xb;
    const int64_t x0 = xb + panel * BXW;
    const int64_t y_begin = seg * seg_len;
    const int64_t y_end = (y_begin + seg_len < n) ? (y_begin + seg_len) : n;
    const int64_t row = x0 + wave * 32 + r;
    const bool ok = row < xe;
    const float qbi = (ok && !APPEND) ? qb32[row] : 0.0f;
    const float pi = (STATS && ok) ? p32[row] : 0.0f;
    const float wt = (APPEND && ok) ? wthr[row] : INFINITY;
    double num64 = 0.0, den64 = 0.0;
    unsigned int cnt = 0u;
    float cmax = 0.0f;
    const float slack = row_cert_slack(STATS, cert, row, ok, scale);
    const float sx = ok ? xqs[row] : 0.0f;
    if (!APPEND && tid < BXW) sQB64[tid] = (STATS && x0 + tid < xe) ? cert.qb[x0 + tid] : 0.0;

    const int nchunks = d / KC;
    const int64_t bstride = (int64_t)ld * 32;          // words per 32-row block
    const float* Xw = X + (((x0 - xb) >> 5) + wave) * bstride;  // this wave's X block (X starts at row xb)
    const unsigned lane16 = (unsigned)lane * 16u;
    const unsigned t16 = (unsigned)(tid & 255) * 16u;
    const unsigned bstep = (unsigned)(bstride * 4);     // bytes between consecutive 32-row blocks
    const int bsel = tid >> 8;                          // Y blocks 0 and 2 (waves 0-3) or 1 and 3 (waves 4-7)

    auto load_x = [&](XOps& o, int cc) {
        const float* b = Xw + cc * 1024;
        o.h0 = ld16(b, lane16);
        o.l0 = ld16(b, 1024u + lane16);
        o.h1 = ld16(b, 2048u + lane16);
        o.l1 = ld16(b, 3072u + lane16);
    };
    // Y chunk AHEAD chunks past the one multiplied (ta, ca); past the segment any in-bounds chunk will do, its
    // data is never multiplied. Thread t's 16 bytes of block 2i + bsel go to stage + (2i + bsel)*4 KiB +
    // (t % 256)*16: one wave instruction fills 1 KiB.
    int64_t ta = y_begin;
    int ca = 0;
    auto load_ahead = [&](float4* stage) {
        const bool past = ta >= y_end;
        const char* b = reinterpret_cast<const char*>(Y + ((past ? y_begin : ta) >> 5) * bstride + (past ? 0 : ca) * 1024);
        float4* dst = stage + bsel * 256 + (wave & 3) * 64;
#pragma unroll
        for (int i = 0; i < 2; ++i)
            __builtin_amdgcn_global_load_lds(b + (2 * i + bsel) * bstep + t16,
                                             (__attribute__((address_space(3))) void*)(dst + i * 512), 16, 0, 0);
        ++ca;
        const bool wrap = ca == nchunks;
        ca = wrap ? 0 : ca;
        ta = wrap ? ta + BY : ta;
    };
    // half p (0: hi, 1: lo) of the operands of K-step ks of the Y chunk in `stage`
    auto read_half = [&](YHalf& o, const float4* stage, int ks, int p) {
        const float4* src = stage + ks * 128 + p * 64 + lane;
        o.b0 = src[0];
        o.b1 = src[256];
        o.b2 = src[512];
        o.b3 = src[768];
    };

    XOps xs0, xs1;  // X operands: chunk c in set c % 2
    YHalf yh, yl;   // Y operands of the pass in flight (hi and lo halves of one K-step)
    load_ahead(sY0);
    load_ahead(sY1);
    load_ahead(sY2);
    load_x(xs0, 0);
    wait_vmcnt<0>();
    __syncthreads();

    v16i accA[NB], accB[NB];  // sum h_y h_x and sum (h_y l_x + l_y h_x) of the tile's dots

    // chunk c (U = c % 4: Y stage U, X set U % 2)
    auto step = [&](auto uc, int c) {
        constexpr int U = decltype(uc)::value;
        XOps& xs = xset2<U>(xs0, xs1);
        float4* cur = xset_stage<U>(sY0, sY1, sY2, sY3);
        float4* fill = xset_stage<(U + 3) % 4>(sY0, sY1, sY2, sY3);
        // the next chunk's X into the other set (last used by chunk c - 1)
        load_x(xset2<U + 1>(xs0, xs1), c + 1 == nchunks ? 0 : c + 1);
        // K-step 0, then K-step 1's operands, all read before the barrier
        read_half(yh, cur, 0, 0);
        read_half(yl, cur, 0, 1);
        i8_pass(accA, yh, xs.h0);
        i8_pass(accB, yh, xs.l0);
        __builtin_amdgcn_sched_barrier(0);
        read_half(yh, cur, 1, 0);
        i8_pass(accB, yl, xs.h0);
        __builtin_amdgcn_sched_barrier(0);
        read_half(yl, cur, 1, 1);
        // the Y chunk AHEAD further into the stage chunk - 1 used (all its reads retired at the previous barrier);
        // this wave's loads of the next chunk's Y were issued AHEAD - 1 chunks back, so at most the later chunks'
        // instructions may still be in flight at the barrier
        load_ahead(fill);
        ring_barrier<(AHEAD - 1) * VMEM_STEP>();
        i8_pass(accA, yh, xs.h1);
        i8_pass(accB, yh, xs.l1);
        i8_pass(accB, yl, xs.h1);
        __builtin_amdgcn_sched_barrier(0);
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;

    for (int64_t ytile = y_begin; ytile < y_end; ytile += BY) {
        // biases of this tile's Y rows (read in the epilogue, after at least one chunk barrier)
        if (tid < BY) {
            const int64_t j = ytile + tid;
            sDB[tid] = j < y_end ? db32[j] : 0.0f;
            sGE[tid] = (STATS && j < y_end) ? ge32[j] : 0.0f;
            if (!APPEND) sDB64[tid] = (STATS && j < y_end) ? cert.db[j] : 0.0;
        }
        // the accumulators start from zero here rather than after the previous epilogue, so that they are dead
        // (their registers free) while the epilogue runs
#pragma unroll
        for (int y = 0; y < NB; ++y) {
#pragma unroll
            for (int q = 0; q < 16; ++q) { accA[y][q] = 0; accB[y][q] = 0; }
        }
        for (int c = 0; c < nchunks; c += 4) {
            step(I0{}, c);
            step(I1{}, c + 1);
            step(I2{}, c + 2);
            step(I3{}, c + 3);
        }
        // fp32 dots t = ((65536 A + 256 B) s_y) s_x, with s_y the scale of Y block y (uniform over the wave)
        float outer[NB][16];
#pragma unroll
        for (int y = 0; y < NB; ++y) {
            const float sy = ytile + 32 * y < n ? yqs[ytile + 32 * y] : 0.0f;
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const float u = fmaf(65536.0f, (float)accA[y][q], 256.0f * (float)accB[y][q]);
                outer[y][q] = (u * sy) * sx;
            }
        }
        sweep_epilogue_w<K1, COLS, APPEND, ST>(outer, row, ok, qbi, pi, wt, ytile == y_begin, tid, wave, h, r, ytile,
                                           y_end, x0, xb, rows, seg, panel, n, scale, STATS, slack, sQB64, sDB64, sDB,
                                           sGE, sC,
                                           part,
                                           colpart, colthr, wcnt, wbuf, wcap, num64, den64, cnt, cmax, rowthr);
    }
    wait_vmcnt<0>();  // the loads ahead into LDS land before the workgroup can end
    if (STATS) {
        // the maximum violation (slot 3) is taken exactly from the fp64 row lists after the sweep
        double v[5] = {num64, den64, (double)cnt, 0.0, (double)cmax};
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
                for (int w = 1; w < WAVES_W; ++w) o[e] = (e >= 3) ? fmax(o[e], sRed[w][e]) : o[e] + sRed[w][e];
            }
            double* dst = blockstats + (seg * P + panel) * 5;
            for (int e = 0; e < 5; ++e) dst[e] = o[e];
        }
    }
}

// deterministic reduction of per-block certificate partials (single block); later chunks accumulate
__global__ void l2sq_reduce_stats(const double* __restrict__ blockstats, int64_t blocks, double* __restrict__ stats,
                                  int linf, int accumulate) {
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
        double o[5] = {s[0][0], s[0][1], s[0][2], s[0][3], linf ? s[0][4] : 0.0};
        if (accumulate) {
            o[0] += stats[0];
            o[1] += stats[1];
            o[2] += stats[2];
            o[3] = fmax(o[3], stats[3]);
            o[4] = fmax(o[4], stats[4]);
        }
        // stats[3] is replaced by the exact row maximum when rows are computed
        for (int e = 0; e < 5; ++e) stats[e] = o[e];
    }
}

// -------------------------------------------------------------------------------------------------
// finalize: one wave per row (rows of a chunk, or Y rows for the column lists)
// -------------------------------------------------------------------------------------------------
struct BoundArgs {
    double acc_rel;   // relative bound on |dot32 - dot| in units of ||x||*||y||, plus fp64 slack
    double db_rel;    // relative bound contribution of fp32 bias rounding, in units of max|bias|
    double abs_slack; // absolute slack (flushed denormals)
    // int8 sweep: the finalized side's per-row error terms (alpha, beta, gamma, rho; l2sq_split_i8) and the
    // candidate side's maxima of them; null otherwise
    const double* qterm = nullptr;
    const unsigned long long* qmax = nullptr;
};

// Rigorous bound b on |w - (sigma - abias[row])| for every candidate of row `row`: w is the sweep's fp32 score of the
// pair (ranking without the row's own bias), sigma its exact fp64 score.
__device__ __forceinline__ double row_bound(int64_t row, const double* __restrict__ anorm,
                                            const double* __restrict__ abias,
                                            const unsigned long long* __restrict__ bmaxima, double scale,
                                            const BoundArgs& bnd) {
    const double bmax = key_double(bmaxima[0]);
    const double dmax = key_double(bmaxima[1]);
    const double nxy = scale * anorm[row] * bmax;
    double b = (nxy * bnd.acc_rel + dmax * bnd.db_rel + fabs(abias[row]) * 1e-15 + bnd.abs_slack) * (1.0 + 1e-6);
    if (bnd.qterm) {
        // quantization, dropped limb product and conversion terms of the int8 sweep (l2sq_split_i8)
        const double* qt = bnd.qterm + row * 4;
        const double ma = key_double(bnd.qmax[0]), mb = key_double(bnd.qmax[1]);
        const double mg = key_double(bnd.qmax[2]), mr = key_double(bnd.qmax[3]);
        b += scale * (qt[0] * mb + qt[1] * ma + qt[2] * mg + 5.0 * 0x1p-24 * qt[3] * mr) * (1.0 + 1e-6);
    }
    return b;
}

// A row's floor in the scale of its list values: an entry's exact score is sigma = w + abias to within b, so an
// entry with w < floor_cut scores below the floor (the last term covers the rounding of the cut itself). -inf for
// a floor of -inf.
__device__ __forceinline__ double floor_cut(double floor, double abias, double b) {
    const double fa = floor - abias;
    return (fa - b) - 1e-15 * fabs(fa);
}

// Shared row thresholds of a sweep (row_threshold_*, or the fused sweep's column thresholds) seeded from the
// caller's floors: the largest fp32 value strictly below the row's floor_cut, so that the sweep drops only scores
// whose pairs score below the floor (float_key(-inf) without a floor).
__global__ void seed_floor_thresholds(unsigned int* __restrict__ thr, int64_t rows, const double* __restrict__ floor,
                                      const double* __restrict__ anorm, const double* __restrict__ abias,
                                      const unsigned long long* __restrict__ bmaxima, double scale, BoundArgs bnd) {
    for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < rows; r += (int64_t)gridDim.x * blockDim.x) {
        const double c = floor_cut(floor[r], abias[r], row_bound(r, anorm, abias, bmaxima, scale, bnd));
        float c32 = -INFINITY;
        if (c > -INFINITY) {
            c32 = (float)c;
            if (!((double)c32 < c)) c32 = nextafterf(c32, -INFINITY);
        }
        if (c32 != c32) c32 = -INFINITY;  // a NaN floor seeds nothing
        thr[r] = float_key(c32);
    }
}

// Lists of row r: L in [0, nlists), each of KL entries at base + (((L / G) * R + r) * G + L % G) * KL (sorted,
// missing = -1). One wave per row merges them into the best KM (KM >= KL).
// The row side A (rows A[r], row bias abias[r], norm anorm[r]) pairs with candidates from side B (B[c],
// bias bbias[c]); sigma = COLS ? (s*dot + bbias[c]) + abias[r] : (s*dot + abias[r]) + bbias[c], which keeps
// the (dot + qb) + db association of the caller's (x, y) pair in both directions.
// N dot64 products of the row `a` with rows c[0..N) of B in one pass over the features: the same order as
// wave_dot64 for each (lane l sums features l, l + 64, ... in order, then the halving-stride tree)
template <int N>
__device__ __forceinline__ void multi_dot64(const float* __restrict__ a, const float* __restrict__ B, const int (&c)[4],
                                            int d, int lane, double (&dots)[4]) {
    const float* b[N];
#pragma unroll
    for (int t = 0; t < N; ++t) b[t] = B + (int64_t)c[t] * d;
    double acc[N];
#pragma unroll
    for (int t = 0; t < N; ++t) acc[t] = 0.0;
    // eight strides of loads in flight per pass (the sums still take each lane's features in order)
    constexpr int U = 8;
    int f = lane;
    for (; f + 64 * (U - 1) < d; f += 64 * U) {
        float xa[U], xb[U][N];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            xa[u] = a[f + 64 * u];
#pragma unroll
            for (int t = 0; t < N; ++t) xb[u][t] = b[t][f + 64 * u];
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int t = 0; t < N; ++t) acc[t] = acc[t] + (double)xa[u] * (double)xb[u][t];
    }
    for (; f < d; f += 64) {
        const double xa = (double)a[f];
#pragma unroll
        for (int t = 0; t < N; ++t) acc[t] = acc[t] + xa * (double)b[t][f];
    }
#pragma unroll
    for (int t = 0; t < N; ++t) dots[t] = wave_tree_sum(acc[t]);
}

// Exact evaluation of a row's `need` first candidates c_list[0..need) (lane e owns candidate e; `need` is uniform over
// the wave): fixed-order fp64 dots, up to four per pass over the row's features, then the row's exact top k under the
// tie rule into out_val / out_idx (missing slots -inf / -1).
template <int KM, bool COLS>
__device__ __forceinline__ void exact_topk_write(const float* __restrict__ ar, const float* __restrict__ B, int d,
                                                 int lane, int need, const int (&c_list)[KM], double ab,
                                                 const double* __restrict__ bbias, double scale, int k,
                                                 double* __restrict__ out_val, int* __restrict__ out_idx) {
    double sv = -INFINITY;
    int sj = -1;
    for (int e0 = 0; e0 < need;) {
        const int nb = need - e0 >= 4 ? 4 : (need - e0 >= 2 ? 2 : 1);
        int c[4] = {-1, -1, -1, -1};
#pragma unroll
        for (int e = 0; e < KM; ++e) {
#pragma unroll
            for (int t = 0; t < 4; ++t)
                if (e == e0 + t && t < nb) c[t] = c_list[e];
        }
        double dots[4];
        if (nb == 4) multi_dot64<4>(ar, B, c, d, lane, dots);
        else if (nb == 2) multi_dot64<2>(ar, B, c, d, lane, dots);
        else multi_dot64<1>(ar, B, c, d, lane, dots);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            if (t < nb) {
                const double sdot = scale * dots[t];
                const double sig = COLS ? (sdot + bbias[c[t]]) + ab : (sdot + ab) + bbias[c[t]];
                if (lane == e0 + t) { sv = sig; sj = c[t]; }
            }
        }
        e0 += nb;
    }
    int er = 0;
    for (int src = 0; src < need; ++src) {
        const double v2 = __shfl(sv, src, 64);
        const int j2 = __shfl(sj, src, 64);
        if (lane < need && src != lane && better(v2, j2, sv, sj)) ++er;
    }
    if (lane < need && er < k) {
        out_val[er] = sv;
        out_idx[er] = sj;
    }
    if (lane >= need && lane < k) {
        out_val[lane] = -INFINITY;
        out_idx[lane] = -1;
    }
}

// Deferred exact evaluation (the fused column finalize): the selection kernel stores each row's candidates and
// `need`, and the rows are evaluated later in an order that groups rows by their first candidate, so that the
// candidate side's rows are re-read from cache rather than memory.
struct DeferBufs {
    int* key = nullptr;   // [R] first candidate (a row of B), -1 when the row has nothing to evaluate
    int* need = nullptr;  // [R]
    int* cand = nullptr;  // [R * KM]
};

// Rows of a finalize call that its partial lists resolve (queued with the count at redo_count[1]); without
// `rows` every queued row goes to the sweep queue.
struct ListQueue {
    int* rows = nullptr;
    float* thr = nullptr;
};

// floor (optional, per row of A): the caller already holds k entries of the row scoring at least floor[row], so
// entries whose exact score is below it may be left out of the row's output (they cannot enter the caller's merged
// top k). With a floor the output holds the row's exact top k among the entries that can reach it, and fewer
// (padded with -inf / -1) when fewer can.
template <int KL, int KM, int G, bool COLS, bool DEFER = false>
__global__ __launch_bounds__(256) void l2sq_finalize(
    const float* __restrict__ A, const float* __restrict__ B, int64_t R, int d, int nlists,
    const Entry* __restrict__ lists, const double* __restrict__ abias, const double* __restrict__ bbias,
    const double* __restrict__ anorm, const unsigned long long* __restrict__ bmaxima, double scale, int k,
    BoundArgs bnd, double* __restrict__ out_val, int* __restrict__ out_idx, int* __restrict__ redo,
    float* __restrict__ redo_thr, int* __restrict__ redo_count, DeferBufs defer = DeferBufs{},
    ListQueue lq = ListQueue{}, const double* __restrict__ floor = nullptr) {
    static_assert(KL <= KM, "merged lists hold at least one partial list");
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const bool valid = row < R;   // uniform per wave
    float lw[KM];
    int li[KM];
#pragma unroll
    for (int s = 0; s < KM; ++s) { lw[s] = -INFINITY; li[s] = -1; }
    int nreal = 0, full = 0;
    float tail = -INFINITY;  // largest last entry of a full list: everything its sweep dropped is <= it
    if (valid) {
        static_assert(KL % 2 == 0, "lists are read two entries per 16-byte load");
        for (int L = lane; L < nlists; L += 64) {
            // a list is KL entries, filled from the front (missing entries j = -1), 16-byte aligned: it is read
            // eight entries per group of four independent loads
            const int4* src = reinterpret_cast<const int4*>(lists +
                                                            ((((int64_t)(L / G)) * R + row) * G + (L % G)) * KL);
            int cnt = 0;
            bool open = true;
            float last = -INFINITY;
            for (int g = 0; g < KL / 2 && open; g += 4) {
                int4 q[4];
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (g + u < KL / 2) q[u] = src[g + u];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    if (g + u < KL / 2) {
#pragma unroll
                        for (int h = 0; h < 2; ++h) {
                            const float w = __int_as_float(h ? q[u].z : q[u].x);
                            const int j = h ? q[u].w : q[u].y;
                            open = open && j >= 0;
                            if (open) {
                                ++cnt;
                                last = w;
                                if (better_e(w, j, lw[KM - 1], li[KM - 1])) insert_e<KM>(lw, li, w, j);
                            }
                        }
                    }
                }
            }
            nreal += cnt;
            if (cnt == KL) {
                full = 1;
                tail = fmaxf(tail, last);
            }
        }
    }
    for (int o = 32; o >= 1; o >>= 1) {
        nreal += __shfl_xor(nreal, o, 64);
        full |= __shfl_xor(full, o, 64);
        tail = fmaxf(tail, __shfl_xor(tail, o, 64));
    }
    if (!valid) return;  // uniform per wave; nothing below synchronises across waves
    const int kept = nreal < KM ? nreal : KM;
    const double b = row_bound(row, anorm, abias, bmaxima, scale, bnd);
    const double fcut = floor ? floor_cut(floor[row], abias[row], b) : -INFINITY;
    // wave top-KM: rounds of an arg-best over the lanes' list heads (tw non-increasing). The rounds stop after the
    // first entry t >= k - 1 below wk - 2b, at the first entry below fcut (or after the last real entry): no later
    // entry is evaluated, and one that the merge drops then has w <= tw[t] < max(wk - 2b, fcut), so every decision
    // below is what all KM rounds give.
    float tw[KM];
    int ti[KM];
#pragma unroll
    for (int t = 0; t < KM; ++t) { tw[t] = -INFINITY; ti[t] = -1; }
    float wk = -INFINITY;
    bool more = true;  // uniform per wave: every lane holds the same round results
#pragma unroll
    for (int t = 0; t < KM; ++t) {
        if (more) {
            float bw = lw[0];
            int bi = li[0];
            int bl = lane;
            for (int o = 32; o >= 1; o >>= 1) {
                const float ow = __shfl_xor(bw, o, 64);
                const int oi = __shfl_xor(bi, o, 64);
                const int ol = __shfl_xor(bl, o, 64);
                if (better_e(ow, oi, bw, bi)) { bw = ow; bi = oi; bl = ol; }
            }
            tw[t] = bw;
            ti[t] = bi;
            if (lane == bl) {
#pragma unroll
                for (int s = 0; s + 1 < KM; ++s) { lw[s] = lw[s + 1]; li[s] = li[s + 1]; }
                lw[KM - 1] = -INFINITY;
                li[KM - 1] = -1;
            }
            if (t == k - 1) wk = nreal < k ? -INFINITY : bw;
            if ((t + 1 >= k && (t + 1 >= kept || (double)bw < (double)wk - 2.0 * b)) || (double)bw < fcut)
                more = false;
        }
    }
    // Candidates outside the kept list were dropped by a full partial list (w <= tail) or by the merge
    // (w <= tw[KM-1]); they cannot reach the exact top-k when that bound is below wk - 2b, nor the output when it
    // is below fcut.
    const double cut = fmax((double)wk - 2.0 * b, fcut);
    const bool merge_dropped = nreal > KM;
    const bool list_hit = full && (double)tail >= cut;
    const bool merge_hit = merge_dropped && (double)tw[KM - 1] >= cut;
    if (list_hit || merge_hit) {
        // queued for the wide pass: a candidate of the exact top-k has sigma >= sigma_k* >= wk - b, hence
        // w >= wk - 2b (the threshold is rounded down to fp32). Unless a full list's tail reaches that bound, the
        // lists hold every such candidate (a full list dropped, and the shared thresholds skipped, only scores
        // <= tail): the row is then resolved from its lists (queue 1) rather than by a new sweep (queue 0).
        if constexpr (DEFER) {
            if (lane == 0) defer.key[row] = -1;  // nothing to evaluate later
        }
        if (lane == 0) {
            const bool from_lists = !list_hit && lq.rows != nullptr;
            const int slot = atomicAdd(redo_count + (from_lists ? 1 : 0), 1);
            const double t = cut;
            float t32 = (float)t;
            if ((double)t32 > t) t32 = nextafterf(t32, -INFINITY);
            if (from_lists) {
                lq.rows[slot] = (int)row;
                lq.thr[slot] = t32;
            } else {
                redo[slot] = (int)row;
                redo_thr[slot] = t32;
            }
        }
        return;
    }
    // Exact re-evaluation of the kept entries that can reach the exact top-k: an entry with w < wk - 2b has an
    // exact score below wk - b, under each of the k entries with w >= wk, so only the sorted prefix with
    // w >= cut is evaluated (without a floor for the row always at least the first min(k, kept)). Lane e owns
    // entry e.
    int need = 0;
#pragma unroll
    for (int e = 0; e < KM; ++e)
        if (e < kept && (double)tw[e] >= cut) need = e + 1;
    if (fcut == -INFINITY && need < (kept < k ? kept : k)) need = kept < k ? kept : k;
    if constexpr (DEFER) {
        if (lane == 0) {
            defer.need[row] = need;
            defer.key[row] = need > 0 ? ti[0] : -1;
#pragma unroll
            for (int e = 0; e < KM; ++e)
                if (e < need) defer.cand[row * KM + e] = ti[e];
        }
        if (need == 0 && lane < k) {
            out_val[row * k + lane] = -INFINITY;
            out_idx[row * k + lane] = -1;
        }
        return;
    }
    exact_topk_write<KM, COLS>(A + row * (int64_t)d, B, d, lane, need, ti, abias[row], bbias, scale, k,
                               out_val + row * k, out_idx + row * k);
}

// Deferred finalize, step 2: rows bucketed by their first candidate (a counting sort; the order within a bucket is
// whatever the atomics give, which changes no result).
// (keys outside [base, base + nb) cannot occur: every stored key is a candidate of this chunk; the test keeps the
// counts in bounds regardless)
__global__ void defer_count(const int* __restrict__ key, int64_t R, int base, int nb, int* __restrict__ count) {
    for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < R; r += (int64_t)gridDim.x * blockDim.x) {
        const int b = key[r] - base;
        if (key[r] >= 0 && b >= 0 && b < nb) atomicAdd(&count[b], 1);
    }
}

// exclusive prefix sum of count[0..nb) into offset[0..nb] (one workgroup of 1024 threads)
__global__ __launch_bounds__(1024) void defer_scan(const int* __restrict__ count, int nb, int* __restrict__ offset,
                                                   int* __restrict__ total) {
    __shared__ int part[1024];
    const int t = threadIdx.x;
    const int per = (nb + 1023) / 1024;
    int s = 0;
    for (int i = t * per; i < nb && i < (t + 1) * per; ++i) s += count[i];
    part[t] = s;
    __syncthreads();
    for (int o = 1; o < 1024; o <<= 1) {
        const int v = t >= o ? part[t - o] : 0;
        __syncthreads();
        part[t] += v;
        __syncthreads();
    }
    int run = t > 0 ? part[t - 1] : 0;
    for (int i = t * per; i < nb && i < (t + 1) * per; ++i) {
        offset[i] = run;
        run += count[i];
    }
    if (t == 1023) {
        offset[nb] = part[1023];
        *total = part[1023];
    }
}

__global__ void defer_scatter(const int* __restrict__ key, int64_t R, int base, int nb, int* __restrict__ offset,
                              int* __restrict__ order) {
    for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < R; r += (int64_t)gridDim.x * blockDim.x) {
        const int b = key[r] - base;
        if (key[r] >= 0 && b >= 0 && b < nb) order[atomicAdd(&offset[b], 1)] = (int)r;
    }
}

// Deferred finalize, step 3: one wave per bucketed row, the exact evaluation of its stored candidates. `total`
// (the number of bucketed rows) is read from the device.
template <int KM, bool COLS>
__global__ __launch_bounds__(256) void l2sq_finalize_exact(const float* __restrict__ A, const float* __restrict__ B,
                                                           int d, const int* __restrict__ order,
                                                           const int* __restrict__ total, DeferBufs defer,
                                                           const double* __restrict__ abias,
                                                           const double* __restrict__ bbias, double scale, int k,
                                                           double* __restrict__ out_val, int* __restrict__ out_idx) {
    const int lane = threadIdx.x & 63;
    const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (w >= *total) return;  // uniform per wave
    const int64_t row = order[w];
    const int need = defer.need[row];
    int c_list[KM];
#pragma unroll
    for (int e = 0; e < KM; ++e) c_list[e] = e < need ? defer.cand[row * KM + e] : -1;
    exact_topk_write<KM, COLS>(A + row * (int64_t)d, B, d, lane, need, c_list, abias[row], bbias, scale, k,
                               out_val + row * k, out_idx + row * k);
}

// Sliced exact rescan: item (queued row, candidate slice) is one wave. Candidates are evaluated four at a time
// (four independent accumulators share each load of the row's features); every candidate's dot keeps the dot64
// order (lane l sums features l, l+64, ... in order, then the halving-stride tree), so all lanes hold the same
// exact list. Lists go to pv / pi per item.
template <int K>
__global__ __launch_bounds__(256) void l2sq_rescan_slices(const float* __restrict__ A, const float* __restrict__ B,
                                                          int64_t nb, int d, const double* __restrict__ abias,
                                                          const double* __restrict__ bbias, double scale, int k,
                                                          const int* __restrict__ redo, int r0, int nrows, int slices,
                                                          int64_t per, int COLS, int cbase, double* __restrict__ pv,
                                                          int* __restrict__ pi) {
    const int lane = threadIdx.x & 63;
    const int64_t items = (int64_t)nrows * slices;
    for (int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); item < items; item += (int64_t)gridDim.x * 4) {
        const int64_t row = redo[r0 + item / slices];
        const int64_t j0 = (item % slices) * per;
        const int64_t j1 = j0 + per < nb ? j0 + per : nb;
        const float* ar = A + row * (int64_t)d;
        double v[K];
        int id[K];
#pragma unroll
        for (int s = 0; s < K; ++s) { v[s] = -INFINITY; id[s] = -1; }
        for (int64_t j = j0; j < j1; j += 4) {
            const float* b0 = B + j * d;
            const bool ok1 = j + 1 < j1, ok2 = j + 2 < j1, ok3 = j + 3 < j1;
            const float* b1 = ok1 ? b0 + d : b0;
            const float* b2 = ok2 ? b0 + 2 * (int64_t)d : b0;
            const float* b3 = ok3 ? b0 + 3 * (int64_t)d : b0;
            double a0 = 0.0, a1 = 0.0, a2 = 0.0, a3 = 0.0;
#pragma unroll 4
            for (int f = lane; f < d; f += 64) {
                const double x = (double)ar[f];
                a0 = a0 + x * (double)b0[f];
                a1 = a1 + x * (double)b1[f];
                a2 = a2 + x * (double)b2[f];
                a3 = a3 + x * (double)b3[f];
            }
            const double dots[4] = {wave_tree_sum(a0), wave_tree_sum(a1), wave_tree_sum(a2), wave_tree_sum(a3)};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                if (j + t < j1) {
                    const double sdot = scale * dots[t];
                    const double sig = COLS ? (sdot + bbias[j + t]) + abias[row] : (sdot + abias[row]) + bbias[j + t];
                    if (sig == sig) put_sorted<K>(v, id, k, sig, (int)(cbase + j + t));
                }
            }
        }
        if (lane == 0) {
            for (int s = 0; s < k; ++s) {
                double ov = -INFINITY;
                int oi = -1;
#pragma unroll
                for (int t = 0; t < K; ++t)
                    if (t == s) { ov = v[t]; oi = id[t]; }
                pv[item * k + s] = ov;
                pi[item * k + s] = oi;
            }
        }
    }
}

template <int K>
__global__ void l2sq_rescan_merge(const double* __restrict__ pv, const int* __restrict__ pi, int nrows, int slices,
                                  int k, const int* __restrict__ redo, int r0, double* __restrict__ out_val,
                                  int* __restrict__ out_idx) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nrows) return;
    double v[K];
    int id[K];
#pragma unroll
    for (int s = 0; s < K; ++s) { v[s] = -INFINITY; id[s] = -1; }
    for (int sl = 0; sl < slices; ++sl) {
        const int64_t base = ((int64_t)t * slices + sl) * k;
        for (int s = 0; s < k; ++s)
            if (pi[base + s] >= 0) put_sorted<K>(v, id, k, pv[base + s], pi[base + s]);
    }
    const int64_t row = redo[r0 + t];
#pragma unroll
    for (int s = 0; s < K; ++s)
        if (s < k) { out_val[row * k + s] = v[s]; out_idx[row * k + s] = id[s]; }
}

// Wide pass, step 1: queued rows q0 .. q0+Q-1 of the row side's sweep copy gathered into a compact panel-padded
// buffer (zero rows past Q), with their thresholds and cleared candidate counters.
__global__ void l2sq_wide_gather(const float* __restrict__ src, int ld, const int* __restrict__ redo, int q0, int Q,
                                 int Qpad, const float* __restrict__ redo_thr, float* __restrict__ dst,
                                 float* __restrict__ thr, int* __restrict__ cnt) {
    const int64_t total = (int64_t)Qpad * ld;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t q = e / ld;
        const int64_t f = e % ld;
        dst[e] = q < Q ? src[(int64_t)redo[q0 + q] * ld + f] : 0.0f;
    }
    for (int q = blockIdx.x * blockDim.x + threadIdx.x; q < Qpad; q += gridDim.x * blockDim.x) {
        thr[q] = q < Q ? redo_thr[q0 + q] : INFINITY;
        cnt[q] = 0;
    }
}

// The same for split copies (operand order, split-bf16 or int8): item (destination 32-row block, chunk, 16-byte unit
// of the row's eight, row within the block); consecutive threads write consecutive units. With `qsrc` (int8) the
// rows' scales are gathered too.
__global__ void l2sq_wide_gather_split(const float* __restrict__ src, int ld, int sd, const int* __restrict__ redo,
                                       int q0, int Q, int Qpad, const float* __restrict__ redo_thr,
                                       float* __restrict__ dst, float* __restrict__ thr, int* __restrict__ cnt,
                                       const float* __restrict__ qsrc, float* __restrict__ qdst) {
    const int nch = sd / KC;
    const int64_t total = (int64_t)Qpad * nch * 8;
    const uint4* s4 = reinterpret_cast<const uint4*>(src);
    uint4* d4 = reinterpret_cast<uint4*>(dst);
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
        const int rr = (int)(e & 31);
        const int j = (int)((e >> 5) & 7);  // (group g4 = 2s + h, part p) as 2 * g4 + p
        const int64_t t = e >> 8;
        const int c = (int)(t % nch);
        const int64_t q = (t / nch) * 32 + rr;
        const int g4 = j >> 1, p = j & 1;
        const int64_t du = split_unit(q, c, g4, ld) + 64 * p;
        d4[du] = q < Q ? s4[split_unit(redo[q0 + q], c, g4, ld) + 64 * p] : make_uint4(0, 0, 0, 0);
    }
    for (int q = blockIdx.x * blockDim.x + threadIdx.x; q < Qpad; q += gridDim.x * blockDim.x) {
        thr[q] = q < Q ? redo_thr[q0 + q] : INFINITY;
        cnt[q] = 0;
        if (qsrc) qdst[q] = q < Q ? qsrc[redo[q0 + q]] : 0.0f;
    }
}

// Wide pass from the partial lists (steps 1 and 2 for the rows of queue 1): queued row q0 + q is one wave; it
// collects the entries of its partial lists with w >= its threshold (a prefix of each sorted list) into
// buf[q * cap ...] as candidate ids relative to cbase, the first row of the candidate side the exact step reads.
// A count above cap sends the row to the next round (l2sq_wide_merge). The list layout is l2sq_finalize's.
template <int KL>
__global__ __launch_bounds__(256) void l2sq_list_collect(const Entry* __restrict__ lists, int64_t R, int nlists, int G,
                                                         const int* __restrict__ queue, int q0, int Q,
                                                         const float* __restrict__ queue_thr, int cbase, int cap,
                                                         float* __restrict__ thr, int* __restrict__ cnt,
                                                         int* __restrict__ buf) {
    const int lane = threadIdx.x & 63;
    for (int q = blockIdx.x * 4 + (threadIdx.x >> 6); q < Q; q += gridDim.x * 4) {  // uniform per wave
        const int64_t row = queue[q0 + q];
        const float t = queue_thr[q0 + q];
        int* dst = buf + (int64_t)q * cap;
        int pos = 0;  // entries collected so far (uniform)
        for (int L0 = 0; L0 < nlists; L0 += 64) {
            const int L = L0 + lane;
            const Entry* src = lists + ((((int64_t)(L / G)) * R + row) * G + (L % G)) * KL;
            int c = 0;
            if (L < nlists)
                while (c < KL && src[c].j >= 0 && src[c].w >= t) ++c;
            int incl = c;  // inclusive prefix sum over the lanes
            for (int o = 1; o < 64; o <<= 1) {
                const int v = __shfl_up(incl, o, 64);
                if (lane >= o) incl += v;
            }
            const int off = pos + incl - c;
            for (int e = 0; e < c; ++e)
                if (off + e < cap) dst[off + e] = src[e].j - cbase;
            pos += __shfl(incl, 63, 64);
        }
        if (lane == 0) {
            cnt[q] = pos;
            thr[q] = t;
        }
    }
}

// Wide pass, step 3: item (row q, slice of its collected candidates) is one wave; it evaluates WIDE_SLICE
// candidates with the fixed-order fp64 dot (four at a time, as the rescan) and keeps their exact top-k under the
// tie rule in pv / pi. A row whose candidates overflowed the capacity yields empty lists (it goes to the next
// round, see l2sq_wide_merge).
template <int K>
__global__ __launch_bounds__(256) void l2sq_wide_slices(const float* __restrict__ A, const float* __restrict__ B, int d,
                                                        const double* __restrict__ abias,
                                                        const double* __restrict__ bbias, double scale, int k,
                                                        const int* __restrict__ queue, int q0, int Q,
                                                        const int* __restrict__ cnt, const int* __restrict__ buf,
                                                        int cap, int spr, int COLS, int cbase, double* __restrict__ pv,
                                                        int* __restrict__ pi) {
    const int lane = threadIdx.x & 63;
    const int64_t items = (int64_t)Q * spr;
    for (int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); item < items; item += (int64_t)gridDim.x * 4) {
        const int q = (int)(item / spr);
        const int sl = (int)(item % spr);
        const int c = cnt[q];
        const int t0 = sl * WIDE_SLICE;
        const int t1 = c > cap ? t0 : (c < t0 + WIDE_SLICE ? c : t0 + WIDE_SLICE);
        const int64_t row = queue[q0 + q];
        const float* ar = A + row * (int64_t)d;
        const int* cand = buf + (int64_t)q * cap;
        double v[K];
        int id[K];
#pragma unroll
        for (int s = 0; s < K; ++s) { v[s] = -INFINITY; id[s] = -1; }
        for (int t = t0; t < t1; t += 4) {
            const int j0 = cand[t];
            const int j1 = t + 1 < t1 ? cand[t + 1] : j0;
            const int j2 = t + 2 < t1 ? cand[t + 2] : j0;
            const int j3 = t + 3 < t1 ? cand[t + 3] : j0;
            const float* b0 = B + (int64_t)j0 * d;
            const float* b1 = B + (int64_t)j1 * d;
            const float* b2 = B + (int64_t)j2 * d;
            const float* b3 = B + (int64_t)j3 * d;
            double a0 = 0.0, a1 = 0.0, a2 = 0.0, a3 = 0.0;
#pragma unroll 4
            for (int f = lane; f < d; f += 64) {
                const double x = (double)ar[f];
                a0 = a0 + x * (double)b0[f];
                a1 = a1 + x * (double)b1[f];
                a2 = a2 + x * (double)b2[f];
                a3 = a3 + x * (double)b3[f];
            }
            const double dots[4] = {wave_tree_sum(a0), wave_tree_sum(a1), wave_tree_sum(a2), wave_tree_sum(a3)};
            const int js[4] = {j0, j1, j2, j3};
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                if (t + u < t1) {
                    const int j = js[u];
                    const double sdot = scale * dots[u];
                    const double sig = COLS ? (sdot + bbias[j]) + abias[row] : (sdot + abias[row]) + bbias[j];
                    if (sig == sig) put_sorted<K>(v, id, k, sig, cbase + j);
                }
            }
        }
#pragma unroll
        for (int s = 0; s < K; ++s)
            if (s < k && lane == s) {
                pv[item * k + s] = v[s];
                pi[item * k + s] = id[s];
            }
    }
}

// Wide pass, step 4: one thread per row merges its slices' lists into the output, or passes a row whose
// candidates overflowed the capacity (and its threshold) on to the next round's queue.
template <int K>
__global__ void l2sq_wide_merge(const double* __restrict__ pv, const int* __restrict__ pi, int Q, int spr, int k,
                                const int* __restrict__ cnt, int cap, const int* __restrict__ queue,
                                const float* __restrict__ thr, int q0, double* __restrict__ out_val,
                                int* __restrict__ out_idx, int* __restrict__ next, float* __restrict__ next_thr,
                                int* __restrict__ next_count) {
    const int q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= Q) return;
    const int64_t row = queue[q0 + q];
    if (cnt[q] > cap) {
        const int slot = atomicAdd(next_count, 1);
        next[slot] = (int)row;
        next_thr[slot] = thr[q];
        return;
    }
    double v[K];
    int id[K];
#pragma unroll
    for (int s = 0; s < K; ++s) { v[s] = -INFINITY; id[s] = -1; }
    for (int sl = 0; sl < spr; ++sl) {
        const int64_t base = ((int64_t)q * spr + sl) * k;
        for (int s = 0; s < k; ++s)
            if (pi[base + s] >= 0) put_sorted<K>(v, id, k, pv[base + s], pi[base + s]);
    }
#pragma unroll
    for (int s = 0; s < K; ++s)
        if (s < k) { out_val[row * k + s] = v[s]; out_idx[row * k + s] = id[s]; }
}

}  // namespace

// Scratch of the wide pass (workspace slices; layout() sizes them).
struct WideBufs {
    float* redo_thr;   // [m + n] thresholds of the rows a finalize queued, by queue slot
    float* qs;         // [panel_rows(WIDE_ROWS)] int8 scales of the gathered rows (int8 sweep)
    // deferred column finalize (fused columns): per column its first candidate, need and candidates, the
    // bucket counts / offsets of a chunk's X rows, the bucketed order and its length
    DeferBufs defer;
    int* dcount;
    int* doffset;
    int* dorder;
    int* dtotal;
    float* rows;       // [panel_rows(WIDE_ROWS) * ld] gathered sweep rows
    float* thr;        // [panel_rows(WIDE_ROWS)]
    int* cnt;          // [panel_rows(WIDE_ROWS)]
    int* buf;          // [WIDE_BUF] candidate ids
    int* redo2;        // [m + n] rows that overflowed the first round, with
    float* redo2_thr;  // [m + n] their thresholds
    int* redo3;        // [m + n] rows that overflowed the second round (exact full rescan)
    float* redo3_thr;  // [m + n]
    int* redo_l;       // [m + n] queued rows their partial lists resolve (ListQueue of the finalize), with
    float* redo_l_thr;  // [m + n] their thresholds
    int* counts;       // [4]: redo2 and redo3 lengths
    unsigned int* rowthr;  // [rows of a sweep launch] the sweeps' shared row thresholds (row_threshold_*)
    const double* col_floor = nullptr;  // [n] the caller's column floors (l2sq_finalize's floor), or none
    double* floor_run;  // [n] (fused columns) the floors of a chunk: its k-th running column value, or the caller's
};

// Per-side data of the int8 sweep (HM_INT8X3; null otherwise): row scales, ||.||_1, the rows' error terms
// (l2sq_split_i8) and the maxima of each side's terms (4 keys per side). With y_ready the Y side's sweep copy
// and data come prepared (a resident side, hm_l2sq_resident_prepare) and are not rebuilt.
struct I8Bufs {
    float* xqs = nullptr;
    float* yqs = nullptr;
    double* xl1 = nullptr;
    double* yl1 = nullptr;
    double* xterm = nullptr;
    double* yterm = nullptr;
    unsigned long long* qmax_x = nullptr;
    unsigned long long* qmax_y = nullptr;
    bool y_ready = false;
};

// Resolves the rows a finalize queued (defined in pricing_l2sq.hip): the wide pass over them, then the exact full
// rescan of rows that overflowed it. A / B are the fp32 row and candidate sides (row stride d), Asw / Bsw their
// sweep copies (split-bf16 or int8 with row stride ld when `split`, else A / B), cand32 the candidates' fp32 biases,
// aqs / bqs the int8 scales of both sides (null unless the sweep is the int8 one).
// The partial lists a finalize call merged (its lists, R, nlists, G and KL), for the rows it queued to be
// resolved from them (WideBufs::redo_l, count at redo_count[1]); lists == nullptr when there are none.
struct ListSource {
    const Entry* lists = nullptr;
    int64_t R = 0;
    int nlists = 0;
    int G = 1;
    int KL = 8;
};

int wide_resolve(hipStream_t st, bool split, bool two_level, const float* A, const float* Asw, const float* B,
                 const float* Bsw, int64_t nb, int d, int sd, int ld, const float* cand32, const double* abias,
                 const double* bbias, double scale, int k, const int* redo, const int* redo_count,
                 double* out_val, int* out_idx, int cols, int cbase, const WideBufs& w, double* rpv, int* rpi,
                 const float* aqs, const float* bqs, const ListSource& ls = ListSource{});

namespace {

// merge a chunk's exact column lists into the running ones (both sorted by the tie rule)
__global__ void l2sq_merge_columns(double* __restrict__ val, int* __restrict__ idx, const double* __restrict__ cval,
                                   const int* __restrict__ cidx, int64_t n, int k, int first) {
    const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= n) return;
    double* v = val + j * k;
    int* id = idx + j * k;
    const double* cv = cval + j * k;
    const int* ci = cidx + j * k;
    if (first) {
        for (int s = 0; s < k; ++s) { v[s] = cv[s]; id[s] = ci[s]; }
        return;
    }
    double ov[32];
    int oi[32];
    int a = 0, b = 0;
    for (int s = 0; s < k; ++s) {
        if (better(cv[b], ci[b], v[a], id[a])) { ov[s] = cv[b]; oi[s] = ci[b]; ++b; }
        else { ov[s] = v[a]; oi[s] = id[a]; ++a; }
    }
    for (int s = 0; s < k; ++s) { v[s] = ov[s]; id[s] = oi[s]; }
}

// Floors of a chunk's fused column lists: the k-th value of each column's running list (every entry of which is
// an exact score of a pair already listed), or the caller's floor when that is higher.
__global__ void running_floor(double* __restrict__ out, int64_t n, const double* __restrict__ val, int k,
                              const double* __restrict__ user) {
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < n; j += (int64_t)gridDim.x * blockDim.x) {
        const double v = val[j * k + k - 1];
        out[j] = user ? fmax(v, user[j]) : v;
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

__global__ void fill_u32(unsigned int* p, int64_t count, unsigned int v) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

// -------------------------------------------------------------------------------------------------
// host orchestration
// -------------------------------------------------------------------------------------------------
// Candidates per row the finalize merges and keeps (KM), and entries per partial list of the sweep (KL).
// The int8 sweep's error bound is about three times the split-bf16 one (its quantization terms), so for k <= 2
// it keeps 16: fewer rows whose kept candidates do not separate from the dropped ones go to the wide pass.
inline int merge_k(int k, uint32_t flags) {
    if ((flags & HM_INT8X3) && k <= 2) return 16;
    return k <= 2 ? 8 : (k <= 8 ? 16 : 40);
}

// A partial list sees about 1/nlists of a row's candidates. Its last entry bounds what it dropped; that bound
// stays far below the k-th best unless the list holds KL of the best k + 2, so KL = 8 while (k + 2) / nlists <= 2
// and KL = 16 while <= 6 (a row whose bound does not separate is rescanned exactly).
inline int list_k_for(int64_t nlists, int k) {
    if ((int64_t)(k + 2) <= 2 * nlists) return 8;
    if ((int64_t)(k + 2) <= 6 * nlists) return 16;
    return 40;
}

// columns ride on the row sweep when that sweep runs anyway (rows or certificate requested); a columns-only call
// sweeps with the roles swapped, which needs no column epilogue
inline bool fused_columns(int d, uint32_t flags) {
    return (flags & HM_COLS) && (flags & (HM_ROWS | HM_STATS)) && d >= FUSE_MIN_D;
}

// split copies: features padded to 1, 2 or 4 chunks of 32, beyond that to whole groups of 4 chunks (the fp32
// block of the sweep); a row stride that is a multiple of 2 KiB gets one more chunk so the 32-row blocks do not
// all start on the same memory channel
inline int split_features(int d) { return d <= 32 ? 32 : d <= 64 ? 64 : (d + 127) / 128 * 128; }
inline int split_ld(int d) { return split_features(d) + (split_features(d) % 512 == 0 ? KC : 0); }
inline int64_t panel_rows(int64_t rows, int bx = BX) { return (rows + bx - 1) / bx * bx; }

// X rows per sweep workgroup: 256 for the split sweep with outer sums (l2sq_sweep_split_w), else 128
inline int sweep_panel(int d, uint32_t flags) {
    return ((flags & HM_INT8X3) || ((flags & HM_BF16X3) && d > KC * FLUSH_SPLIT)) ? BXW : BX;
}

// Rows per internal chunk of the swept side (m rows against n): balanced chunks of whole bx-row panels, and with
// fused columns the chunk's column partial lists (kl entries per panel and column) within COLPART_CAP.
inline int64_t chunk_rows(int64_t m, int64_t n, int kl, bool fused, int bx, int64_t cap = CHUNK_MAX) {
    int64_t ch = cap;
    if (fused) {
        const int64_t per_panel = n * (int64_t)kl * (int64_t)sizeof(Entry);
        int64_t panels = (int64_t)(COLPART_CAP / (size_t)per_panel);
        if (panels < 1) panels = 1;
        if (panels * bx < ch) ch = panels * bx;
    }
    const int64_t whole = panel_rows(m, bx);
    if (ch >= whole) return whole;
    const int64_t nch = (m + ch - 1) / ch;
    return panel_rows((m + nch - 1) / nch, bx);
}

// Y segments per sweep launch: enough workgroups to fill the chip (SWEEP_WGS), and for k > 2 at least 8 so each
// row has 16 partial lists; at most `cap`, and segments of at least `min_tiles` tiles (4 amortise a workgroup's
// start; the wide pass, whose few gathered rows make it latency-bound, takes 1). Among up to twice that many
// segments the first whose workgroups fill whole rounds of the CUs (within 3%) is taken: a partial last round
// idles CUs.
inline int choose_segments(int64_t m, int64_t n, int k, int cap, int bx, int min_tiles = 4) {
    const int64_t panels = (m + bx - 1) / bx;
    const int64_t tiles = (n + BY - 1) / BY;
    int64_t s = (SWEEP_WGS + panels - 1) / panels;
    if (k > 2 && s < 8) s = 8;
    int64_t max_s = tiles / min_tiles > 0 ? tiles / min_tiles : 1;
    if (max_s > cap) max_s = cap;
    if (s > max_s) s = max_s;
    if (s < 1) s = 1;
    int64_t best = s;
    double best_waste = 1e30;
    for (int64_t t = s; t <= max_s && t <= 2 * s; ++t) {
        const int64_t wgs = panels * t;  // padding workgroups of the blocked order exit at once
        const double waste = (double)((wgs + SWEEP_CUS - 1) / SWEEP_CUS * SWEEP_CUS) / (double)wgs - 1.0;
        if (waste < best_waste - 1e-12) {
            best = t;
            best_waste = waste;
        }
        if (waste <= 0.03) break;
    }
    return (int)best;
}

inline DirPlan plan_dir(int64_t rows, int64_t cols, int k, int cap, int bx, int min_tiles = 4) {
    DirPlan p;
    p.rows = rows;
    p.cols = cols;
    p.S = choose_segments(rows, cols, k, cap, bx, min_tiles);
    const int64_t tiles = (cols + BY - 1) / BY;
    const int64_t tiles_per = (tiles + p.S - 1) / p.S;
    p.seg_len = tiles_per * BY;
    p.S = (int)((cols + p.seg_len - 1) / p.seg_len);
    return p;
}

// Everything the workspace layout and the driver derive from the call's shape.
struct CallPlan {
    int kl, km;
    int bx;  // X rows per sweep workgroup
    bool fused, swapped, row_pass;
    // split copies made per internal chunk of the swept side (the other side's copy is whole): X's when only the
    // row pass runs, Y's when only the swapped pass runs; both whole when both run
    bool x_chunked, y_chunked;
    int64_t ch, ch2;  // chunk rows of the row pass and of the swapped pass
    DirPlan plan, plan2;
};

inline CallPlan plan_call(int64_t m, int64_t n, int d, int k, uint32_t flags, bool y_resident = false) {
    CallPlan c;
    c.km = merge_k(k, flags);
    c.fused = fused_columns(d, flags);
    c.swapped = (flags & HM_COLS) && !c.fused;
    c.row_pass = (flags & HM_ROWS) || c.fused || (flags & HM_STATS);
    c.bx = sweep_panel(d, flags);
    const bool split = (flags & (HM_BF16X3 | HM_INT8X3)) != 0;
    c.x_chunked = split && c.row_pass && !c.swapped;
    c.y_chunked = split && c.swapped && !c.row_pass;
    static const int sizes[3] = {8, 16, 40};
    // the int8 sweep's wider bound also wants deeper partial lists once k > 2 (their last entries bound what
    // they dropped)
    const int t0 = ((flags & HM_INT8X3) && k > 2) ? 1 : 0;
    for (int t = t0; t < 3; ++t) {
        c.kl = sizes[t];
        c.ch = chunk_rows(m, n, c.kl, c.fused, c.bx);
        c.plan = plan_dir(c.ch, n, k, 64, c.bx);
        c.ch2 = c.swapped ? chunk_rows(n, m, c.kl, false, c.bx, y_resident ? CHUNK_MAX_RESIDENT : CHUNK_MAX) : 0;
        c.plan2 = plan_dir(c.swapped ? c.ch2 : 1, m, k, 64, c.bx);
        if (c.kl >= c.km) break;
        // fewest partial lists any finalized row or column of this call merges
        int64_t nl = INT64_MAX;
        if (flags & HM_ROWS) nl = std::min<int64_t>(nl, 2 * (int64_t)c.plan.S);
        if (c.fused) {
            const int64_t last = m - (m - 1) / c.ch * c.ch;
            nl = std::min<int64_t>(nl, std::min<int64_t>(c.ch / c.bx, (last + c.bx - 1) / c.bx));
        }
        if (c.swapped) nl = std::min<int64_t>(nl, 2 * (int64_t)c.plan2.S);
        if (nl == INT64_MAX || list_k_for(nl, k) <= c.kl) break;
    }
    return c;
}

template <class A>
void layout(A& a, int64_t m, int64_t n, int d, int k, uint32_t flags, double** xnorm, double** ynorm, float** qb32,
            float** p32, float** db32, float** ge32, unsigned long long** maxima, Entry** part, Entry** colpart,
            unsigned int** colthr, double** cval, int** cidx, double** blockstats, int** redo, int** redo_count,
            float** xsplit, float** ysplit, double** rpv, int** rpi, WideBufs* wide, I8Bufs* q8,
            bool y_resident = false) {
    const CallPlan c = plan_call(m, n, d, k, flags, y_resident);
    const int64_t panels = c.ch / c.bx;
    size_t part_entries = (size_t)c.plan.S * c.ch * 2 * c.kl;
    if (c.swapped && (size_t)c.plan2.S * c.ch2 * 2 * c.kl > part_entries)
        part_entries = (size_t)c.plan2.S * c.ch2 * 2 * c.kl;
    const bool fused = c.fused;
    // with a resident Y side its norms, sweep copy and int8 data live in the resident buffer (resident_layout)
    *xnorm = a.template take<double>(m);
    *ynorm = y_resident ? nullptr : a.template take<double>(n);
    *qb32 = a.template take<float>(m);
    *p32 = a.template take<float>(m);
    *db32 = a.template take<float>(n);
    *ge32 = a.template take<float>(n);
    *maxima = a.template take<unsigned long long>(4);
    *part = a.template take<Entry>(part_entries);
    *colpart = a.template take<Entry>(fused ? (size_t)panels * n * c.kl : 1);
    *colthr = a.template take<unsigned int>(fused ? (size_t)n : 1);
    *cval = a.template take<double>(fused ? (size_t)n * k : 1);
    *cidx = a.template take<int>(fused ? (size_t)n * k : 1);
    *blockstats = a.template take<double>((size_t)5 * panels * c.plan.S);
    *redo = a.template take<int>((size_t)(m + n));
    *redo_count = a.template take<int>(2);
    const bool i8 = (flags & HM_INT8X3) != 0;
    const bool split = (flags & (HM_BF16X3 | HM_INT8X3)) != 0;
    const size_t ldw = (size_t)(i8 ? i8_ld(d) : split_ld(d));
    // split copies cover whole 256-row panels: either side may be the swept one
    *xsplit = a.template take<float>(split ? (size_t)panel_rows(c.x_chunked ? c.ch : m, BXW) * ldw : 1);
    *ysplit = y_resident ? nullptr
                         : a.template take<float>(split ? (size_t)panel_rows(c.y_chunked ? c.ch2 : n, BXW) * ldw : 1);
    *rpv = a.template take<double>((size_t)RESCAN_ITEMS * k);
    *rpi = a.template take<int>((size_t)RESCAN_ITEMS * k);
    const int64_t wq = panel_rows(WIDE_ROWS, BXW);
    wide->redo_thr = a.template take<float>((size_t)(m + n));
    wide->rows = a.template take<float>((size_t)wq * (split ? ldw : (size_t)d));
    wide->thr = a.template take<float>((size_t)wq);
    wide->cnt = a.template take<int>((size_t)wq);
    wide->buf = a.template take<int>((size_t)WIDE_BUF);
    wide->redo2 = a.template take<int>((size_t)(m + n));
    wide->redo2_thr = a.template take<float>((size_t)(m + n));
    wide->redo3 = a.template take<int>((size_t)(m + n));
    wide->redo3_thr = a.template take<float>((size_t)(m + n));
    wide->redo_l = a.template take<int>((size_t)(m + n));
    wide->redo_l_thr = a.template take<float>((size_t)(m + n));
    wide->counts = a.template take<int>(4);
    wide->rowthr = a.template take<unsigned int>((size_t)std::max<int64_t>(std::max<int64_t>(c.ch, c.ch2), 1));
    wide->floor_run = a.template take<double>(fused ? (size_t)n : 1);
    wide->qs = a.template take<float>((size_t)wq);
    wide->defer.key = a.template take<int>(fused ? (size_t)n : 1);
    wide->defer.need = a.template take<int>(fused ? (size_t)n : 1);
    wide->defer.cand = a.template take<int>(fused ? (size_t)n * c.km : 1);
    wide->dcount = a.template take<int>(fused ? (size_t)c.ch + 1 : 1);
    wide->doffset = a.template take<int>(fused ? (size_t)c.ch + 1 : 1);
    wide->dorder = a.template take<int>(fused ? (size_t)n : 1);
    wide->dtotal = a.template take<int>(1);
    *q8 = I8Bufs{};
    if (i8) {
        q8->xqs = a.template take<float>((size_t)m);
        q8->xl1 = a.template take<double>((size_t)m);
        q8->xterm = a.template take<double>((size_t)m * 4);
        q8->qmax_x = a.template take<unsigned long long>(4);
        if (!y_resident) {
            q8->yqs = a.template take<float>((size_t)n);
            q8->yl1 = a.template take<double>((size_t)n);
            q8->yterm = a.template take<double>((size_t)n * 4);
            q8->qmax_y = a.template take<unsigned long long>(4);
        }
    }
}

// A resident Y side (hm_l2sq_resident_*): its norms, its sweep copy for the precision in `flags` and, for the int8
// sweep, its scales, ||.||_1, error terms and their maxima, plus max ||y|| (an ordered key).
struct ResidentY {
    double* ynorm;
    float* ysplit;
    unsigned long long* ynorm_max;
    I8Bufs q8;  // the Y half
};

template <class A>
void resident_layout(A& a, int64_t n, int d, uint32_t flags, ResidentY* r) {
    const bool i8 = (flags & HM_INT8X3) != 0;
    const bool split = (flags & (HM_BF16X3 | HM_INT8X3)) != 0;
    const size_t ldw = (size_t)(i8 ? i8_ld(d) : split_ld(d));
    *r = ResidentY{};
    r->ynorm = a.template take<double>((size_t)n);
    r->ysplit = split ? a.template take<float>((size_t)panel_rows(n, BXW) * ldw) : nullptr;
    r->ynorm_max = a.template take<unsigned long long>(2);  // [max ||y||, unused slot of the prep kernel]
    if (i8) {
        r->q8.yqs = a.template take<float>((size_t)n);
        r->q8.yl1 = a.template take<double>((size_t)n);
        r->q8.yterm = a.template take<double>((size_t)n * 4);
        r->q8.qmax_y = a.template take<unsigned long long>(4);
    }
}

// Exact rescan of the rows queued by a finalize: reads the queue length back (one host synchronisation), then
// splits every queued row's candidates into slices scanned by separate waves and merges the slice lists.
inline int rescan_exact(hipStream_t st, const float* A, const float* B, int64_t nb, int d, const double* abias,
                        const double* bbias, double scale, int k, const int* redo, const int* redo_count,
                        double* out_val, int* out_idx, int cols, int cbase, double* pv, int* pi) {
    int count = 0;
    HM_HIP(hipMemcpyAsync(&count, redo_count, sizeof(int), hipMemcpyDeviceToHost, st));
    HM_HIP(hipStreamSynchronize(st));
    prof_count(cols ? "l2sq_rescan_columns" : "l2sq_rescan_rows", count);
    if (count <= 0) return HM_OK;
    int64_t slices = (nb + RESCAN_SLICE - 1) / RESCAN_SLICE;
    if (slices > 1024) slices = 1024;
    if (slices < 1) slices = 1;
    const int64_t per = (nb + slices - 1) / slices;
    const int64_t batch = RESCAN_ITEMS / slices > 0 ? RESCAN_ITEMS / slices : 1;
    prof_begin(st, "l2sq_rescan");
    for (int64_t r0 = 0; r0 < count; r0 += batch) {
        const int nrows = (int)(count - r0 < batch ? count - r0 : batch);
        const int64_t items = (int64_t)nrows * slices;
        const unsigned grid = (unsigned)((items + 3) / 4 < 4096 ? (items + 3) / 4 : 4096);
        const unsigned mgrid = (unsigned)((nrows + 255) / 256);
#define HM_RESCAN(KK)                                                                                               \
    do {                                                                                                            \
        hipLaunchKernelGGL((l2sq_rescan_slices<KK>), dim3(grid), dim3(256), 0, st, A, B, nb, d, abias, bbias, scale, \
                           k, redo, (int)r0, nrows, (int)slices, per, cols, cbase, pv, pi);                        \
        hipLaunchKernelGGL((l2sq_rescan_merge<KK>), dim3(mgrid), dim3(256), 0, st, pv, pi, nrows, (int)slices, k,    \
                           redo, (int)r0, out_val, out_idx);                                                       \
    } while (0)
        if (k <= 2) HM_RESCAN(2);
        else if (k <= 8) HM_RESCAN(8);
        else HM_RESCAN(32);
#undef HM_RESCAN
        HM_LAUNCH_CHECK("l2sq_rescan");
    }
    prof_end(st);
    return HM_OK;
}

// int8 copy of one side (its maxima are cleared first, with a kernel)
inline void launch_split_i8(hipStream_t st, const float* X, int64_t rows, int d, int sd, int ld, float* qs,
                            const double* l1, const double* norm, float* out, double* qterm,
                            unsigned long long* qmax) {
    hipLaunchKernelGGL(zero_words, dim3(1), dim3(64), 0, st, qmax, 4);
    hipLaunchKernelGGL(l2sq_split_i8, dim3((unsigned)std::min<int64_t>(panel_rows(rows, BXW) / 32, 8192)), dim3(256),
                       0, st, X, rows, panel_rows(rows, BXW), d, sd, ld, qs, l1, norm,
                       reinterpret_cast<unsigned int*>(out), qterm, qmax);
}

template <int K1, int KM>
int run_bidir(hipStream_t st, const float* X, const float* Y, int64_t m, int64_t n, int d, int k, double scale,
              uint32_t flags, const double* qb, const double* db, const double* xnorm, const double* ynorm,
              const unsigned long long* maxima, const float* qb32, const float* db32, const float* p32,
              const float* ge32, Entry* part, Entry* colpart, unsigned int* colthr, double* cval, int* cidx,
              double* blockstats, int* redo, int* redo_count, double* row_val, int* row_idx, double* col_val,
              int* col_idx, double* stats, float* xsplit, float* ysplit, double* rpv, int* rpi,
              const WideBufs& wide, const I8Bufs& q8) {
    // K1: entries per partial list of the sweep; KM: candidates the finalize merges and keeps
    const CallPlan cp = plan_call(m, n, d, k, flags, q8.y_ready);
    if (cp.kl != K1 || cp.km != KM) return fail(HM_EINVAL, "l2sq pricing: list sizes %d/%d do not match the plan %d/%d", K1, KM, cp.kl, cp.km);
    const bool want_rows = (flags & HM_ROWS) != 0;
    const bool fused = cp.fused;
    const bool swapped = cp.swapped;
    const bool want_stats = (flags & HM_STATS) != 0;
    const int linf = (flags & HM_LINF) ? 1 : 0;
    const bool i8 = (flags & HM_INT8X3) != 0;
    const bool split = (flags & (HM_BF16X3 | HM_INT8X3)) != 0;  // the sweep reads operand-order copies
    const int flush = KC * (split ? FLUSH_SPLIT : FLUSH_CHUNKS);
    const bool two_level = i8 || d > flush;  // the int8 sweep is always the 256-row one
    const bool vec4 = split || (d % 4) == 0;
    // swept 4-byte words per row of the copy, and its row stride
    const int sd = i8 ? i8_words(d) : split ? split_features(d) : d;
    const int ld = i8 ? i8_ld(d) : split ? split_ld(d) : d;
    const float* SX = split ? xsplit : X;
    const float* SY = split ? ysplit : Y;
    const int64_t ch = cp.ch;
    const DirPlan plan = cp.plan;
    const int bx = cp.bx;
    unsigned int* rowthr = wide.rowthr;
    // Sweep copies: rows [r0, r0 + rows) of one side into `out` (its row r0 first). A side whose copy is made per
    // internal chunk (CallPlan::x_chunked / y_chunked) is copied in the chunk loops below, the others here whole (the
    // Y side not at all when it is a prepared resident side). The int8 row scales and ||.||_1 come from the prep
    // pass; the int8 copy adds ||l||_2, the rows' error terms and the copied rows' maxima.
    auto copy_rows = [&](bool y_side, int64_t r0, int64_t rows, float* out) {
        const float* src = (y_side ? Y : X) + r0 * d;
        if (i8) {
            if (y_side)
                launch_split_i8(st, src, rows, d, sd, ld, q8.yqs + r0, q8.yl1 + r0, ynorm + r0, out,
                                q8.yterm + 4 * r0, q8.qmax_y);
            else
                launch_split_i8(st, src, rows, d, sd, ld, q8.xqs + r0, q8.xl1 + r0, xnorm + r0, out,
                                q8.xterm + 4 * r0, q8.qmax_x);
        } else {
            hipLaunchKernelGGL(l2sq_split_bf16, dim3(4096), dim3(256), 0, st, src, rows, panel_rows(rows, BXW), d, sd,
                               ld, reinterpret_cast<unsigned short*>(out));
        }
        HM_LAUNCH_CHECK("split copy");
        return HM_OK;
    };
    if (split && !cp.x_chunked)
        if (int rc = copy_rows(false, 0, m, xsplit)) return rc;
    if (split && !cp.y_chunked && !q8.y_ready)
        if (int rc = copy_rows(true, 0, n, ysplit)) return rc;
    // Rigorous bound on |w - exact| in units of scale*||x||*||y||: accumulation of B-feature blocks in fp32
    // (gamma over the additions of a block, then over the blocks), plus for the split products the dropped
    // terms lo*lo + hi*e + e*hi + ... <= (3 * 2^-16 * (1 + 2^-7) + 3 * 2^-24) |x_k y_k|.
    const double fb = two_level ? (double)flush : (double)d;
    // (the 256-row split sweep restarts its 4 accumulator blocks at staggered chunks: one block more per dot)
    const double nblk = two_level ? std::ceil((double)d / flush) + (split ? 1.0 : 0.0) : 1.0;
    const double terms = split ? 3.0 * fb * (1.0 + 1.0 / 8.0) : fb;
    const double ea = gamma_fp32(terms) + gamma_fp32(nblk) + gamma_fp32(terms) * gamma_fp32(nblk);
    const double split_rel = split ? 3.0 * std::ldexp(1.0, -16) * (1.0 + std::ldexp(1.0, -7)) + 3.0 * std::ldexp(1.0, -24)
                                   : 0.0;
    const double u = std::ldexp(1.0, -24);
    BoundArgs bnd;
    bnd.acc_rel = split_rel + ea * (split ? 1.01 : 1.0) + u * (1.0 + ea + split_rel) + 4e-15 * (d / 64.0 + 8.0);
    if (i8) bnd.acc_rel = 1.01 * u + 4e-15 * (d / 64.0 + 8.0);  // the rounding of w; the dot's terms come per row
    bnd.db_rel = 2.0 * u + 1e-15;
    bnd.abs_slack = 1e-30 * (double)d;
    // finalizes of X rows (candidates Y) and of Y rows (candidates X); the int8 terms are indexed from `base` rows
    auto bound_for = [&](bool y_rows, int64_t base) {
        BoundArgs b = bnd;
        if (i8) {
            b.qterm = (y_rows ? q8.yterm : q8.xterm) + 4 * base;
            b.qmax = y_rows ? q8.qmax_x : q8.qmax_y;
        }
        return b;
    };
    const CertArgs cert{qb, db, maxima + 2, xnorm};  // the row pass sweeps X rows against Y (maxima[2..3]: Y side)
    int chunk_index = 0;
    const bool row_pass = cp.row_pass;  // a columns-only call without fusion skips it
    for (int64_t xb = 0; row_pass && xb < m; xb += ch, ++chunk_index) {
        const int64_t xe = xb + ch < m ? xb + ch : m;
        const int64_t rows = xe - xb;
        const int64_t panels = (rows + bx - 1) / bx;
        const dim3 grid(sweep_grid(panels, plan.S));
        const unsigned neg_inf_key = 0x007fffffu;  // float_key(-INFINITY)
        // this chunk's split copy of X (the sweeps take the copy from the chunk's first row)
        if (split && cp.x_chunked)
            if (int rc = copy_rows(false, xb, rows, xsplit)) return rc;
        const float* SXc = !split ? SX : (cp.x_chunked ? xsplit : SX + xb * ld);
        // floors of this chunk's column lists: the caller's, and after the first chunk the running lists' k-th
        // values (a chunk's lists then only keep what can enter the merged lists)
        const double* cfloor = wide.col_floor;
        if (fused && chunk_index > 0) {
            hipLaunchKernelGGL(running_floor, dim3((unsigned)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096)),
                               dim3(256), 0, st, wide.floor_run, n, col_val, k, wide.col_floor);
            HM_LAUNCH_CHECK("running_floor");
            cfloor = wide.floor_run;
        }
        if (fused) {
            // column thresholds start at -inf for every chunk (its lists only rank its own X rows), or at the floors
            const dim3 tgrid((unsigned)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096));
            if (cfloor)
                hipLaunchKernelGGL(seed_floor_thresholds, tgrid, dim3(256), 0, st, colthr, n, cfloor, ynorm, db,
                                   maxima, scale, bound_for(true, 0));
            else
                hipLaunchKernelGGL(fill_u32, tgrid, dim3(256), 0, st, colthr, n, neg_inf_key);
            HM_LAUNCH_CHECK("column thresholds");
        }
        // row thresholds start at -inf for every chunk (they index the chunk's rows)
        hipLaunchKernelGGL(fill_u32, dim3((unsigned)((rows + 255) / 256 < 4096 ? (rows + 255) / 256 : 4096)), dim3(256), 0,
                           st, rowthr, rows, neg_inf_key);
        HM_LAUNCH_CHECK("fill_u32");
#define NOWIDE (const float*)nullptr, (int*)nullptr, (int*)nullptr, 0
#define HM_SWEEP(TL, CL, ST)                                                                                         \
    do {                                                                                                             \
        if (i8)                                                                                                      \
            hipLaunchKernelGGL((l2sq_sweep_i8_w<K1, CL, false, ST>), grid, dim3(THREADS_W), 0, st, SXc, SY, xb, xe, n, sd, ld,  \
                               qb32, db32, p32, ge32, (float)scale, plan.seg_len, (int)panels, plan.S, part,         \
                               colpart, colthr, blockstats, (int)want_stats, cert, q8.xqs, q8.yqs, NOWIDE, rowthr); \
        else if (split && TL)                                                                                        \
            hipLaunchKernelGGL((l2sq_sweep_split_w<K1, CL, false, ST>), grid, dim3(THREADS_W), 0, st, SXc, SY, xb,   \
                               xe, n, sd,                                                                            \
                               ld, qb32, db32, p32, ge32, (float)scale, plan.seg_len, (int)panels, plan.S, part,     \
                               colpart, colthr, blockstats, (int)want_stats, cert, NOWIDE, rowthr);                 \
        else if (split)                                                                                              \
            hipLaunchKernelGGL((l2sq_sweep_split<K1, CL, false, ST>), grid, dim3(256), 0, st, SXc, SY, xb, xe, n,    \
                               sd, ld,                                                                               \
                               qb32, db32, p32, ge32, (float)scale, plan.seg_len, (int)panels, plan.S, part,         \
                               colpart, colthr, blockstats, (int)want_stats, cert, NOWIDE, rowthr);                 \
        else                                                                                                         \
            hipLaunchKernelGGL((l2sq_sweep<K1, TL, CL, false, ST>), grid, dim3(256), 0, st, X, Y, xb, xe, n, d, d,   \
                               qb32,                                                                                 \
                               db32, p32, ge32, (float)scale, plan.seg_len, (int)panels, plan.S, part, colpart,      \
                               colthr, blockstats, (int)vec4, (int)want_stats, cert, NOWIDE, rowthr);               \
    } while (0)
        prof_begin(st, "l2sq_sweep");
        // sweeps without the certificate take the instantiation without its code (ST of sweep_epilogue)
        if (want_stats) {
            if (two_level) {
                if (fused) HM_SWEEP(true, true, true);
                else HM_SWEEP(true, false, true);
            } else {
                if (fused) HM_SWEEP(false, true, true);
                else HM_SWEEP(false, false, true);
            }
        } else {
            if (two_level) {
                if (fused) HM_SWEEP(true, true, false);
                else HM_SWEEP(true, false, false);
            } else {
                if (fused) HM_SWEEP(false, true, false);
                else HM_SWEEP(false, false, false);
            }
        }
        prof_end(st);
#undef HM_SWEEP
        HM_LAUNCH_CHECK("l2sq_sweep");
        if (want_stats) {
            hipLaunchKernelGGL(l2sq_reduce_stats, dim3(1), dim3(256), 0, st, blockstats, (int64_t)panels * plan.S,
                               stats, linf, chunk_index > 0 ? 1 : 0);
            HM_LAUNCH_CHECK("l2sq_reduce_stats");
        }
        if (want_rows) {
            // row finalize: lists (seg, half) of each chunk row; candidates are Y rows
            hipLaunchKernelGGL(zero_words, dim3(1), dim3(64), 0, st, reinterpret_cast<unsigned long long*>(redo_count), 1);
            prof_begin(st, "l2sq_finalize");
            hipLaunchKernelGGL((l2sq_finalize<K1, KM, 2, false>), dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st,
                               X + xb * d, Y, rows, d, 2 * plan.S, part, qb + xb, db, xnorm + xb, maxima + 2, scale, k,
                               bound_for(false, xb), row_val + xb * k, row_idx + xb * k, redo, wide.redo_thr,
                               redo_count, DeferBufs{}, ListQueue{wide.redo_l, wide.redo_l_thr});
            prof_end(st);
            HM_LAUNCH_CHECK("l2sq_finalize");
            if (int rc = wide_resolve(st, split, two_level, X + xb * d, SXc, Y, SY, n, d, sd, ld, db32,
                                      qb + xb, db, scale, k, redo, redo_count, row_val + xb * k, row_idx + xb * k, 0,
                                      0, wide, rpv, rpi, i8 ? q8.xqs + xb : nullptr, q8.yqs,
                                      ListSource{part, rows, 2 * plan.S, 2, K1}))
                return rc;
        }
        if (fused) {
            // column finalize: one list per X panel of this chunk; candidates are the chunk's X rows (global ids)
            hipLaunchKernelGGL(zero_words, dim3(1), dim3(64), 0, st, reinterpret_cast<unsigned long long*>(redo_count), 1);
            prof_begin(st, "l2sq_col_finalize");
            // selection (queued columns go to the wide pass), then the exact evaluation with the columns grouped by
            // their first candidate: the chunk's X rows are then read about once each rather than once per column
            hipLaunchKernelGGL((l2sq_finalize<K1, KM, 1, true, true>), dim3((unsigned)((n + 3) / 4)), dim3(256), 0, st,
                               Y, X, n, d, (int)panels, colpart, db, qb, ynorm, maxima, scale, k, bound_for(true, 0),
                               cval, cidx, redo, wide.redo_thr, redo_count, wide.defer,
                               ListQueue{wide.redo_l, wide.redo_l_thr}, cfloor);
            HM_LAUNCH_CHECK("l2sq_col_finalize");
            const unsigned egrid = (unsigned)((n + 255) / 256 < 8192 ? (n + 255) / 256 : 8192);
            hipLaunchKernelGGL(fill_u32, dim3((unsigned)((rows + 256) / 256)), dim3(256), 0, st,
                               reinterpret_cast<unsigned int*>(wide.dcount), rows, 0u);
            hipLaunchKernelGGL(defer_count, dim3(egrid), dim3(256), 0, st, wide.defer.key, n, (int)xb, (int)rows,
                               wide.dcount);
            hipLaunchKernelGGL(defer_scan, dim3(1), dim3(1024), 0, st, wide.dcount, (int)rows, wide.doffset,
                               wide.dtotal);
            hipLaunchKernelGGL(defer_scatter, dim3(egrid), dim3(256), 0, st, wide.defer.key, n, (int)xb, (int)rows,
                               wide.doffset, wide.dorder);
            hipLaunchKernelGGL((l2sq_finalize_exact<KM, true>), dim3((unsigned)((n + 3) / 4)), dim3(256), 0, st, Y, X,
                               d, wide.dorder, wide.dtotal, wide.defer, db, qb, scale, k, cval, cidx);
            prof_end(st);
            HM_LAUNCH_CHECK("l2sq_col_finalize (exact)");
            if (int rc = wide_resolve(st, split, two_level, Y, SY, X + xb * d, SXc, rows, d, sd, ld,
                                      qb32 + xb, db, qb + xb, scale, k, redo, redo_count, cval, cidx, 1, (int)xb,
                                      wide, rpv, rpi, q8.yqs, i8 ? q8.xqs + xb : nullptr,
                                      ListSource{colpart, n, (int)panels, 1, K1}))
                return rc;
            hipLaunchKernelGGL(l2sq_merge_columns, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, col_val, col_idx,
                               cval, cidx, n, k, chunk_index == 0 ? 1 : 0);
            HM_LAUNCH_CHECK("l2sq_merge_columns");
        }
    }
    if (swapped) {
        // columns by a second sweep with the roles swapped: Y chunks are the rows, X is segmented; the
        // finalize keeps the (dot + qb) + db association of the caller's pairs
        const int64_t ch2 = cp.ch2;
        const DirPlan plan2 = cp.plan2;
        for (int64_t yb = 0; yb < n; yb += ch2) {
            const int64_t ye = yb + ch2 < n ? yb + ch2 : n;
            const int64_t rows = ye - yb;
            const int64_t panels2 = (rows + bx - 1) / bx;
            const dim3 grid(sweep_grid(panels2, plan2.S));
            // this chunk's split copy of Y (from its first row; a resident side's copy is whole)
            if (split && cp.y_chunked && !q8.y_ready)
                if (int rc = copy_rows(true, yb, rows, ysplit)) return rc;
            const float* SYc = !split ? SY : ((cp.y_chunked && !q8.y_ready) ? ysplit : SY + yb * ld);
            // the rows' shared thresholds start at -inf, or at the caller's column floors
            const dim3 tgrid((unsigned)((rows + 255) / 256 < 4096 ? (rows + 255) / 256 : 4096));
            if (wide.col_floor)
                hipLaunchKernelGGL(seed_floor_thresholds, tgrid, dim3(256), 0, st, rowthr, rows, wide.col_floor + yb,
                                   ynorm + yb, db + yb, maxima, scale, bound_for(true, yb));
            else
                hipLaunchKernelGGL(fill_u32, tgrid, dim3(256), 0, st, rowthr, rows,
                                   0x007fffffu /* float_key(-INFINITY) */);
            HM_LAUNCH_CHECK("row thresholds");
#define HM_SWEEP2(TL)                                                                                                \
    do {                                                                                                             \
        if (i8)                                                                                                      \
            hipLaunchKernelGGL((l2sq_sweep_i8_w<K1, false>), grid, dim3(THREADS_W), 0, st, SYc, SX, yb, ye, m, sd,   \
                               ld, db32, qb32, ge32, p32, (float)scale, plan2.seg_len, (int)panels2, plan2.S, part,  \
                               colpart, colthr, blockstats, 0, CertArgs{}, q8.yqs, q8.xqs, NOWIDE, rowthr);         \
        else if (split && TL)                                                                                        \
            hipLaunchKernelGGL((l2sq_sweep_split_w<K1, false>), grid, dim3(THREADS_W), 0, st, SYc, SX, yb, ye, m, sd,\
                               ld, db32, qb32, ge32, p32, (float)scale, plan2.seg_len, (int)panels2, plan2.S, part,  \
                               colpart, colthr, blockstats, 0, CertArgs{}, NOWIDE, rowthr);                         \
        else if (split)                                                                                              \
            hipLaunchKernelGGL((l2sq_sweep_split<K1, false>), grid, dim3(256), 0, st, SYc, SX, yb, ye, m, sd, \
                               ld, db32, qb32, ge32, p32, (float)scale, plan2.seg_len, (int)panels2, plan2.S, part,  \
                               colpart, colthr, blockstats, 0, CertArgs{}, NOWIDE, rowthr);                         \
        else                                                                                                         \
            hipLaunchKernelGGL((l2sq_sweep<K1, TL, false>), grid, dim3(256), 0, st, Y, X, yb, ye, m, d, d, db32,     \
                               qb32, ge32, p32, (float)scale, plan2.seg_len, (int)panels2, plan2.S, part, colpart,   \
                               colthr, blockstats, (int)vec4, 0, CertArgs{}, NOWIDE, rowthr);                       \
    } while (0)
            prof_begin(st, "l2sq_sweep");
            if (two_level) HM_SWEEP2(true);
            else HM_SWEEP2(false);
            prof_end(st);
#undef HM_SWEEP2
#undef NOWIDE
            HM_LAUNCH_CHECK("l2sq_sweep");
            hipLaunchKernelGGL(zero_words, dim3(1), dim3(64), 0, st, reinterpret_cast<unsigned long long*>(redo_count), 1);
            prof_begin(st, "l2sq_col_finalize");
            hipLaunchKernelGGL((l2sq_finalize<K1, KM, 2, true>), dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st,
                               Y + yb * d, X, rows, d, 2 * plan2.S, part, db + yb, qb, ynorm + yb, maxima, scale, k,
                               bound_for(true, yb), col_val + yb * k, col_idx + yb * k, redo, wide.redo_thr,
                               redo_count, DeferBufs{}, ListQueue{wide.redo_l, wide.redo_l_thr},
                               wide.col_floor ? wide.col_floor + yb : nullptr);
            prof_end(st);
            HM_LAUNCH_CHECK("l2sq_col_finalize");
            if (int rc = wide_resolve(st, split, two_level, Y + yb * d, SYc, X, SX, m, d, sd, ld, qb32,
                                      db + yb, qb, scale, k, redo, redo_count, col_val + yb * k, col_idx + yb * k, 1,
                                      0, wide, rpv, rpi, i8 ? q8.yqs + yb : nullptr, q8.xqs,
                                      ListSource{part, rows, 2 * plan2.S, 2, K1}))
                return rc;
        }
    }
    if (want_stats) {
        if (!want_rows) return fail(HM_EINVAL, "l2sq pricing: the certificate needs the row lists");
        hipLaunchKernelGGL(exact_row_max, dim3(1), dim3(256), 0, st, row_val, m, k, stats);
        HM_LAUNCH_CHECK("exact_row_max");
    }
    return HM_OK;
}

}  // namespace
}  // namespace hm

// driver signature shared by the per-K1 translation units
#define L2SQ_RUN_ARGS                                                                                              \
    hipStream_t st, const float *X, const float *Y, int64_t m, int64_t n, int d, int k, double scale, uint32_t flags, \
        const double *qb, const double *db, const double *xnorm, const double *ynorm,                              \
        const unsigned long long *maxima, const float *qb32, const float *db32, const float *p32, const float *ge32, \
        ::hm::Entry *part, ::hm::Entry *colpart, unsigned int *colthr, double *cval, int *cidx, double *blockstats, \
        int *redo, int *redo_count, double *row_val, int *row_idx, double *col_val, int *col_idx, double *stats,   \
        float *xsplit, float *ysplit, double *rpv, int *rpi, const ::hm::WideBufs &wide, const ::hm::I8Bufs &q8
#define L2SQ_RUN_PASS                                                                                               \
    st, X, Y, m, n, d, k, scale, flags, qb, db, xnorm, ynorm, maxima, qb32, db32, p32, ge32, part, colpart, colthr, \
        cval, cidx, blockstats, redo, redo_count, row_val, row_idx, col_val, col_idx, stats, xsplit, ysplit, rpv, rpi, \
        wide, q8
