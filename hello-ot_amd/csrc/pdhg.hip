// Restricted-OT Halpern-PDHG on gfx950.
//
// Algorithm: _native/cpp/solver.cpp:39-378 (= _internal/lp/torch_restricted_ot.py:105-393; the same update
// CuPDLPx runs in cupdlpx/solver.cu:581-715): degree-sqrt constraint scaling, variable scale sqrt(2),
// constant step 0.998, reflected Halpern iterations, PID primal-weight restarts and relative L2 KKT checks
// every `evaluation_frequency` iterations.
//
// Device layout: the per-edge primal state is mirrored in two orders so that both halves of an iteration
// stream their edges contiguously and never gather per-edge values.
//   source order (position p): edges sorted by source, ascending caller edge id within a source (stable
//     sort), so source i owns [off[i], off[i+1]); perm[p] = caller edge id. Arrays: col, row, scaled cost cs,
//     iterate x, anchor ax, PDHG point px (stored only when the next iteration evaluates), checkpoint delta dx.
//   target order (slot k): edges sorted by target, ascending caller edge id within a target, so target t owns
//     [off[n+t]-e, off[n+t+1]-e). Arrays: row_t, cs_t, x_t, ax_t, px_t.
// Both copies receive identical operands in identical order and therefore stay bit-identical.
// Per node (sources then targets): scale, bs, ns, y, ay, py, dy; td = y / ns for targets and sd = y / ns for
// sources (the value the current iteration's primal step used).
//
// One iteration = source pass + target pass (the restatement's two loops):
//   source pass: per source node, its edges' PDHG step and reflection, their iterates (Halpern), and the node's
//                dual from the in-order sum of the reflections;
//   target pass: per target node, the same steps for its edges from the mirrored state and the source duals sd,
//                and the target dual from its in-order sum.
// Each side runs in one of two shapes, chosen per solve from the side's largest degree: G-lane groups per node
// (lanes sum in edge order through shuffles) when every node fits in one chunk of the group, else node blocks
// (edge-parallel steps, then one thread per node sums its reflections in edge order from LDS). Both are
// bit-identical to a sequential sum.
// The only gathers are of node values (sd, td). Scalars read back to the host only at evaluations and checkpoints.
//
// Node numbering: on large problems (at least HELLOOT_PDHG_REORDER nodes, default 2^20, where the duals outgrow
// an XCD's L2) the nodes are renumbered inside the solve so that nodes joined by many edges get nearby numbers:
// each node's position is a few rounds of neighbour averaging from pseudo-random target values (integer arithmetic,
// so the numbering is the same on every run), then each side is sorted by it. On HELLO's supports, which join a
// point to its near neighbours, this groups the support's clusters and the dual gathers hit L2 (1.6x faster
// iterations at 1.28M x 1.28M than with shuffled numbers). A node's edges keep ascending caller ids, so every
// per-node and per-edge operation is unchanged; only the orders of the global norm sums differ.
#include <hipcub/hipcub.hpp>

#include <chrono>
#include <climits>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "common.h"

namespace hm {
namespace {

constexpr int RB = 1024;     // blocks of the fixed-shape reductions
constexpr int RT = 256;      // threads per reduction block

struct Pdhg {
    int64_t n, nt, nodes, e;
    // edges, source order
    int32_t *row, *col, *perm;
    double *cs, *x, *ax, *px, *dx;
    // edges, target order
    int32_t *row_t, *col_t;
    double *cs_t, *x_t, *ax_t, *px_t;
    // node-block passes: each edge's own node within its block (the low bits of row / col_t; blocks hold a power
    // of two of consecutive nodes), one byte per edge instead of the four-byte node number
    uint8_t *loc_s, *loc_t;
    // node-block passes: the other side's node each edge gathers from (col / row_t) as a 16-bit offset from its
    // block's smallest one, when the block's edges span fewer than 65536 nodes of that side (gbase = that
    // smallest node), else gbase = -1 and the pass reads the 4-byte number
    uint16_t *g16_s, *g16_t;
    int32_t *gbase_s, *gbase_t;
    // nodes
    double *scale, *bs, *ns, *y, *ay, *py, *dy, *td, *sd;
    int32_t *deg, *off, *eid;
    // node numbering (map_s / map_t: internal number of a caller source / target, or null for the identity;
    // inv: caller node of an internal node, sources then targets) and its scratch
    int32_t *map_s, *map_t, *inv, *odeg;
    uint32_t* ov;
    unsigned long long *osum, *okeys_in, *okeys_out;
    void* osort_tmp;
    size_t osort_tmp_bytes;
    // sort scratch
    uint32_t *keys_in, *keys_out;
    int32_t *vals_in;
    void* sort_tmp;
    size_t sort_tmp_bytes;
    // reductions
    double* partial;   // RB * 4
    double* result;    // 4
    int* flag;         // 1
};

template <class A>
void pdhg_layout(A& a, int64_t n, int64_t nt, int64_t e, size_t sort_tmp, size_t osort_tmp, Pdhg& P) {
    const int64_t nodes = n + nt, side = n > nt ? n : nt;
    P.row = a.template take<int32_t>(e);
    P.col = a.template take<int32_t>(e);
    P.perm = a.template take<int32_t>(e);
    P.cs = a.template take<double>(e);
    P.x = a.template take<double>(e);
    P.ax = a.template take<double>(e);
    P.px = a.template take<double>(e);
    P.dx = a.template take<double>(e);
    P.row_t = a.template take<int32_t>(e);
    P.col_t = a.template take<int32_t>(e);
    P.cs_t = a.template take<double>(e);
    P.x_t = a.template take<double>(e);
    P.ax_t = a.template take<double>(e);
    P.px_t = a.template take<double>(e);
    P.loc_s = a.template take<uint8_t>(e);
    P.loc_t = a.template take<uint8_t>(e);
    P.g16_s = a.template take<uint16_t>(e);
    P.g16_t = a.template take<uint16_t>(e);
    P.gbase_s = a.template take<int32_t>(n + 1);
    P.gbase_t = a.template take<int32_t>(nt + 1);
    P.scale = a.template take<double>(nodes);
    P.bs = a.template take<double>(nodes);
    P.ns = a.template take<double>(nodes);
    P.y = a.template take<double>(nodes);
    P.ay = a.template take<double>(nodes);
    P.py = a.template take<double>(nodes);
    P.dy = a.template take<double>(nodes);
    P.td = a.template take<double>(nt);
    P.sd = a.template take<double>(n);
    P.deg = a.template take<int32_t>(nodes + 1);
    P.off = a.template take<int32_t>(nodes + 1);
    P.eid = a.template take<int32_t>(2 * e);
    P.keys_in = a.template take<uint32_t>(2 * e);
    P.keys_out = a.template take<uint32_t>(2 * e);
    P.vals_in = a.template take<int32_t>(2 * e);
    P.sort_tmp = a.template take<char>(sort_tmp > 0 ? sort_tmp : 1);
    P.sort_tmp_bytes = sort_tmp;
    P.partial = a.template take<double>((size_t)RB * 4);
    P.result = a.template take<double>(4);
    P.flag = a.template take<int>(4);
    P.map_s = a.template take<int32_t>(n);
    P.map_t = a.template take<int32_t>(nt);
    P.inv = a.template take<int32_t>(nodes);
    P.odeg = a.template take<int32_t>(nodes);
    P.ov = a.template take<uint32_t>(nodes);
    P.osum = a.template take<unsigned long long>(nodes);
    P.okeys_in = a.template take<unsigned long long>(side);
    P.okeys_out = a.template take<unsigned long long>(side);
    P.osort_tmp = a.template take<char>(osort_tmp > 0 ? osort_tmp : 1);
    P.osort_tmp_bytes = osort_tmp;
}

inline int end_bit_for(int64_t nodes) {
    int b = 1;
    while (b < 32 && (int64_t(1) << b) < nodes) ++b;
    return b;
}

inline size_t sort_tmp_bytes(int64_t nodes, int64_t e) {
    size_t bytes = 0;  // a size query: it only writes `bytes`
    (void)hipcub::DeviceRadixSort::SortPairs(nullptr, bytes, (const uint32_t*)nullptr, (uint32_t*)nullptr,
                                             (const int32_t*)nullptr, (int32_t*)nullptr, (int)(2 * e), 0,
                                             end_bit_for(nodes));
    return bytes;
}

// key of a node in the numbering sort: position (32 bits) above the node's side-local number (31 bits)
constexpr int ORDER_KEY_BITS = 63;

inline size_t order_sort_tmp_bytes(int64_t n, int64_t nt) {
    size_t bytes = 0;  // a size query: it only writes `bytes`
    (void)hipcub::DeviceRadixSort::SortKeys(nullptr, bytes, (const unsigned long long*)nullptr,
                                            (unsigned long long*)nullptr, (int)(n > nt ? n : nt), 0,
                                            ORDER_KEY_BITS);
    return bytes;
}

// smallest node count whose solve renumbers its nodes (HELLOOT_PDHG_REORDER: a count, or "off")
inline int64_t reorder_min_nodes() {
    const char* v = std::getenv("HELLOOT_PDHG_REORDER");
    if (v == nullptr || *v == 0) return int64_t(1) << 20;
    if (std::strcmp(v, "off") == 0) return INT64_MAX;
    char* end = nullptr;
    const long long t = std::strtoll(v, &end, 10);
    return (end && *end == 0 && t >= 0) ? (int64_t)t : (int64_t(1) << 20);
}

constexpr int ORDER_ROUNDS = 6;  // neighbour-averaging rounds (each: sources from targets, then targets)

// ---------------------------------------------------------------------------------------------------------
// setup kernels
// ---------------------------------------------------------------------------------------------------------
// Per node block (one workgroup each): the range of the other side's nodes its edges gather from, and when it spans
// fewer than 65536 nodes, each edge's gathered node as an offset from the smallest (Pdhg::g16_*, gbase_*). The
// block's edges are [off[b * npb] - ebase, off[min((b + 1) * npb, nodes)] - ebase).
__global__ __launch_bounds__(256) void k_gather_base(const int32_t* __restrict__ off, int64_t nodes, int npb,
                                                     int32_t ebase, const int32_t* __restrict__ gidx,
                                                     int32_t* __restrict__ gbase, uint16_t* __restrict__ g16) {
    __shared__ int32_t smin[256], smax[256];
    const int64_t b = blockIdx.x;
    const int64_t n0 = b * npb, n1 = n0 + npb < nodes ? n0 + npb : nodes;
    const int32_t e0 = off[n0] - ebase, e1 = off[n1] - ebase;
    int32_t lo = INT32_MAX, hi = INT32_MIN;
    for (int32_t p = e0 + (int32_t)threadIdx.x; p < e1; p += 256) {
        const int32_t g = gidx[p];
        lo = g < lo ? g : lo;
        hi = g > hi ? g : hi;
    }
    smin[threadIdx.x] = lo;
    smax[threadIdx.x] = hi;
    __syncthreads();
    for (int w = 128; w >= 1; w >>= 1) {
        if ((int)threadIdx.x < w) {
            smin[threadIdx.x] = smin[threadIdx.x + w] < smin[threadIdx.x] ? smin[threadIdx.x + w] : smin[threadIdx.x];
            smax[threadIdx.x] = smax[threadIdx.x + w] > smax[threadIdx.x] ? smax[threadIdx.x + w] : smax[threadIdx.x];
        }
        __syncthreads();
    }
    lo = smin[0];
    hi = smax[0];
    const bool narrow = e1 > e0 && (int64_t)hi - (int64_t)lo < 65536;
    if (threadIdx.x == 0) gbase[b] = narrow ? lo : -1;
    if (narrow)
        for (int32_t p = e0 + (int32_t)threadIdx.x; p < e1; p += 256) g16[p] = (uint16_t)(gidx[p] - lo);
}

// low bits of each edge's node number (its index within a node block of mask + 1 nodes)
__global__ void k_low_bits(const int32_t* __restrict__ node, int64_t e, int32_t mask, uint8_t* __restrict__ out) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < e; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = (uint8_t)(node[i] & mask);
}

__global__ void k_fill_i32(int32_t* p, int64_t count, int32_t v) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

// validation, degrees and the (node key, caller edge id) pairs of the incidence sort
__global__ void k_edges(const int64_t* __restrict__ rows, const int64_t* __restrict__ cols, int64_t e, int64_t n,
                        int64_t nt, const int32_t* __restrict__ map_s, const int32_t* __restrict__ map_t,
                        int32_t* __restrict__ deg, uint32_t* __restrict__ keys, int32_t* __restrict__ vals,
                        int* __restrict__ flag) {
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < e; j += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = rows[j], c = cols[j];
        if (r < 0 || r >= n || c < 0 || c >= nt) {
            atomicOr(flag, 1);
            keys[j] = 0;
            keys[e + j] = (uint32_t)n;
        } else {
            const int64_t ri = map_s ? map_s[r] : r, ci = map_t ? map_t[c] : c;
            atomicAdd(&deg[ri], 1);
            atomicAdd(&deg[n + ci], 1);
            keys[j] = (uint32_t)ri;
            keys[e + j] = (uint32_t)(n + ci);
        }
        vals[j] = (int32_t)j;
        vals[e + j] = (int32_t)j;
    }
}

// flag[1] / flag[2] = largest source / target degree (flag[1..2] start at 0)
__global__ void k_degree_max(const int32_t* __restrict__ deg, int64_t n, int64_t nodes, int* __restrict__ flag) {
    int ms = 0, mt = 0;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nodes; i += (int64_t)gridDim.x * blockDim.x) {
        if (i < n) ms = deg[i] > ms ? deg[i] : ms;
        else mt = deg[i] > mt ? deg[i] : mt;
    }
    for (int o = 32; o >= 1; o >>= 1) {
        ms = max(ms, __shfl_xor(ms, o, 64));
        mt = max(mt, __shfl_xor(mt, o, 64));
    }
    if ((threadIdx.x & 63) == 0) {
        if (ms > 0) atomicMax(&flag[1], ms);
        if (mt > 0) atomicMax(&flag[2], mt);
    }
}

// After the stable sort eid[0..e) lists caller edge ids by source and eid[e..2e) by target.
__global__ void k_source_setup(const int32_t* __restrict__ eid, int64_t e, const int64_t* __restrict__ rows,
                               const int64_t* __restrict__ cols, const double* __restrict__ c,
                               const double* __restrict__ x0, double bound, double objective, double variable,
                               Pdhg P) {
    for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < e; p += (int64_t)gridDim.x * blockDim.x) {
        const int32_t j = eid[p];
        P.perm[p] = j;
        P.row[p] = P.map_s ? P.map_s[rows[j]] : (int32_t)rows[j];
        P.col[p] = P.map_t ? P.map_t[cols[j]] : (int32_t)cols[j];
        P.cs[p] = c[j] * objective / variable;
        const double a = x0 ? fmax(x0[j], 0.0) * variable * bound : 0.0;
        P.ax[p] = a;
        P.x[p] = a;
        P.px[p] = a;
        P.dx[p] = 0.0;
    }
}

__global__ void k_target_setup(const int32_t* __restrict__ eid, int64_t e, const int64_t* __restrict__ rows,
                               const int64_t* __restrict__ cols, const double* __restrict__ c,
                               const double* __restrict__ x0, double bound, double objective, double variable,
                               Pdhg P) {
    for (int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; k < e; k += (int64_t)gridDim.x * blockDim.x) {
        const int32_t j = eid[e + k];
        P.row_t[k] = P.map_s ? P.map_s[rows[j]] : (int32_t)rows[j];
        P.col_t[k] = P.map_t ? P.map_t[cols[j]] : (int32_t)cols[j];
        P.cs_t[k] = c[j] * objective / variable;
        const double a = x0 ? fmax(x0[j], 0.0) * variable * bound : 0.0;
        P.ax_t[k] = a;
        P.x_t[k] = a;
        P.px_t[k] = a;
    }
}

// exclusive scan of deg[0..nodes) into off[0..nodes] with a single workgroup (setup only)
__global__ void k_scan(const int32_t* __restrict__ deg, int64_t nodes, int32_t* __restrict__ off) {
    __shared__ int64_t sums[1024];
    const int t = threadIdx.x;
    const int64_t per = (nodes + 1023) / 1024;
    const int64_t b0 = t * per, b1 = (b0 + per < nodes) ? b0 + per : nodes;
    int64_t s = 0;
    for (int64_t i = b0; i < b1; ++i) s += deg[i];
    sums[t] = s;
    __syncthreads();
    if (t == 0) {
        int64_t run = 0;
        for (int i = 0; i < 1024; ++i) {
            const int64_t v = sums[i];
            sums[i] = run;
            run += v;
        }
    }
    __syncthreads();
    int64_t run = sums[t];
    for (int64_t i = b0; i < b1; ++i) {
        off[i] = (int32_t)run;
        run += deg[i];
    }
    if (t == 1023) off[nodes] = (int32_t)run;  // the last range ends at `nodes`, so run is the total
}

__global__ void k_node_setup(const int32_t* __restrict__ deg, const double* __restrict__ b,
                             const double* __restrict__ y0, const int32_t* __restrict__ inv, int64_t nodes, int64_t n,
                             double bound, double objective, double variable, double* __restrict__ scale,
                             double* __restrict__ bs, double* __restrict__ ns, double* __restrict__ y,
                             double* __restrict__ ay, double* __restrict__ py, double* __restrict__ dy,
                             double* __restrict__ td) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nodes; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t o = inv ? inv[i] : i;  // the caller's number of internal node i
        const double sc = sqrt((double)(deg[i] > 1 ? deg[i] : 1));
        scale[i] = sc;
        bs[i] = b[o] * bound / sc;
        const double nsv = variable * sc;
        ns[i] = nsv;
        const double a = y0 ? y0[o] * sc * objective : 0.0;
        ay[i] = a;
        y[i] = a;
        py[i] = a;
        dy[i] = 0.0;
        if (i >= n) td[i - n] = a / nsv;
    }
}

// ---------------------------------------------------------------------------------------------------------
// node numbering (large problems): positions from neighbour averaging, then a sort of each side
// ---------------------------------------------------------------------------------------------------------
// validation and the caller-numbered degrees
__global__ void k_order_degrees(const int64_t* __restrict__ rows, const int64_t* __restrict__ cols, int64_t e,
                                int64_t n, int64_t nt, int32_t* __restrict__ odeg, int* __restrict__ flag) {
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < e; j += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = rows[j], c = cols[j];
        if (r < 0 || r >= n || c < 0 || c >= nt) {
            atomicOr(flag, 1);
        } else {
            atomicAdd(&odeg[r], 1);
            atomicAdd(&odeg[n + c], 1);
        }
    }
}

// targets start from pseudo-random 32-bit positions (a 64-bit mix of the target number), sources from 0
__global__ void k_order_seed(uint32_t* __restrict__ ov, int64_t n, int64_t nodes) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nodes; i += (int64_t)gridDim.x * blockDim.x) {
        uint64_t z = (uint64_t)(i - n) + 0x9E3779B97F4A7C15ull;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        z ^= z >> 31;
        ov[i] = i < n ? 0u : (uint32_t)(z >> 32);
    }
}

__global__ void k_order_clear(unsigned long long* __restrict__ osum, int64_t count) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x)
        osum[i] = 0ull;
}

// integer sums of the other side's positions over each node's edges (exact, so independent of the order)
__global__ void k_order_gather(const int64_t* __restrict__ rows, const int64_t* __restrict__ cols, int64_t e,
                               int64_t n, int to_sources, const uint32_t* __restrict__ ov,
                               unsigned long long* __restrict__ osum) {
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < e; j += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = rows[j], c = n + cols[j];
        if (to_sources) atomicAdd(&osum[r], (unsigned long long)ov[c]);
        else atomicAdd(&osum[c], (unsigned long long)ov[r]);
    }
}

// mean position of nodes [lo, hi) (a node without edges keeps its position)
__global__ void k_order_mean(const unsigned long long* __restrict__ osum, const int32_t* __restrict__ odeg,
                             int64_t lo, int64_t hi, uint32_t* __restrict__ ov) {
    for (int64_t i = lo + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < hi; i += (int64_t)gridDim.x * blockDim.x)
        if (odeg[i] > 0) ov[i] = (uint32_t)(osum[i] / (unsigned long long)odeg[i]);
}

// sort keys of nodes [lo, lo + count): position, then side-local number
__global__ void k_order_keys(const uint32_t* __restrict__ ov, int64_t lo, int64_t count,
                             unsigned long long* __restrict__ keys) {
    for (int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; k < count; k += (int64_t)gridDim.x * blockDim.x)
        keys[k] = ((unsigned long long)ov[lo + k] << 31) | (unsigned long long)k;
}

// rank r of the sorted keys is the internal number of side-local node k: map[k] = r, inv[base + r] = base + k
__global__ void k_order_ranks(const unsigned long long* __restrict__ sorted, int64_t count, int64_t base,
                              int32_t* __restrict__ map, int32_t* __restrict__ inv) {
    for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < count; r += (int64_t)gridDim.x * blockDim.x) {
        const int64_t k = (int64_t)(sorted[r] & 0x7FFFFFFFull);
        map[k] = (int32_t)r;
        inv[base + r] = (int32_t)(base + k);
    }
}

// ---------------------------------------------------------------------------------------------------------
// fixed-shape reductions: grid RB x RT, grid-stride partial sums, then one block combines RB partials
// ---------------------------------------------------------------------------------------------------------
template <int Q>
__device__ inline void block_reduce_store(double (&v)[Q], double* __restrict__ partial) {
    __shared__ double s[RT / 64][4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int q = 0; q < Q; ++q)
        for (int o = 32; o >= 1; o >>= 1) v[q] = v[q] + __shfl_xor(v[q], o, 64);
    if (lane == 0)
        for (int q = 0; q < Q; ++q) s[wave][q] = v[q];
    __syncthreads();
    if (threadIdx.x == 0)
        for (int q = 0; q < Q; ++q) {
            double t = s[0][q];
            for (int w = 1; w < RT / 64; ++w) t = t + s[w][q];
            partial[(size_t)blockIdx.x * 4 + q] = t;
        }
}

__global__ void k_combine(const double* __restrict__ partial, double* __restrict__ result, int q) {
    __shared__ double s[RT][4];
    const int t = threadIdx.x;
    double v[4] = {0, 0, 0, 0};
    for (int b = t; b < RB; b += RT)
        for (int k = 0; k < q; ++k) v[k] = v[k] + partial[(size_t)b * 4 + k];
    for (int k = 0; k < 4; ++k) s[t][k] = v[k];
    __syncthreads();
    for (int w = RT / 2; w >= 1; w >>= 1) {
        if (t < w)
            for (int k = 0; k < 4; ++k) s[t][k] = s[t][k] + s[t + w][k];
        __syncthreads();
    }
    if (t == 0)
        for (int k = 0; k < q; ++k) result[k] = s[0][k];
}

__global__ void k_sumsq(const double* __restrict__ a, int64_t count, double* __restrict__ partial) {
    double v[1] = {0.0};
    for (int64_t i = (int64_t)blockIdx.x * RT + threadIdx.x; i < count; i += (int64_t)RB * RT) v[0] = v[0] + a[i] * a[i];
    block_reduce_store<1>(v, partial);
}

__global__ void k_diffsq2(const double* __restrict__ a, const double* __restrict__ b, int64_t na,
                          const double* __restrict__ c, const double* __restrict__ d, int64_t nc,
                          double* __restrict__ partial) {
    double v[2] = {0.0, 0.0};
    for (int64_t i = (int64_t)blockIdx.x * RT + threadIdx.x; i < na; i += (int64_t)RB * RT) {
        const double t = a[i] - b[i];
        v[0] = v[0] + t * t;
    }
    for (int64_t i = (int64_t)blockIdx.x * RT + threadIdx.x; i < nc; i += (int64_t)RB * RT) {
        const double t = c[i] - d[i];
        v[1] = v[1] + t * t;
    }
    block_reduce_store<2>(v, partial);
}

// evaluation: [primal_sq, dobj, dual_sq, pobj]
__global__ void k_evaluate(const Pdhg P, const double* __restrict__ b, const double* __restrict__ c, double variable,
                           double bound, double objective, double* __restrict__ partial) {
    double v[4] = {0.0, 0.0, 0.0, 0.0};
    const double vb = variable * bound;
    for (int64_t i = (int64_t)blockIdx.x * RT + threadIdx.x; i < P.nodes; i += (int64_t)RB * RT) {
        double sum = 0.0;
        if (i < P.n) {
            for (int32_t k = P.off[i]; k < P.off[i + 1]; ++k) sum += P.px[k] / vb;
        } else {
            for (int32_t k = P.off[i]; k < P.off[i + 1]; ++k) sum += P.px_t[k - P.e] / vb;
        }
        const double bi = b[P.inv ? P.inv[i] : i];
        const double delta = sum - bi;
        v[0] = v[0] + delta * delta;
        v[1] = v[1] + bi * (P.py[i] / (P.scale[i] * objective));
    }
    for (int64_t j = (int64_t)blockIdx.x * RT + threadIdx.x; j < P.e; j += (int64_t)RB * RT) {
        const int32_t r = P.row[j], cc = P.col[j];
        const double cj = c[P.perm[j]];
        const double score = P.py[r] / (P.scale[r] * objective) + P.py[P.n + cc] / (P.scale[P.n + cc] * objective) - cj;
        const double viol = fmax(score, 0.0);
        v[2] = v[2] + viol * viol;
        v[3] = v[3] + cj * (P.px[j] / vb);
    }
    block_reduce_store<4>(v, partial);
}

// fixed-point error pieces: [movement, dual_movement, interaction]
__global__ void k_fixed_point(const Pdhg P, double* __restrict__ partial) {
    double v[3] = {0.0, 0.0, 0.0};
    for (int64_t j = (int64_t)blockIdx.x * RT + threadIdx.x; j < P.e; j += (int64_t)RB * RT) {
        const double d = P.dx[j];
        const int32_t r = P.row[j], cc = P.col[j];
        v[0] = v[0] + d * d;
        v[2] = v[2] + (P.dy[r] / P.ns[r] + P.dy[P.n + cc] / P.ns[P.n + cc]) * d;
    }
    for (int64_t i = (int64_t)blockIdx.x * RT + threadIdx.x; i < P.nodes; i += (int64_t)RB * RT)
        v[1] = v[1] + P.dy[i] * P.dy[i];
    block_reduce_store<3>(v, partial);
}

// ---------------------------------------------------------------------------------------------------------
// iteration kernels
// ---------------------------------------------------------------------------------------------------------
// Sum of the group's per-lane values in lane order 0..count-1 (every lane of the group gets the same bits as
// a sequential loop over the group's edges).
template <int G>
__device__ inline double group_ordered_sum(double running, double value, int count) {
    if (count == G) {  // a whole group: every shuffle issued before the first add
        double t[G];
#pragma unroll
        for (int u = 0; u < G; ++u) t[u] = __shfl(value, u, G);
#pragma unroll
        for (int u = 0; u < G; ++u) running += t[u];
        return running;
    }
    for (int t = 0; t < count; ++t) running += __shfl(value, t, G);
    return running;
}

// Source pass: a G-lane group per source node (the restatement's first loop, solver.cpp:210-251 order).
// A chunk covers G*U edges: lane g owns edges g, g+G, ..., g+(U-1)G of the chunk, all loaded before any sum.
template <int G, int U, bool CHECKPOINT, bool STORE>
__global__ __launch_bounds__(256) void k_source_pass(const Pdhg P, double primal_step, double dual_step,
                                                     double halpern) {
    const double keep = 1.0 - halpern;
    const int g = threadIdx.x % G;
    const int64_t stride = (int64_t)gridDim.x * (blockDim.x / G);
    for (int64_t i = (int64_t)blockIdx.x * (blockDim.x / G) + threadIdx.x / G; i < P.n; i += stride) {
        const int32_t k0 = P.off[i], k1 = P.off[i + 1];
        const double yi = P.y[i], nsi = P.ns[i];
        const double source_dual = yi / nsi;
        double sum = 0.0;
        for (int32_t base = k0; base < k1; base += G * U) {
            double r[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int32_t p = base + u * G + g;
                r[u] = 0.0;
                if (p < k1) {
                    const double at = source_dual + P.td[P.col[p]];
                    const double xj = P.x[p];
                    const double pxj = fmax(xj - primal_step * (P.cs[p] - at), 0.0);
                    r[u] = 2.0 * pxj - xj;
                    if (STORE) P.px[p] = pxj;
                    if (CHECKPOINT) P.dx[p] = r[u] - xj;
                    P.x[p] = halpern * r[u] + keep * P.ax[p];
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int32_t left = k1 - (base + u * G);
                if (left > 0) sum = group_ordered_sum<G>(sum, r[u], left < G ? left : G);
            }
        }
        if (g == 0) {
            P.sd[i] = source_dual;
            const double pyi = yi - dual_step * (sum / nsi - P.bs[i]);
            const double refl = 2.0 * pyi - yi;
            if (STORE) P.py[i] = pyi;
            if (CHECKPOINT) P.dy[i] = refl - yi;
            P.y[i] = halpern * refl + keep * P.ay[i];
        }
    }
}

// Target pass: a G-lane group per target node recomputes its edges' steps from the target-order mirror (the
// operands are those the source pass used: sd of this iteration, td before this update) and updates the dual.
template <int G, int U, bool CHECKPOINT, bool STORE>
__global__ __launch_bounds__(256) void k_target_pass(const Pdhg P, double primal_step, double dual_step,
                                                     double halpern) {
    const double keep = 1.0 - halpern;
    const int g = threadIdx.x % G;
    const int64_t stride = (int64_t)gridDim.x * (blockDim.x / G);
    for (int64_t t = (int64_t)blockIdx.x * (blockDim.x / G) + threadIdx.x / G; t < P.nt; t += stride) {
        const int64_t i = P.n + t;
        const int32_t k0 = P.off[i] - (int32_t)P.e, k1 = P.off[i + 1] - (int32_t)P.e;
        const double target_dual = P.td[t];
        double sum = 0.0;
        for (int32_t base = k0; base < k1; base += G * U) {
            double r[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int32_t k = base + u * G + g;
                r[u] = 0.0;
                if (k < k1) {
                    const double at = P.sd[P.row_t[k]] + target_dual;
                    const double xj = P.x_t[k];
                    const double pxj = fmax(xj - primal_step * (P.cs_t[k] - at), 0.0);
                    r[u] = 2.0 * pxj - xj;
                    if (STORE) P.px_t[k] = pxj;
                    P.x_t[k] = halpern * r[u] + keep * P.ax_t[k];
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int32_t left = k1 - (base + u * G);
                if (left > 0) sum = group_ordered_sum<G>(sum, r[u], left < G ? left : G);
            }
        }
        if (g == 0) {
            const double yi = P.y[i], nsi = P.ns[i];
            const double pyi = yi - dual_step * (sum / nsi - P.bs[i]);
            const double refl = 2.0 * pyi - yi;
            if (STORE) P.py[i] = pyi;
            if (CHECKPOINT) P.dy[i] = refl - yi;
            const double yn = halpern * refl + keep * P.ay[i];
            P.y[i] = yn;
            P.td[t] = yn / nsi;
        }
    }
}

// Node-block passes: a workgroup owns `npb` consecutive nodes of one side and their edges (contiguous in that side's
// order). Edges are processed EB at a time: every thread computes edge steps (coalesced streams, one gather of the
// other side's dual), the reflections go to LDS, and then one thread per node adds its edges' reflections in edge
// order from LDS, carrying its running sum across the rounds. Same operations, operands and order as the
// lane-group passes above, so the iterates are bit-identical; the work per workgroup follows the edges, not the
// node count, and a node's fold is a run of LDS reads instead of lane shuffles.
constexpr int EB = 2048;  // edges per round
constexpr int PT = 256;   // threads per workgroup (also the largest npb)

// sum + v[a] + v[a+1] + ... + v[b-1], added one by one in that order; the LDS reads go out eight at a time so that
// a long node waits for one read latency per eight values rather than per value.
__device__ __forceinline__ double fold_in_order(const double* v, int a, int b, double sum) {
    int k = a;
    for (; k + 8 <= b; k += 8) {
        double t[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) t[u] = v[k + u];
#pragma unroll
        for (int u = 0; u < 8; ++u) sum += t[u];
    }
    for (; k < b; ++k) sum += v[k];
    return sum;
}

template <bool CHECKPOINT, bool STORE>
__global__ __launch_bounds__(PT) void k_source_block(const Pdhg P, double primal_step, double dual_step,
                                                     double halpern, int npb) {
    __shared__ double sr[EB];
    __shared__ double sdl[PT];
    __shared__ int32_t soff[PT + 1];
    const int tid = threadIdx.x;
    const int64_t n0 = (int64_t)blockIdx.x * npb;
    const int nn = (int)(P.n - n0 < npb ? P.n - n0 : npb);
    const double keep = 1.0 - halpern;
    double yi = 0.0, nsi = 1.0;
    if (tid < nn) {
        yi = P.y[n0 + tid];
        nsi = P.ns[n0 + tid];
        sdl[tid] = yi / nsi;
    }
    for (int t = tid; t <= nn; t += PT) soff[t] = P.off[n0 + t];
    __syncthreads();
    const int32_t e0 = soff[0], e1 = soff[nn];
    const int32_t k0 = tid < nn ? soff[tid] : 0, k1 = tid < nn ? soff[tid + 1] : 0;
    double sum = 0.0;
    const int32_t gb = P.gbase_s[blockIdx.x];  // uniform: 16-bit gather offsets, or -1 for 4-byte numbers
    // edge p (slot q of the round) with its target c
    auto step = [&](int32_t p, int q, int32_t c) {
        const double at = sdl[P.loc_s[p]] + P.td[c];
        const double xj = P.x[p];
        const double pxj = fmax(xj - primal_step * (P.cs[p] - at), 0.0);
        const double r = 2.0 * pxj - xj;
        if (STORE) P.px[p] = pxj;
        if (CHECKPOINT) P.dx[p] = r - xj;
        P.x[p] = halpern * r + keep * P.ax[p];
        sr[q] = r;
    };
    for (int32_t base = e0; base < e1; base += EB) {
        const int len = e1 - base < EB ? e1 - base : EB;
        if (gb >= 0) {
            for (int q = tid; q < len; q += PT) step(base + q, q, gb + (int32_t)P.g16_s[base + q]);
        } else {
            for (int q = tid; q < len; q += PT) step(base + q, q, P.col[base + q]);
        }
        __syncthreads();
        sum = fold_in_order(sr, (k0 > base ? k0 : base) - base, (k1 < base + len ? k1 : base + len) - base, sum);
        __syncthreads();
    }
    if (tid < nn) {
        const int64_t i = n0 + tid;
        P.sd[i] = sdl[tid];
        const double pyi = yi - dual_step * (sum / nsi - P.bs[i]);
        const double refl = 2.0 * pyi - yi;
        if (STORE) P.py[i] = pyi;
        if (CHECKPOINT) P.dy[i] = refl - yi;
        P.y[i] = halpern * refl + keep * P.ay[i];
    }
}

template <bool CHECKPOINT, bool STORE>
__global__ __launch_bounds__(PT) void k_target_block(const Pdhg P, double primal_step, double dual_step,
                                                     double halpern, int npb) {
    __shared__ double sr[EB];
    __shared__ double tdl[PT];
    __shared__ int32_t soff[PT + 1];
    const int tid = threadIdx.x;
    const int64_t t0 = (int64_t)blockIdx.x * npb;
    const int nn = (int)(P.nt - t0 < npb ? P.nt - t0 : npb);
    const double keep = 1.0 - halpern;
    if (tid < nn) tdl[tid] = P.td[t0 + tid];
    for (int t = tid; t <= nn; t += PT) soff[t] = P.off[P.n + t0 + t] - (int32_t)P.e;
    __syncthreads();
    const int32_t e0 = soff[0], e1 = soff[nn];
    const int32_t k0 = tid < nn ? soff[tid] : 0, k1 = tid < nn ? soff[tid + 1] : 0;
    double sum = 0.0;
    const int32_t gb = P.gbase_t[blockIdx.x];  // uniform: 16-bit gather offsets, or -1 for 4-byte numbers
    // edge k (slot q of the round) with its source c
    auto step = [&](int32_t k, int q, int32_t c) {
        const double at = P.sd[c] + tdl[P.loc_t[k]];
        const double xj = P.x_t[k];
        const double pxj = fmax(xj - primal_step * (P.cs_t[k] - at), 0.0);
        const double r = 2.0 * pxj - xj;
        if (STORE) P.px_t[k] = pxj;
        P.x_t[k] = halpern * r + keep * P.ax_t[k];
        sr[q] = r;
    };
    for (int32_t base = e0; base < e1; base += EB) {
        const int len = e1 - base < EB ? e1 - base : EB;
        if (gb >= 0) {
            for (int q = tid; q < len; q += PT) step(base + q, q, gb + (int32_t)P.g16_t[base + q]);
        } else {
            for (int q = tid; q < len; q += PT) step(base + q, q, P.row_t[base + q]);
        }
        __syncthreads();
        sum = fold_in_order(sr, (k0 > base ? k0 : base) - base, (k1 < base + len ? k1 : base + len) - base, sum);
        __syncthreads();
    }
    if (tid < nn) {
        const int64_t i = P.n + t0 + tid;
        const double yi = P.y[i], nsi = P.ns[i];
        const double pyi = yi - dual_step * (sum / nsi - P.bs[i]);
        const double refl = 2.0 * pyi - yi;
        if (STORE) P.py[i] = pyi;
        if (CHECKPOINT) P.dy[i] = refl - yi;
        const double yn = halpern * refl + keep * P.ay[i];
        P.y[i] = yn;
        P.td[t0 + tid] = yn / nsi;
    }
}

__global__ void k_restart(const Pdhg P) {
    const int64_t total = P.e > P.nodes ? P.e : P.nodes;
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < total; j += (int64_t)gridDim.x * blockDim.x) {
        if (j < P.e) {
            const double v = P.px[j];
            P.ax[j] = v;
            P.x[j] = v;
            const double vt = P.px_t[j];
            P.ax_t[j] = vt;
            P.x_t[j] = vt;
        }
        if (j < P.nodes) {
            const double v = P.py[j];
            P.ay[j] = v;
            P.y[j] = v;
            if (j >= P.n) P.td[j - P.n] = v / P.ns[j];
        }
    }
}

__global__ void k_output(const Pdhg P, double vb, double objective, double* __restrict__ xo, double* __restrict__ yo) {
    const int64_t total = P.e > P.nodes ? P.e : P.nodes;
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < total; j += (int64_t)gridDim.x * blockDim.x) {
        if (j < P.e) xo[P.perm[j]] = P.px[j] / vb;
        if (j < P.nodes) yo[P.inv ? P.inv[j] : j] = P.py[j] / (P.scale[j] * objective);
    }
}

inline unsigned grid_of(int64_t items) {
    int64_t b = (items + 255) / 256;
    if (b > 8192) b = 8192;
    if (b < 1) b = 1;
    return (unsigned)b;
}

inline unsigned group_grid(int64_t nodes, int g) {
    int64_t b = (nodes + (256 / g) - 1) / (256 / g);
    if (b > 65536) b = 65536;
    if (b < 1) b = 1;
    return (unsigned)b;
}

// Both passes run GL-lane groups with U edges per lane per chunk (U = 1, 2 or 4 from the side's mean degree).
constexpr int GL = 8;

inline int edges_per_lane(int64_t e, int64_t nodes) {
    const int64_t mean = (e + nodes - 1) / nodes;
    return mean <= GL ? 1 : (mean <= 12 ? 2 : 4);
}

// nodes per workgroup of a node-block pass: about 2048 workgroups, at most PT nodes each
inline int nodes_per_block(int64_t nodes) {
    int npb = 1;
    while (npb < PT && (int64_t)npb * 2 * 2048 <= nodes) npb *= 2;
    return npb;
}

// How one side's pass runs: lane groups of U edges per lane (u > 0), or node blocks (u = 0). Lane groups when
// every node of the side fits in one chunk of GL * U edges: each lane then holds at most U independent edges and
// no group waits for a longer neighbour. Otherwise node blocks, whose work follows the edges (on the supports of
// the HELLO levels, where degrees spread to several times their mean, they take 27-32% less time per iteration;
// on uniform degree 16 the lane groups are 8% faster).
struct SidePlan {
    int u, npb;
};

inline SidePlan side_plan(int64_t e, int64_t nodes, int max_degree) {
    const int u = edges_per_lane(e, nodes);
    return SidePlan{max_degree <= GL * u ? u : 0, nodes_per_block(nodes)};
}

template <bool C, bool S>
void launch_source(hipStream_t st, const Pdhg& P, const SidePlan& sp, double ps, double ds, double h) {
    const dim3 grid(group_grid(P.n, GL)), block(256);
    if (sp.u == 0)
        hipLaunchKernelGGL((k_source_block<C, S>), dim3((unsigned)((P.n + sp.npb - 1) / sp.npb)), dim3(PT), 0, st, P,
                           ps, ds, h, sp.npb);
    else if (sp.u == 1) hipLaunchKernelGGL((k_source_pass<GL, 1, C, S>), grid, block, 0, st, P, ps, ds, h);
    else if (sp.u == 2) hipLaunchKernelGGL((k_source_pass<GL, 2, C, S>), grid, block, 0, st, P, ps, ds, h);
    else hipLaunchKernelGGL((k_source_pass<GL, 4, C, S>), grid, block, 0, st, P, ps, ds, h);
}

template <bool C, bool S>
void launch_target(hipStream_t st, const Pdhg& P, const SidePlan& sp, double ps, double ds, double h) {
    const dim3 grid(group_grid(P.nt, GL)), block(256);
    if (sp.u == 0)
        hipLaunchKernelGGL((k_target_block<C, S>), dim3((unsigned)((P.nt + sp.npb - 1) / sp.npb)), dim3(PT), 0, st, P,
                           ps, ds, h, sp.npb);
    else if (sp.u == 1) hipLaunchKernelGGL((k_target_pass<GL, 1, C, S>), grid, block, 0, st, P, ps, ds, h);
    else if (sp.u == 2) hipLaunchKernelGGL((k_target_pass<GL, 2, C, S>), grid, block, 0, st, P, ps, ds, h);
    else hipLaunchKernelGGL((k_target_pass<GL, 4, C, S>), grid, block, 0, st, P, ps, ds, h);
}

template <bool C, bool S>
void launch_pair(hipStream_t st, const Pdhg& P, const SidePlan& src, const SidePlan& tgt, double ps, double ds,
                 double h) {
    launch_source<C, S>(st, P, src, ps, ds, h);
    launch_target<C, S>(st, P, tgt, ps, ds, h);
}

// One PDHG iteration (source pass + target pass). px / py are stored only on major iterations: they are read
// only by the evaluation that follows one.
int launch_iteration(hipStream_t st, const Pdhg& P, const SidePlan& src, const SidePlan& tgt, bool checkpoint,
                     bool major, double ps, double ds, double h) {
    if (major) launch_pair<true, true>(st, P, src, tgt, ps, ds, h);
    else if (checkpoint) launch_pair<true, false>(st, P, src, tgt, ps, ds, h);
    else launch_pair<false, false>(st, P, src, tgt, ps, ds, h);
    HM_LAUNCH_CHECK("pdhg iteration");
    return HM_OK;
}

// Internal node numbers (see the header): positions by ORDER_ROUNDS rounds of neighbour averaging, then each side
// sorted by (position, caller number). Also validates the endpoints.
int number_nodes(hipStream_t st, const int64_t* rows, const int64_t* cols, int64_t n, int64_t nt, int64_t e,
                 const Pdhg& P) {
    const int64_t nodes = n + nt;
    const unsigned ge = grid_of(e), gn = grid_of(nodes);
    hipLaunchKernelGGL(k_fill_i32, dim3(gn), dim3(256), 0, st, P.odeg, nodes, 0);
    hipLaunchKernelGGL(k_order_degrees, dim3(ge), dim3(256), 0, st, rows, cols, e, n, nt, P.odeg, P.flag);
    HM_LAUNCH_CHECK("k_order_degrees");
    int bad = 0;
    HM_HIP(hipMemcpyAsync(&bad, P.flag, sizeof(int), hipMemcpyDeviceToHost, st));
    HM_HIP(hipStreamSynchronize(st));
    if (bad) return fail(HM_EINVAL, "active-support endpoint index is out of bounds");
    hipLaunchKernelGGL(k_order_seed, dim3(gn), dim3(256), 0, st, P.ov, n, nodes);
    for (int round = 0; round < ORDER_ROUNDS; ++round) {
        for (int to_sources = 1; to_sources >= 0; --to_sources) {
            hipLaunchKernelGGL(k_order_clear, dim3(gn), dim3(256), 0, st, P.osum, nodes);
            hipLaunchKernelGGL(k_order_gather, dim3(ge), dim3(256), 0, st, rows, cols, e, n, to_sources, P.ov, P.osum);
            hipLaunchKernelGGL(k_order_mean, dim3(gn), dim3(256), 0, st, P.osum, P.odeg, to_sources ? 0 : n,
                               to_sources ? n : nodes, P.ov);
        }
    }
    HM_LAUNCH_CHECK("node numbering rounds");
    for (int side = 0; side < 2; ++side) {
        const int64_t lo = side ? n : 0, count = side ? nt : n;
        hipLaunchKernelGGL(k_order_keys, dim3(grid_of(count)), dim3(256), 0, st, P.ov, lo, count, P.okeys_in);
        size_t bytes = P.osort_tmp_bytes;
        HM_HIP(hipcub::DeviceRadixSort::SortKeys(P.osort_tmp, bytes, P.okeys_in, P.okeys_out, (int)count, 0,
                                                 ORDER_KEY_BITS, st));
        hipLaunchKernelGGL(k_order_ranks, dim3(grid_of(count)), dim3(256), 0, st, P.okeys_out, count, lo,
                           side ? P.map_t : P.map_s, P.inv);
    }
    HM_LAUNCH_CHECK("node numbering sort");
    return HM_OK;
}

int read_result(hipStream_t st, const Pdhg& P, int q, double* host) {
    hipLaunchKernelGGL(k_combine, dim3(1), dim3(RT), 0, st, P.partial, P.result, q);
    HM_LAUNCH_CHECK("k_combine");
    HM_HIP(hipMemcpyAsync(host, P.result, sizeof(double) * q, hipMemcpyDeviceToHost, st));
    HM_HIP(hipStreamSynchronize(st));
    return HM_OK;
}

}  // namespace
}  // namespace hm

using namespace hm;

extern "C" size_t hm_pdhg_workspace_bytes(int64_t n_source, int64_t n_target, int64_t e) {
    if (n_source < 1 || n_target < 1 || e < 1) return 0;
    Sizer s;
    Pdhg P;
    pdhg_layout(s, n_source, n_target, e, sort_tmp_bytes(n_source + n_target, e),
                order_sort_tmp_bytes(n_source, n_target), P);
    return s.used;
}

extern "C" int hm_pdhg_solve(void* stream, const int64_t* rows, const int64_t* cols, const double* costs,
                             const double* masses, const double* x0, const double* y0, int64_t n_source,
                             int64_t n_target, int64_t e, const hm_pdhg_params* params, double* x_out, double* y_out,
                             hm_pdhg_result* result, void* workspace, size_t workspace_bytes) {
    const auto started = std::chrono::steady_clock::now();
    HM_CHECK_ARG(params && result, "PDHG: params and result are required");
    HM_CHECK_ARG(n_source >= 1 && n_target >= 1 && e >= 1, "invalid restricted OT dimensions");
    HM_CHECK_ARG(2 * e < INT32_MAX && n_source + n_target < INT32_MAX, "restricted OT too large for int32 indexing");
    HM_CHECK_ARG(rows && cols && costs && masses && x_out && y_out, "PDHG: null pointer argument");
    const int freq = params->evaluation_frequency;
    HM_CHECK_ARG(freq >= 1 && params->iteration_limit >= 1 && params->time_limit_seconds > 0,
                 "invalid restricted OT dimensions or runtime limits");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int64_t n = n_source, nt = n_target, nodes = n + nt;
    const size_t tmp = sort_tmp_bytes(nodes, e), otmp = order_sort_tmp_bytes(n, nt);
    Sizer sz;
    Pdhg P;
    pdhg_layout(sz, n, nt, e, tmp, otmp, P);
    HM_CHECK_ARG(workspace != nullptr, "workspace is required");
    if (workspace_bytes < sz.used) return fail(HM_ENOSPC, "PDHG workspace too small: %zu < %zu", workspace_bytes, sz.used);
    Arena a(workspace, workspace_bytes);
    pdhg_layout(a, n, nt, e, tmp, otmp, P);
    P.n = n;
    P.nt = nt;
    P.nodes = nodes;
    P.e = e;

    // ---- LP assembly: node numbers, endpoints, degrees, per-node incident edge lists (ascending edge id) ----
    hipLaunchKernelGGL(k_fill_i32, dim3(grid_of(nodes + 1)), dim3(256), 0, st, P.deg, nodes + 1, 0);
    hipLaunchKernelGGL(k_fill_i32, dim3(1), dim3(64), 0, st, P.flag, 4, 0);
    if (nodes >= reorder_min_nodes()) {
        if (int rc = number_nodes(st, rows, cols, n, nt, e, P)) return rc;
    } else {
        P.map_s = P.map_t = P.inv = nullptr;  // caller numbers
    }
    hipLaunchKernelGGL(k_edges, dim3(grid_of(e)), dim3(256), 0, st, rows, cols, e, n, nt, P.map_s, P.map_t, P.deg,
                       P.keys_in, P.vals_in, P.flag);
    HM_LAUNCH_CHECK("k_edges");
    hipLaunchKernelGGL(k_degree_max, dim3(grid_of(nodes)), dim3(256), 0, st, P.deg, n, nodes, P.flag);
    HM_LAUNCH_CHECK("k_degree_max");
    int flag[3] = {0, 0, 0};  // out-of-range endpoint, largest source degree, largest target degree
    HM_HIP(hipMemcpyAsync(flag, P.flag, sizeof(flag), hipMemcpyDeviceToHost, st));
    HM_HIP(hipStreamSynchronize(st));
    if (flag[0]) return fail(HM_EINVAL, "active-support endpoint index is out of bounds");
    hipLaunchKernelGGL(k_scan, dim3(1), dim3(1024), 0, st, P.deg, nodes, P.off);
    HM_LAUNCH_CHECK("k_scan");
    size_t tmp_bytes = P.sort_tmp_bytes;
    HM_HIP(hipcub::DeviceRadixSort::SortPairs(P.sort_tmp, tmp_bytes, P.keys_in, P.keys_out, P.vals_in, P.eid,
                                              (int)(2 * e), 0, end_bit_for(nodes), st));

    // ---- scaling (solver.cpp:91-110) ----
    double host[4];
    hipLaunchKernelGGL(k_sumsq, dim3(RB), dim3(RT), 0, st, masses, nodes, P.partial);
    HM_LAUNCH_CHECK("k_sumsq");
    if (int rc = read_result(st, P, 1, host)) return rc;
    const double mass_norm = std::sqrt(host[0]);
    hipLaunchKernelGGL(k_sumsq, dim3(RB), dim3(RT), 0, st, costs, e, P.partial);
    HM_LAUNCH_CHECK("k_sumsq");
    if (int rc = read_result(st, P, 1, host)) return rc;
    const double cost_norm = std::sqrt(host[0]);
    const bool rescale = params->rescale != 0;
    const double bound = rescale ? 1.0 / std::max(1.0, mass_norm) : 1.0;
    const double objective = rescale ? 1.0 / std::max(1.0, cost_norm) : 1.0;
    const double variable = std::sqrt(2.0);
    // source-order edge state and its target-order mirror
    hipLaunchKernelGGL(k_source_setup, dim3(grid_of(e)), dim3(256), 0, st, P.eid, e, rows, cols, costs, x0, bound,
                       objective, variable, P);
    HM_LAUNCH_CHECK("k_source_setup");
    hipLaunchKernelGGL(k_target_setup, dim3(grid_of(e)), dim3(256), 0, st, P.eid, e, rows, cols, costs, x0, bound,
                       objective, variable, P);
    HM_LAUNCH_CHECK("k_target_setup");
    hipLaunchKernelGGL(k_node_setup, dim3(grid_of(nodes)), dim3(256), 0, st, P.deg, masses, y0, P.inv, nodes, n, bound,
                       objective, variable, P.scale, P.bs, P.ns, P.y, P.ay, P.py, P.dy, P.td);
    HM_LAUNCH_CHECK("k_node_setup");
    double weight = 1.0;
    if (!rescale) {
        hipLaunchKernelGGL(k_sumsq, dim3(RB), dim3(RT), 0, st, P.cs, e, P.partial);
        if (int rc = read_result(st, P, 1, host)) return rc;
        const double ncs = std::sqrt(host[0]);
        hipLaunchKernelGGL(k_sumsq, dim3(RB), dim3(RT), 0, st, P.bs, nodes, P.partial);
        if (int rc = read_result(st, P, 1, host)) return rc;
        const double nbs = std::sqrt(host[0]);
        weight = std::max(ncs / std::max(nbs, 1e-16), 1e-16);
    }

    // ---- Halpern PDHG loop (solver.cpp:157-312) ----
    double best_weight = weight, error_sum = 0.0;
    const double inf = INFINITY;
    double best_balance = inf, initial_error = inf, last_trial_error = inf, fixed_error = inf;
    bool restart = false;
    int32_t reason = 0;
    int64_t count = 0, inner = 0, restarts = 0;
    double pobj = 0, dobj = 0, ap = 0, rp = 0, ad = 0, rd = 0, gap = 0;
    int64_t local_count = 0, local_inner = 0;
    const unsigned gr = grid_of(e > nodes ? e : nodes);
    const SidePlan src = side_plan(e, n, flag[1]), tgt = side_plan(e, nt, flag[2]);
    static_assert(PT <= 256, "a node's index within its block fits one byte");
    if (src.u == 0) {
        hipLaunchKernelGGL(k_low_bits, dim3(grid_of(e)), dim3(256), 0, st, P.row, e, src.npb - 1, P.loc_s);
        hipLaunchKernelGGL(k_gather_base, dim3((unsigned)((n + src.npb - 1) / src.npb)), dim3(256), 0, st, P.off, n,
                           src.npb, 0, P.col, P.gbase_s, P.g16_s);
    }
    if (tgt.u == 0) {
        hipLaunchKernelGGL(k_low_bits, dim3(grid_of(e)), dim3(256), 0, st, P.col_t, e, tgt.npb - 1, P.loc_t);
        hipLaunchKernelGGL(k_gather_base, dim3((unsigned)((nt + tgt.npb - 1) / tgt.npb)), dim3(256), 0, st, P.off + n,
                           nt, tgt.npb, (int32_t)e, P.row_t, P.gbase_t, P.g16_t);
    }
    HM_LAUNCH_CHECK("node-block setup");
    for (;;) {
        if (local_count % freq == 0) {
            hipLaunchKernelGGL(k_evaluate, dim3(RB), dim3(RT), 0, st, P, masses, costs, variable, bound, objective,
                               P.partial);
            HM_LAUNCH_CHECK("k_evaluate");
            if (int rc = read_result(st, P, 4, host)) return rc;
            count = local_count;
            inner = local_inner;
            ap = std::sqrt(host[0]);
            dobj = host[1];
            ad = std::sqrt(host[2]);
            pobj = host[3];
            rp = ap / (1.0 + mass_norm);
            rd = ad / (1.0 + cost_norm);
            gap = std::fabs(pobj - dobj) / (1.0 + std::fabs(pobj) + std::fabs(dobj));
            const bool finite = std::isfinite(pobj) && std::isfinite(dobj) && std::isfinite(ap) && std::isfinite(rp) &&
                                std::isfinite(ad) && std::isfinite(rd) && std::isfinite(gap);
            const double elapsed = std::chrono::duration<double>(std::chrono::steady_clock::now() - started).count();
            if (!finite || !std::isfinite(weight)) reason = 3;
            else if (rp < params->tol_primal && rd < params->tol_dual && gap < params->tol_objective) reason = 1;
            else if (count >= params->iteration_limit) reason = 2;
            else if (elapsed >= params->time_limit_seconds) reason = 4;
            if (reason != 0) break;
            restart = false;
            if (count == freq) restart = true;
            else if (count > freq)
                restart = inner >= 0.36 * count || fixed_error <= 0.2 * initial_error ||
                          (fixed_error <= 0.5 * initial_error && fixed_error > last_trial_error);
            last_trial_error = fixed_error;
            if (restart) {
                hipLaunchKernelGGL(k_diffsq2, dim3(RB), dim3(RT), 0, st, P.px, P.ax, e, P.py, P.ay, nodes, P.partial);
                HM_LAUNCH_CHECK("k_diffsq2");
                if (int rc = read_result(st, P, 2, host)) return rc;
                const double pd = std::sqrt(host[0]), dd = std::sqrt(host[1]);
                const double ratio = rd / std::max(rp, 1e-300);
                if (pd > 1e-16 && pd < 1e12 && dd > 1e-16 && dd < 1e12 && ratio > 1e-8 && ratio < 1e8) {
                    const double error = std::log(dd) - std::log(pd) - std::log(weight);
                    error_sum = 0.3 * error_sum + error;
                    weight *= std::exp(0.99 * error + 0.01 * error_sum);
                } else {
                    weight = best_weight;
                    error_sum = 0;
                }
                if (rp > 0 && rd > 0) {
                    const double balance = std::fabs(std::log10(rd / rp));
                    if (balance < best_balance) {
                        best_balance = balance;
                        best_weight = weight;
                    }
                }
                inner = 0;
                last_trial_error = inf;
                ++restarts;
                hipLaunchKernelGGL(k_restart, dim3(gr), dim3(256), 0, st, P);
                HM_LAUNCH_CHECK("k_restart");
                local_inner = 0;
            }
        }
        const double primal_step = 0.998 / weight;
        const double dual_step = 0.998 * weight;
        const double halpern = double(local_inner + 1) / double(local_inner + 2);
        const bool major = ((local_count + 1) % freq) == 0;
        const bool is_restart = (local_count % freq == 0) && restart;
        const bool checkpoint = major || is_restart;
        // px / py are read only by the evaluation that follows a major iteration
        prof_begin(st, "pdhg_iteration");
        if (int rc = launch_iteration(st, P, src, tgt, checkpoint, major, primal_step, dual_step, halpern)) return rc;
        prof_end(st);
        HM_LAUNCH_CHECK("pdhg iteration");
        if (checkpoint) {
            hipLaunchKernelGGL(k_fixed_point, dim3(RB), dim3(RT), 0, st, P, P.partial);
            HM_LAUNCH_CHECK("k_fixed_point");
            if (int rc = read_result(st, P, 3, host)) return rc;
            const double squared = host[0] * weight + host[1] / weight + 2.0 * 0.998 * host[2];
            fixed_error = std::sqrt(std::max(0.0, squared));
            if (is_restart) initial_error = fixed_error;
        }
        ++local_count;
        ++local_inner;
    }
    hipLaunchKernelGGL(k_output, dim3(gr), dim3(256), 0, st, P, variable * bound, objective, x_out, y_out);
    HM_LAUNCH_CHECK("k_output");
    HM_HIP(hipStreamSynchronize(st));
    result->iterations = count;
    result->restarts = restarts;
    result->reason = reason;
    result->pad = 0;
    result->primal_objective = pobj;
    result->dual_objective = dobj;
    result->abs_primal = ap;
    result->rel_primal = rp;
    result->abs_dual = ad;
    result->rel_dual = rd;
    result->rel_gap = gap;
    result->primal_weight = weight;
    result->seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - started).count();
    return HM_OK;
}
