/*
 * CPU oracle for the HELLO hot path (pricing scan, SDDMM, restricted-LP Halpern-PDHG).
 *
 * TEST INFRASTRUCTURE ONLY. This file is a plain-C restatement of the reference algorithm and is the
 * checker the GPU path is compared against. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library never links or calls it.
 *
 * Arithmetic contract (what "bit-exact" means for the floating-point parts):
 *
 *  dot64(x, y)  -- fp64 dot product of two fp32 rows in a fixed order: 64 "lane" partial sums,
 *                  lane l accumulates (double)x[64t+l]*(double)y[64t+l] for t = 0,1,... sequentially,
 *                  then a pairwise tree with halving stride (lane l += lane l+s for s = 32,16,...,1).
 *                  fp32*fp32 products are exact in fp64, so FMA contraction cannot change a bit.
 *                  The reference ranks by an fp32 SGEMM dot (cost.cu:202-220, pricing_small.cu:241-256)
 *                  whose rounding is cuBLAS-specific; this oracle fixes the fp64 order instead, and the
 *                  GPU kernels re-evaluate every reported candidate in exactly this order.
 *  l2sq score   -- sigma_ij = (scale*dot64 + qb_i) + db_j, the reference's raw association
 *                  (matrix_selection.cuh:23, pricing.cu:114-116) with qb = f - p and db = g - q.
 *  l2sq cost    -- c_ij = (p_i + q_j) - scale*dot64 (matrix_selection.cuh:23; gpu_resident/cost.py:59-71).
 *  norm cost    -- fp32 distance accumulated sequentially inside 32-feature chunks that are then added in
 *                  order (pricing.cu:89-103 and cost.cu:20-77 with F=32): l1 sum|x-y|, linf max|x-y|,
 *                  l2 sqrtf(sum fmaf(z,z,.)) (nvcc contracts a+z*z, pricing.cu:65-70); the score is
 *                  (g_j - (double)c) + f_i (pricing.cu:113, matrix_selection.cuh:25).
 *  norm cost64  -- compute_precision = 1 (generic_scan.py:166-167 -> direct_norm_fp64, cost.cu:84-104, which
 *                  instantiates direct_norm_kernel with one chain and a double accumulator, cost.cu:10-80): each
 *                  difference (double)x - (double)y, the features combined one after another in order (l1 sum|z|,
 *                  linf max|z|, l2 sum z*z contracted to fma(z,z,acc) by nvcc, then sqrt); same score association.
 *  tie rule     -- better(a,b) = a.v > b.v || (a.v == b.v && a.i < b.i); -0 == +0; NaN never enters
 *                  (pricing.cu:38-51). Missing slots hold (-inf, -1).
 *  pair costs   -- fp64 norms of fp32 rows for the sparse support (norm_cost_scan_kernel.cu:233-245):
 *                  per-lane fp64 partials in the dot64 lane layout and the same tree.
 *  PDHG         -- restatement of _native/cpp/solver.cpp:39-378 with the reference's one-thread summation
 *                  order: only the per-node passes run in parallel (disjoint writes), every reduction is serial.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <float.h>

#define LANES 64

static double dot64(const float* x, const float* y, int64_t d) {
    double acc[LANES];
    for (int l = 0; l < LANES; ++l) acc[l] = 0.0;
    /* lane l accumulates features l, l+64, l+128, ... in order; the lanes are independent, so the compiler may
       vectorise across them without changing any lane's order */
    int64_t t = 0;
    for (; t + LANES <= d; t += LANES)
        for (int l = 0; l < LANES; ++l) acc[l] = acc[l] + (double)x[t + l] * (double)y[t + l];
    for (int l = 0; t + l < d; ++l) acc[l] = acc[l] + (double)x[t + l] * (double)y[t + l];
    for (int s = LANES / 2; s >= 1; s >>= 1)
        for (int l = 0; l < s; ++l) acc[l] = acc[l] + acc[l + s];
    return acc[0];
}

double orc_dot64(const float* x, const float* y, int64_t d) { return dot64(x, y, d); }

/* Full l2^2 score and cost matrices (m x n, row-major). Inputs are small test cases. */
void orc_l2sq_matrices(const float* X, const float* Y, const double* p, const double* q,
                       const double* qb, const double* db, int64_t m, int64_t n, int64_t d,
                       double scale, double* sigma, double* cost) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < m; ++i) {
        for (int64_t j = 0; j < n; ++j) {
            const double dot = dot64(X + i * d, Y + j * d, d);
            const double s = scale * dot;
            if (sigma) sigma[i * n + j] = (s + qb[i]) + db[j];
            if (cost) cost[i * n + j] = (p[i] + q[j]) - s;
        }
    }
}

static float norm_distance(const float* x, const float* y, int64_t d, int kind) {
    float acc = 0.0f;
    for (int64_t base = 0; base < d; base += 32) {
        float part = 0.0f;
        const int64_t end = base + 32 < d ? base + 32 : d;
        for (int64_t k = base; k < end; ++k) {
            const float z = x[k] - y[k];
            if (kind == 0) part = part + fabsf(z);
            else if (kind == 1) part = fmaxf(part, fabsf(z));
            else part = fmaf(z, z, part);
        }
        acc = kind == 1 ? fmaxf(acc, part) : acc + part;
    }
    return kind == 2 ? sqrtf(acc) : acc;
}

/* Norm score/cost matrices: cost = fp32 distance, sigma = (g_j - cost) + f_i. kind 0=l1, 1=linf, 2=l2. */
void orc_norm_matrices(const float* X, const float* Y, const double* f, const double* g,
                       int64_t m, int64_t n, int64_t d, int kind, double* sigma, double* cost) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < m; ++i) {
        for (int64_t j = 0; j < n; ++j) {
            const double c = (double)norm_distance(X + i * d, Y + j * d, d, kind);
            if (sigma) sigma[i * n + j] = (g[j] - c) + f[i];
            if (cost) cost[i * n + j] = c;
        }
    }
}

static double norm_distance64(const float* x, const float* y, int64_t d, int kind) {
    double acc = 0.0;
    for (int64_t k = 0; k < d; ++k) {
        const double z = (double)x[k] - (double)y[k];
        if (kind == 0) acc = acc + fabs(z);
        else if (kind == 1) acc = fmax(acc, fabs(z));
        else acc = fma(z, z, acc);
    }
    return kind == 2 ? sqrt(acc) : acc;
}

/* As orc_norm_matrices with fp64 costs (compute_precision = 1, cost.cu:84-104). */
void orc_norm_matrices64(const float* X, const float* Y, const double* f, const double* g,
                         int64_t m, int64_t n, int64_t d, int kind, double* sigma, double* cost) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < m; ++i) {
        for (int64_t j = 0; j < n; ++j) {
            const double c = norm_distance64(X + i * d, Y + j * d, d, kind);
            if (sigma) sigma[i * n + j] = (g[j] - c) + f[i];
            if (cost) cost[i * n + j] = c;
        }
    }
}

static int better(double a, int32_t ai, double b, int32_t bi) {
    if (a > b) return 1;
    if (a == b && ai >= 0 && (bi < 0 || ai < bi)) return 1;
    return 0;
}

static void put(double* v, int32_t* idx, int k, double value, int32_t index) {
    if (!better(value, index, v[k - 1], idx[k - 1])) return;
    int p = k - 1;
    while (p > 0 && better(value, index, v[p - 1], idx[p - 1])) {
        v[p] = v[p - 1];
        idx[p] = idx[p - 1];
        --p;
    }
    v[p] = value;
    idx[p] = index;
}

/* Row-wise (transpose=0) or column-wise (transpose=1) top-k of a dense m x n score matrix. */
void orc_topk(const double* sigma, int64_t m, int64_t n, int k, int transpose,
              double* vals, int32_t* idx) {
    const int64_t outer = transpose ? n : m, inner = transpose ? m : n;
    #pragma omp parallel for schedule(static)
    for (int64_t o = 0; o < outer; ++o) {
        double* v = vals + o * k;
        int32_t* id = idx + o * k;
        for (int j = 0; j < k; ++j) { v[j] = -INFINITY; id[j] = -1; }
        for (int64_t t = 0; t < inner; ++t) {
            const double s = transpose ? sigma[t * n + o] : sigma[o * n + t];
            if (s != s) continue;
            put(v, id, k, s, (int32_t)t);
        }
    }
}

/* Certificate statistics over the dense matrices: num = sum sigma+^2, den = sum cost^2, count = #{sigma>0},
 * max = max sigma+, costmax = max|cost| (pricing.cu:120-123; scan.cpp:189-196). Row partials are added in
 * row order so the result is deterministic. */
void orc_stats(const double* sigma, const double* cost, int64_t m, int64_t n, double* out5) {
    double* part = (double*)calloc((size_t)m * 5, sizeof(double));
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < m; ++i) {
        double num = 0, den = 0, cnt = 0, mx = 0, cm = 0;
        for (int64_t j = 0; j < n; ++j) {
            const double s = sigma[i * n + j], c = cost[i * n + j];
            den += c * c;
            cm = fmax(cm, fabs(c));
            if (s > 0) { num += s * s; mx = fmax(mx, s); cnt += 1; }
        }
        part[i * 5 + 0] = num; part[i * 5 + 1] = den; part[i * 5 + 2] = cnt;
        part[i * 5 + 3] = mx; part[i * 5 + 4] = cm;
    }
    double num = 0, den = 0, cnt = 0, mx = 0, cm = 0;
    for (int64_t i = 0; i < m; ++i) {
        num += part[i * 5]; den += part[i * 5 + 1]; cnt += part[i * 5 + 2];
        mx = fmax(mx, part[i * 5 + 3]); cm = fmax(cm, part[i * 5 + 4]);
    }
    out5[0] = num; out5[1] = den; out5[2] = cnt; out5[3] = mx; out5[4] = cm;
    free(part);
}

/* SDDMM on a CSR support: c_e = (p_i + q_j) - scale*dot64(x_i, y_j) (pairs.py:394-407 association). */
void orc_sddmm_l2sq(const float* X, const float* Y, const double* p, const double* q,
                    const int32_t* rowptr, const int32_t* col, int64_t m, int64_t d, double scale,
                    double* out) {
    #pragma omp parallel for schedule(dynamic, 64)
    for (int64_t i = 0; i < m; ++i) {
        for (int64_t e = rowptr[i]; e < rowptr[i + 1]; ++e) {
            const int64_t j = col[e];
            out[e] = (p[i] + q[j]) - scale * dot64(X + i * d, Y + j * d, d);
        }
    }
}

/* Sparse fp64 norm pair costs: kind 0=l1, 1=linf, 2=l2 (norm_cost_scan_kernel.cu:233-245). */
void orc_pair_costs_norm(const float* X, const float* Y, const int64_t* rows, const int64_t* cols,
                         int64_t count, int64_t d, int kind, double* out) {
    #pragma omp parallel for schedule(static)
    for (int64_t e = 0; e < count; ++e) {
        const float* x = X + rows[e] * d;
        const float* y = Y + cols[e] * d;
        double acc[LANES];
        for (int l = 0; l < LANES; ++l) acc[l] = 0.0;
        for (int64_t k = 0; k < d; ++k) {
            const double z = (double)x[k] - (double)y[k];
            const int l = (int)(k % LANES);
            if (kind == 0) acc[l] = acc[l] + fabs(z);
            else if (kind == 1) acc[l] = fmax(acc[l], fabs(z));
            else acc[l] = acc[l] + z * z;
        }
        for (int s = LANES / 2; s >= 1; s >>= 1)
            for (int l = 0; l < s; ++l) acc[l] = kind == 1 ? fmax(acc[l], acc[l + s]) : acc[l] + acc[l + s];
        out[e] = kind == 2 ? sqrt(acc[0]) : acc[0];
    }
}

/* ------------------------------------------------------------------------------------------------ */
/* Halpern-reflected PDHG for the balanced restricted OT LP, single-thread restatement of            */
/* _native/cpp/solver.cpp:39-378 (and _internal/lp/torch_restricted_ot.py:105-393).                   */
/* Variables x_e >= 0 (one per support edge e=(rows[e], cols[e])), constraints: source marginals then  */
/* target marginals (nodes = n_source + n_target). Degree-sqrt constraint scaling, variable scale √2. */
/* ------------------------------------------------------------------------------------------------ */

typedef struct {
    int64_t iterations;
    int64_t restarts;
    int32_t reason; /* 0 UNSPECIFIED, 1 OPTIMAL, 2 ITERATION_LIMIT, 3 NUMERICAL_DIVERGENCE */
    int32_t pad;
    double pobj, dobj, ap, rp, ad, rd, gap, weight;
} orc_pdhg_info;

static double vnorm(const double* x, int64_t n) {
    double s = 0.0;
    for (int64_t i = 0; i < n; ++i) s += x[i] * x[i];
    return sqrt(s);
}

int orc_pdhg_solve(const int64_t* rows, const int64_t* cols, const double* c, const double* b,
                   int64_t n_source, int64_t n_target, int64_t e, const double* initial_x,
                   const double* initial_y, int frequency, int64_t iteration_limit, double tol_objective,
                   double tol_primal, double tol_dual, int rescale, double* output_x, double* output_y,
                   orc_pdhg_info* info) {
    const int64_t n = n_source, nodes = n_source + n_target;
    if (n < 1 || n_target < 1 || e < 1 || frequency < 1 || iteration_limit < 1) return -1;
    for (int64_t j = 0; j < e; ++j)
        if (rows[j] < 0 || rows[j] >= n || cols[j] < 0 || cols[j] >= n_target) return -2;
    int64_t* offsets = (int64_t*)calloc((size_t)nodes + 1, sizeof(int64_t));
    int64_t* cursor = (int64_t*)calloc((size_t)nodes + 1, sizeof(int64_t));
    int64_t* edge_ids = (int64_t*)malloc(sizeof(int64_t) * 2 * (size_t)e);
    double* scale = (double*)malloc(sizeof(double) * nodes);
    for (int64_t j = 0; j < e; ++j) { ++offsets[rows[j] + 1]; ++offsets[n + cols[j] + 1]; }
    for (int64_t i = 0; i < nodes; ++i) scale[i] = sqrt((double)(offsets[i + 1] > 1 ? offsets[i + 1] : 1));
    for (int64_t i = 0; i < nodes; ++i) offsets[i + 1] += offsets[i];
    memcpy(cursor, offsets, sizeof(int64_t) * (nodes + 1));
    for (int64_t j = 0; j < e; ++j) { edge_ids[cursor[rows[j]]++] = j; edge_ids[cursor[n + cols[j]]++] = j; }
    const double mass_norm = vnorm(b, nodes), cost_norm = vnorm(c, e);
    const double bound = rescale ? 1.0 / fmax(1.0, mass_norm) : 1.0;
    const double objective = rescale ? 1.0 / fmax(1.0, cost_norm) : 1.0;
    const double variable = sqrt(2.0);
    double* cs = (double*)malloc(sizeof(double) * e);
    double* ax = (double*)malloc(sizeof(double) * e);
    double* x = (double*)malloc(sizeof(double) * e);
    double* px = (double*)malloc(sizeof(double) * e);
    double* rx = (double*)malloc(sizeof(double) * e);
    double* dx = (double*)malloc(sizeof(double) * e);
    double* bs = (double*)malloc(sizeof(double) * nodes);
    double* ns = (double*)malloc(sizeof(double) * nodes);
    double* ay = (double*)malloc(sizeof(double) * nodes);
    double* y = (double*)malloc(sizeof(double) * nodes);
    double* py = (double*)malloc(sizeof(double) * nodes);
    double* dy = (double*)malloc(sizeof(double) * nodes);
    double* td = (double*)malloc(sizeof(double) * n_target);
    for (int64_t j = 0; j < e; ++j) {
        cs[j] = c[j] * objective / variable;
        ax[j] = fmax(initial_x[j], 0.0) * variable * bound;
    }
    for (int64_t i = 0; i < nodes; ++i) {
        bs[i] = b[i] * bound / scale[i];
        ns[i] = variable * scale[i];
        ay[i] = initial_y[i] * scale[i] * objective;
    }
    memcpy(x, ax, sizeof(double) * e); memcpy(px, ax, sizeof(double) * e);
    memcpy(y, ay, sizeof(double) * nodes); memcpy(py, ay, sizeof(double) * nodes);
    memset(dx, 0, sizeof(double) * e); memset(dy, 0, sizeof(double) * nodes); memset(rx, 0, sizeof(double) * e);
    for (int64_t j = 0; j < n_target; ++j) td[j] = y[n + j] / ns[n + j];
    double weight = rescale ? 1.0 : fmax(vnorm(cs, e) / fmax(vnorm(bs, nodes), 1e-16), 1e-16);
    double best_weight = weight, error_sum = 0.0;
    const double inf = INFINITY;
    double best_balance = inf, initial_error = inf, last_trial_error = inf, fixed_error = inf;
    int restart = 0;
    int32_t reason = 0;
    int64_t count = 0, inner = 0, restarts = 0;
    double pobj = 0, dobj = 0, ap = 0, rp = 0, ad = 0, rd = 0, gap = 0;
    int64_t local_count = 0, local_inner = 0;
    for (;;) {
        if (local_count % frequency == 0) {
            double primal_sq = 0, dual_sq = 0;
            pobj = 0; dobj = 0;
            for (int64_t i = 0; i < nodes; ++i) {
                double sum = 0;
                for (int64_t k = offsets[i]; k < offsets[i + 1]; ++k) sum += px[edge_ids[k]] / (variable * bound);
                const double delta = sum - b[i];
                primal_sq += delta * delta;
                dobj += b[i] * (py[i] / (scale[i] * objective));
            }
            for (int64_t j = 0; j < e; ++j) {
                const double score = py[rows[j]] / (scale[rows[j]] * objective)
                    + py[n + cols[j]] / (scale[n + cols[j]] * objective) - c[j];
                const double violation = fmax(score, 0.0);
                dual_sq += violation * violation;
                pobj += c[j] * (px[j] / (variable * bound));
            }
            count = local_count;
            inner = local_inner;
            ap = sqrt(primal_sq);
            ad = sqrt(dual_sq);
            rp = ap / (1.0 + mass_norm);
            rd = ad / (1.0 + cost_norm);
            gap = fabs(pobj - dobj) / (1.0 + fabs(pobj) + fabs(dobj));
            const int finite = isfinite(pobj) && isfinite(dobj) && isfinite(ap) && isfinite(rp)
                && isfinite(ad) && isfinite(rd) && isfinite(gap);
            if (!finite || !isfinite(weight)) reason = 3;
            else if (rp < tol_primal && rd < tol_dual && gap < tol_objective) reason = 1;
            else if (count >= iteration_limit) reason = 2;
            if (reason != 0) break;
            restart = 0;
            if (count == frequency) restart = 1;
            else if (count > frequency)
                restart = inner >= 0.36 * count || fixed_error <= 0.2 * initial_error
                    || (fixed_error <= 0.5 * initial_error && fixed_error > last_trial_error);
            last_trial_error = fixed_error;
            if (restart) {
                double pd = 0, dd = 0;
                for (int64_t j = 0; j < e; ++j) { const double t = px[j] - ax[j]; pd += t * t; }
                for (int64_t i = 0; i < nodes; ++i) { const double t = py[i] - ay[i]; dd += t * t; }
                pd = sqrt(pd);
                dd = sqrt(dd);
                const double ratio = rd / fmax(rp, 1e-300);
                if (pd > 1e-16 && pd < 1e12 && dd > 1e-16 && dd < 1e12 && ratio > 1e-8 && ratio < 1e8) {
                    const double error = log(dd) - log(pd) - log(weight);
                    error_sum = 0.3 * error_sum + error;
                    weight *= exp(0.99 * error + 0.01 * error_sum);
                } else {
                    weight = best_weight;
                    error_sum = 0;
                }
                if (rp > 0 && rd > 0) {
                    const double balance = fabs(log10(rd / rp));
                    if (balance < best_balance) { best_balance = balance; best_weight = weight; }
                }
                inner = 0;
                last_trial_error = inf;
                ++restarts;
                for (int64_t j = 0; j < e; ++j) ax[j] = x[j] = px[j];
                for (int64_t i = 0; i < nodes; ++i) {
                    ay[i] = y[i] = py[i];
                    if (i >= n) td[i - n] = y[i] / ns[i];
                }
                local_inner = 0;
            }
        }
        const double primal_step = 0.998 / weight;
        const double dual_step = 0.998 * weight;
        const double halpern = (double)(local_inner + 1) / (double)(local_inner + 2);
        const int major = ((local_count + 1) % frequency) == 0;
        const int is_restart = (local_count % frequency == 0) && restart;
        const int checkpoint = major || is_restart;
        /* Node passes: every edge belongs to exactly one source and one target, so the iterations of each pass
           write disjoint entries and threads cannot change a single bit of the result. */
        #pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < n; ++i) {
            const double source_dual = y[i] / ns[i];
            double sum = 0.0;
            for (int64_t k = offsets[i]; k < offsets[i + 1]; ++k) {
                const int64_t j = edge_ids[k];
                const double at = source_dual + td[cols[j]];
                px[j] = fmax(x[j] - primal_step * (cs[j] - at), 0.0);
                rx[j] = 2.0 * px[j] - x[j];
                if (checkpoint) dx[j] = rx[j] - x[j];
                x[j] = halpern * rx[j] + (1.0 - halpern) * ax[j];
                sum += rx[j];
            }
            py[i] = y[i] - dual_step * (sum / ns[i] - bs[i]);
            const double reflected = 2.0 * py[i] - y[i];
            if (checkpoint) dy[i] = reflected - y[i];
            y[i] = halpern * reflected + (1.0 - halpern) * ay[i];
        }
        #pragma omp parallel for schedule(static)
        for (int64_t i = n; i < nodes; ++i) {
            double sum = 0.0;
            for (int64_t k = offsets[i]; k < offsets[i + 1]; ++k) sum += rx[edge_ids[k]];
            py[i] = y[i] - dual_step * (sum / ns[i] - bs[i]);
            const double reflected = 2.0 * py[i] - y[i];
            if (checkpoint) dy[i] = reflected - y[i];
            y[i] = halpern * reflected + (1.0 - halpern) * ay[i];
            td[i - n] = y[i] / ns[i];
        }
        if (checkpoint) {
            double movement = 0, dual_movement = 0, interaction = 0;
            for (int64_t j = 0; j < e; ++j) {
                movement += dx[j] * dx[j];
                interaction += (dy[rows[j]] / ns[rows[j]] + dy[n + cols[j]] / ns[n + cols[j]]) * dx[j];
            }
            for (int64_t i = 0; i < nodes; ++i) dual_movement += dy[i] * dy[i];
            const double squared = movement * weight + dual_movement / weight + 2.0 * 0.998 * interaction;
            fixed_error = sqrt(fmax(0.0, squared));
            if (is_restart) initial_error = fixed_error;
        }
        ++local_count;
        ++local_inner;
    }
    for (int64_t j = 0; j < e; ++j) output_x[j] = px[j] / (variable * bound);
    for (int64_t i = 0; i < nodes; ++i) output_y[i] = py[i] / (scale[i] * objective);
    info->iterations = count;
    info->restarts = restarts;
    info->reason = reason;
    info->pobj = pobj; info->dobj = dobj; info->ap = ap; info->rp = rp; info->ad = ad; info->rd = rd;
    info->gap = gap; info->weight = weight;
    free(offsets); free(cursor); free(edge_ids); free(scale); free(cs); free(ax); free(x); free(px);
    free(rx); free(dx); free(bs); free(ns); free(ay); free(y); free(py); free(dy); free(td);
    return 0;
}
