// Exact solve of a small dense balanced transport problem by the primal network simplex (host code).
//
// HELLO solves its coarsest level exactly (the reference calls POT's emd, a network simplex, on the CPU:
// gpu_resident/solver.py:168-191, hierarchy/coarsest.py:38-60); this is this library's own solver for that step.
//
//   min sum_ij c_ij x_ij  s.t.  sum_j x_ij = a_i,  sum_i x_ij = b_j,  x >= 0     (dense c, n x m)
//
// Network: sources 0..n-1, targets n..n+m-1 and a root R = n+m. The transport arcs i -> n+j have infinite
// capacity. The start basis is the star of artificial arcs i -> R (flow a_i) and R -> n+j (flow b_j) with cost
// BIG; every tree arc then carries positive flow, so the tree is strongly feasible (Cunningham) and stays so:
// the leaving arc is the last blocking arc of the cycle met from its apex in the direction of the push, which
// rules out cycling on degenerate pivots.
//
// BIG is symbolic (the big-M method): a potential is k * BIG + r with an integer k (artificial arcs on the tree
// path to the root, with their orientation) and a double r (the transport costs on that path), and reduced costs
// compare lexicographically, first by their BIG multiple and then by their remainder. No value ever carries a
// rounding error at the scale of BIG, so the entering threshold eps sits far above the rounding of the remainders
// (sums of at most n + m costs) at every problem size.
//
// Pricing: block search over the n*m arcs (blocks of about sqrt(n*m)), the most negative reduced cost of the
// first block that has one below -eps enters. Tree: parent, the arc to the parent, its orientation, depth, and
// child lists; a pivot re-hangs the subtree cut off by the leaving arc and recomputes its depths and potentials
// from its new parent.
//
// Duals: with potentials pi (c_a + pi_tail - pi_head = 0 on tree arcs), u_i = -pi_i and v_j = pi_{n+j} satisfy
// u_i + v_j = c_ij on basic transport arcs and <= c_ij everywhere (the optimality test); they are returned centered
// (u + t, v - t with sum a u = sum b v), which changes no u_i + v_j. If degenerate artificial
// arcs are still basic at the end, the transport arcs of the basis form several components whose potentials differ
// by multiples of BIG; each component is then shifted (sources +s, targets -s, which keeps its equalities) by the
// shortest-path distances over the components with edge weights min reduced cost between them, which keeps every
// reduced cost nonnegative and makes at least one arc into each component tight.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <vector>

#include "../../include/helloot_hip.h"

namespace hm {
int fail(int code, const char* fmt, ...);
}

namespace {

constexpr int UP = 1;     // the tree arc to the parent is oriented child -> parent
constexpr int DOWN = -1;  // ... parent -> child

struct Simplex {
    int n, m, V, root;
    const double* c;
    std::vector<int> parent, pred_arc, dir, depth;
    std::vector<double> flow_up;   // flow of the tree arc to the parent
    std::vector<int> kbig;         // potential = kbig * BIG + rem
    std::vector<double> rem;
    std::vector<std::vector<int>> children;
    std::vector<int> child_slot;   // position of a node in its parent's child list

    // arc ids: transport i*m + j; artificial source i: n*m + i; artificial target j: n*m + n + j
    int64_t art_base() const { return (int64_t)n * m; }
    bool artificial(int64_t a) const { return a >= art_base(); }

    void attach(int x, int p) {
        child_slot[x] = (int)children[p].size();
        children[p].push_back(x);
    }
    void detach(int x) {
        auto& list = children[parent[x]];
        const int slot = child_slot[x];
        const int last = list.back();
        list[slot] = last;
        child_slot[last] = slot;
        list.pop_back();
    }

    // depths and potentials of the subtree under `top` from its parent's
    void refresh(int top, std::vector<int>& stack) {
        stack.clear();
        stack.push_back(top);
        while (!stack.empty()) {
            const int x = stack.back();
            stack.pop_back();
            const int p = parent[x];
            depth[x] = depth[p] + 1;
            // tree arc (tail -> head): c + pi_tail - pi_head = 0, the artificial cost counted in kbig
            const int sign = dir[x] == UP ? -1 : 1;
            if (artificial(pred_arc[x])) {
                kbig[x] = kbig[p] + sign;
                rem[x] = rem[p];
            } else {
                kbig[x] = kbig[p];
                rem[x] = sign < 0 ? rem[p] - c[pred_arc[x]] : rem[p] + c[pred_arc[x]];
            }
            for (int ch : children[x]) stack.push_back(ch);
        }
    }
};

}  // namespace

extern "C" int hm_transport_simplex(int64_t n_source, int64_t n_target, const double* costs, const double* a,
                                    const double* b, int64_t max_pivots, int32_t* basis_rows, int32_t* basis_cols,
                                    double* basis_flows, int64_t* basis_count, double* u, double* v,
                                    int64_t* pivots_out) {
    if (n_source < 1 || n_target < 1 || n_source > (1 << 20) || n_target > (1 << 20) ||
        n_source * n_target > (int64_t(1) << 31) || !costs || !a || !b || !basis_rows || !basis_cols ||
        !basis_flows || !basis_count || !u || !v)
        return hm::fail(HM_EINVAL, "transport simplex: invalid sizes or pointers (n=%lld m=%lld)",
                            (long long)n_source, (long long)n_target);
    const int n = (int)n_source, m = (int)n_target;
    double cmax = 0.0;
    for (int64_t e = 0; e < (int64_t)n * m; ++e) {
        if (!std::isfinite(costs[e])) return hm::fail(HM_EINVAL, "transport simplex: costs must be finite");
        cmax = std::max(cmax, std::fabs(costs[e]));
    }
    double sa = 0.0, sb = 0.0;
    for (int i = 0; i < n; ++i) {
        if (!(a[i] >= 0.0) || !std::isfinite(a[i])) return hm::fail(HM_EINVAL, "transport simplex: bad source mass");
        sa += a[i];
    }
    for (int j = 0; j < m; ++j) {
        if (!(b[j] >= 0.0) || !std::isfinite(b[j])) return hm::fail(HM_EINVAL, "transport simplex: bad target mass");
        sb += b[j];
    }
    if (std::fabs(sa - sb) > 1e-9 * std::max(1.0, std::max(sa, sb)))
        return hm::fail(HM_EINVAL, "transport simplex: unbalanced masses (%.17g vs %.17g)", sa, sb);

    Simplex s;
    s.n = n;
    s.m = m;
    s.V = n + m + 1;
    s.root = n + m;
    s.c = costs;
    s.parent.assign(s.V, -1);
    s.pred_arc.assign(s.V, -1);
    s.dir.assign(s.V, 0);
    s.depth.assign(s.V, 0);
    s.flow_up.assign(s.V, 0.0);
    s.kbig.assign(s.V, 0);
    s.rem.assign(s.V, 0.0);
    s.children.assign(s.V, {});
    s.child_slot.assign(s.V, 0);
    for (int i = 0; i < n; ++i) {
        s.parent[i] = s.root;
        s.pred_arc[i] = (int)(s.art_base() + i);
        s.dir[i] = UP;
        s.flow_up[i] = a[i];
        s.depth[i] = 1;
        s.kbig[i] = -1;
        s.attach(i, s.root);
    }
    for (int j = 0; j < m; ++j) {
        const int x = n + j;
        s.parent[x] = s.root;
        s.pred_arc[x] = (int)(s.art_base() + n + j);
        s.dir[x] = DOWN;
        s.flow_up[x] = b[j];
        s.depth[x] = 1;
        s.kbig[x] = 1;
        s.attach(x, s.root);
    }

    const int64_t arcs = (int64_t)n * m;
    const int64_t block = std::max<int64_t>(16, (int64_t)std::sqrt((double)arcs));
    // entering threshold, against the rounding of the remainders (tree-path sums of costs)
    const double eps = 1e-12 * (cmax + 1.0);
    int64_t next = 0, pivots = 0;
    std::vector<int> stack;
    stack.reserve(s.V);
    for (;;) {
        // --- pricing: block search ---
        int64_t enter = -1;
        int best_k = 0;         // best reduced cost so far: best_k * BIG + best_r, below (0, -eps)
        double best_r = -eps;
        int64_t scanned = 0;
        while (scanned < arcs) {
            const int64_t stop = std::min<int64_t>(scanned + block, arcs);
            for (int64_t t = scanned; t < stop; ++t) {
                int64_t e = next + t;
                if (e >= arcs) e -= arcs;
                const int i = (int)(e / m), j = (int)(e - (int64_t)i * m);
                const int rk = s.kbig[i] - s.kbig[n + j];
                const double rr = costs[e] + s.rem[i] - s.rem[n + j];
                if (rk < best_k || (rk == best_k && rr < best_r)) {
                    best_k = rk;
                    best_r = rr;
                    enter = e;
                }
            }
            scanned = stop;
            if (enter >= 0) break;
        }
        if (enter < 0) break;  // optimal
        next = (next + scanned) % arcs;
        if (++pivots > max_pivots)
            return hm::fail(HM_ESOLVE, "transport simplex: no optimum within %lld pivots", (long long)max_pivots);
        const int ui = (int)(enter / m), vj = n + (int)(enter - (int64_t)ui * m);
        // --- cycle: apex and the leaving arc (last blocking arc from the apex in the push direction) ---
        int x = ui, y = vj;
        while (s.depth[x] > s.depth[y]) x = s.parent[x];
        while (s.depth[y] > s.depth[x]) y = s.parent[y];
        while (x != y) {
            x = s.parent[x];
            y = s.parent[y];
        }
        const int apex = x;
        double delta = std::numeric_limits<double>::infinity();
        int out = -1;
        bool out_first = true;
        // first side (ui up to the apex): the push runs parent -> child, so UP arcs lose flow; strict < keeps
        // the blocking arc nearest ui, i.e. the last one met from the apex
        for (int w = ui; w != apex; w = s.parent[w]) {
            if (s.dir[w] == UP && s.flow_up[w] < delta) {
                delta = s.flow_up[w];
                out = w;
                out_first = true;
            }
        }
        // second side (vj up to the apex): the push runs child -> parent, so DOWN arcs lose flow; <= keeps the
        // blocking arc nearest the apex
        for (int w = vj; w != apex; w = s.parent[w]) {
            if (s.dir[w] == DOWN && s.flow_up[w] <= delta) {
                delta = s.flow_up[w];
                out = w;
                out_first = false;
            }
        }
        if (out < 0) return hm::fail(HM_ESOLVE, "transport simplex: unbounded cycle");
        // --- flows ---
        if (delta > 0.0) {
            for (int w = ui; w != apex; w = s.parent[w]) s.flow_up[w] += s.dir[w] == UP ? -delta : delta;
            for (int w = vj; w != apex; w = s.parent[w]) s.flow_up[w] += s.dir[w] == DOWN ? -delta : delta;
        }
        // --- tree: cut the leaving arc, hang the cut side from the entering arc ---
        // x0: endpoint of the entering arc in the cut-off subtree, y0: its new parent
        const int x0 = out_first ? ui : vj;
        const int y0 = out_first ? vj : ui;
        int new_parent = y0;
        int new_arc = (int)enter;
        int new_dir = out_first ? UP : DOWN;  // enter = ui -> vj
        double new_flow = delta;
        int w = x0;
        for (;;) {
            const int old_parent = s.parent[w], old_arc = s.pred_arc[w], old_dir = s.dir[w];
            const double old_flow = s.flow_up[w];
            s.detach(w);
            s.parent[w] = new_parent;
            s.pred_arc[w] = new_arc;
            s.dir[w] = new_dir;
            s.flow_up[w] = new_flow;
            s.attach(w, new_parent);
            if (w == out) break;
            new_parent = w;
            new_arc = old_arc;
            new_dir = -old_dir;
            new_flow = old_flow;
            w = old_parent;
        }
        s.refresh(x0, stack);
    }

    // --- duals: potentials recomputed per component from its top node (potential 0) over the transport arcs of
    // the tree, so that they hold no multiple of the artificial cost; then the components are re-joined (see the
    // header comment) ---
    std::vector<int> comp(n + m, -1);
    std::vector<double> local(s.V, 0.0);
    int K = 0;
    for (int top : s.children[s.root]) {
        stack.clear();
        stack.push_back(top);
        comp[top] = K;
        local[top] = 0.0;
        while (!stack.empty()) {
            const int q = stack.back();
            stack.pop_back();
            for (int ch : s.children[q]) {
                comp[ch] = K;
                const double ca = costs[s.pred_arc[ch]];
                local[ch] = s.dir[ch] == UP ? local[q] - ca : local[q] + ca;
                stack.push_back(ch);
            }
        }
        ++K;
    }
    for (int i = 0; i < n; ++i) u[i] = -local[i];
    for (int j = 0; j < m; ++j) v[j] = local[n + j];
    if (K > 1) {
        const double inf = std::numeric_limits<double>::infinity();
        std::vector<double> W((size_t)K * K, inf);
        for (int i = 0; i < n; ++i)
            for (int j = 0; j < m; ++j) {
                const int ki = comp[i], kj = comp[n + j];
                if (ki == kj) continue;
                const double rc = costs[(int64_t)i * m + j] - u[i] - v[j];
                double& slot = W[(size_t)ki * K + kj];
                if (rc < slot) slot = rc;
            }
        std::vector<double> dist(K, inf);
        std::vector<char> done(K, 0);
        dist[comp[0]] = 0.0;
        for (int it = 0; it < K; ++it) {
            int q = -1;
            for (int t = 0; t < K; ++t)
                if (!done[t] && (q < 0 || dist[t] < dist[q])) q = t;
            if (q < 0 || dist[q] == inf) break;
            done[q] = 1;
            for (int t = 0; t < K; ++t) {
                const double wq = W[(size_t)q * K + t];
                if (!done[t] && dist[q] + std::max(wq, 0.0) < dist[t]) dist[t] = dist[q] + std::max(wq, 0.0);
            }
        }
        for (int t = 0; t < K; ++t)
            if (dist[t] == inf) return hm::fail(HM_ESOLVE, "transport simplex: disconnected dual components");
        for (int i = 0; i < n; ++i) u[i] -= dist[comp[i]];
        for (int j = 0; j < m; ++j) v[j] += dist[comp[n + j]];
    }

    // duals are defined up to u + t, v - t: center them (sum a u = sum b v) so that they carry no offset of the
    // artificial cost scale
    {
        double au = 0.0, bv = 0.0;
        for (int i = 0; i < n; ++i) au += a[i] * u[i];
        for (int j = 0; j < m; ++j) bv += b[j] * v[j];
        const double t = (bv - au) / (sa + sb);
        for (int i = 0; i < n; ++i) u[i] += t;
        for (int j = 0; j < m; ++j) v[j] -= t;
    }

    // --- basis output: transport arcs of the final tree; artificial arcs must be empty ---
    int64_t count = 0;
    const double zero_tol = 1e-12 * std::max(1.0, sa);
    for (int x = 0; x < n + m; ++x) {
        const int64_t arc = s.pred_arc[x];
        if (s.artificial(arc)) {
            if (s.flow_up[x] > zero_tol)
                return hm::fail(HM_ESOLVE, "transport simplex: artificial flow %.3e left (infeasible)", s.flow_up[x]);
            continue;
        }
        basis_rows[count] = (int32_t)(arc / m);
        basis_cols[count] = (int32_t)(arc % m);
        basis_flows[count] = std::max(0.0, s.flow_up[x]);
        ++count;
    }
    *basis_count = count;
    if (pivots_out) *pivots_out = pivots;
    return HM_OK;
}
