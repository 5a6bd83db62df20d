// Support sparsification by cycle cancelling (host code; see hm_sparsify_support in include/helloot_hip.h).
//
// What it computes is the reference's sparsifier (restricted_ot/support_sparsification.py:52,
// _native/support_sparsifier/support_sparsifier_lct.cpp:378-555):
//   * the positive edges, in edge order, split into a spanning forest (union-find) and entering edges;
//   * entering edge e = (s, t), in edge order, closes the cycle e + forest path s .. t. Walking that path from s,
//     an edge crossed from its source endpoint to its target endpoint ("forward") gives up what e gains and an edge
//     crossed the other way ("backward") takes it: pushing +theta on e costs theta (c_e - C_forward + C_backward).
//     The push goes the way that does not increase the cost, by the largest step that keeps all flows >= 0. If e
//     stays positive, the first edge from s among those that reached the step leaves the forest and e enters;
//     otherwise e drops to zero;
//   * the exact positive count is taken each time enough cycles have been cancelled to possibly reach the target
//     (a degenerate cycle removes nothing), and the work stops once the count is at most the target.
//
// Representation (this file's own): the forest is a parent-pointer forest over the n_source + n_target vertices
// (parent vertex and the edge to it), and flows are updated eagerly on the cycle's edges, in path order. The path
// is found by two walkers climbing from s and t in lockstep that stamp the vertices they pass: the first vertex a
// walker finds stamped by the other is the apex, so a cycle costs O(its length) whatever the depths. An exchange
// re-hangs the side cut off by the leaving edge from e, reversing the parent pointers between e's endpoint and
// the leaving edge. The count of positive forest edges is kept exact as flows move, so the stopping checks need no
// pass over the forest.
//
// Eager updates round each flow once per cycle through it, in cycle order. The reference accumulates pending
// additions in its link-cut tree and rounds their sums, so the two agree to rounding (about 1e-16 relative per
// cycle), not bit for bit; counts and the choices made agree whenever no two candidate step values are closer
// than that.
#include <cmath>
#include <cstdint>
#include <limits>
#include <vector>

#include "../../include/helloot_hip.h"

namespace hm {
int fail(int code, const char* fmt, ...);
}

namespace {

// disjoint sets over vertices (path halving, union by size)
struct Components {
    std::vector<int64_t> link, size;
    explicit Components(int64_t n) : link(n), size(n, 1) {
        for (int64_t v = 0; v < n; ++v) link[v] = v;
    }
    int64_t root(int64_t v) {
        while (link[v] != v) {
            link[v] = link[link[v]];
            v = link[v];
        }
        return v;
    }
    bool merge(int64_t a, int64_t b) {
        a = root(a);
        b = root(b);
        if (a == b) return false;
        if (size[a] < size[b]) std::swap(a, b);
        link[b] = a;
        size[a] += size[b];
        return true;
    }
};

struct PathEdge {
    int64_t edge;
    bool forward;  // crossed from its source endpoint to its target endpoint
};

}  // namespace

extern "C" int hm_sparsify_support(int64_t n_source, int64_t n_target, int64_t e, const int64_t* rows,
                                   const int64_t* cols, double* values, const double* costs, int64_t target_nnz,
                                   double zero_tolerance, int64_t* stats) {
    using hm::fail;
    if (n_source < 1 || n_target < 1 || e < 0 || (e > 0 && (!rows || !cols || !values || !costs)) || !stats)
        return fail(HM_EINVAL, "sparsify: invalid sizes or pointers");
    if (!std::isfinite(zero_tolerance) || zero_tolerance < 0.0)
        return fail(HM_EINVAL, "sparsify: zero_tolerance must be finite and nonnegative");
    const int64_t V = n_source + n_target;
    if (target_nnz < V - 1) return fail(HM_EINVAL, "sparsify: target_nnz must be at least n_source + n_target - 1");

    // --- forest and entering edges (vertices: source i -> i, target j -> n_source + j) ---
    Components comps(V);
    std::vector<int64_t> forest_edges, entering;
    int64_t positive = 0;
    for (int64_t k = 0; k < e; ++k) {
        if (rows[k] < 0 || rows[k] >= n_source || cols[k] < 0 || cols[k] >= n_target)
            return fail(HM_EINVAL, "sparsify: edge %lld has an endpoint out of range", (long long)k);
        if (!std::isfinite(values[k]) || !std::isfinite(costs[k]) || values[k] < -zero_tolerance)
            return fail(HM_EINVAL, "sparsify: edge %lld has a non-finite or negative flow, or a non-finite cost",
                        (long long)k);
        if (values[k] <= zero_tolerance) {
            values[k] = 0.0;
            continue;
        }
        ++positive;
        (comps.merge(rows[k], n_source + cols[k]) ? forest_edges : entering).push_back(k);
    }

    // parent pointers: each component hung from its lowest vertex, by a breadth-first walk over the forest edges
    std::vector<int64_t> parent(V, -1), up_edge(V, -1);
    {
        std::vector<int64_t> start(V + 1, 0), adj(2 * forest_edges.size());
        for (int64_t k : forest_edges) {
            ++start[rows[k] + 1];
            ++start[n_source + cols[k] + 1];
        }
        for (int64_t v = 0; v < V; ++v) start[v + 1] += start[v];
        std::vector<int64_t> fill(start.begin(), start.end() - 1);
        for (int64_t k : forest_edges) {
            adj[fill[rows[k]]++] = k;
            adj[fill[n_source + cols[k]]++] = k;
        }
        std::vector<char> seen(V, 0);
        std::vector<int64_t> queue;
        queue.reserve(V);
        for (int64_t r = 0; r < V; ++r) {
            if (seen[r]) continue;
            seen[r] = 1;
            queue.clear();
            queue.push_back(r);
            for (size_t h = 0; h < queue.size(); ++h) {
                const int64_t x = queue[h];
                for (int64_t p = start[x]; p < start[x + 1]; ++p) {
                    const int64_t k = adj[p];
                    const int64_t y = rows[k] == x ? n_source + cols[k] : rows[k];
                    if (seen[y]) continue;
                    seen[y] = 1;
                    parent[y] = x;
                    up_edge[y] = k;
                    queue.push_back(y);
                }
            }
        }
    }

    // positive forest edges, kept exact as flows change
    int64_t forest_positive = static_cast<int64_t>(forest_edges.size());
    auto set_flow = [&](int64_t k, double v) {
        const bool was = values[k] > zero_tolerance, now = v > zero_tolerance;
        forest_positive += (int64_t)now - (int64_t)was;
        values[k] = v;
    };

    std::vector<uint64_t> stamp(V, 0);
    uint64_t tick = 0;
    std::vector<PathEdge> from_s, from_t;
    int64_t cycles = 0, exchanges = 0;
    int64_t next_check = std::max<int64_t>(0, positive - target_nnz);
    for (size_t pos = 0; pos < entering.size(); ++pos) {
        if (cycles >= next_check) {
            const int64_t exact = forest_positive + static_cast<int64_t>(entering.size() - pos);
            if (exact <= target_nnz) break;
            next_check = cycles + (exact - target_nnz);
        }
        const int64_t k = entering[pos];
        double flow_e = values[k];
        if (flow_e <= zero_tolerance) continue;
        const int64_t s = rows[k], t = n_source + cols[k];

        // --- the forest path s .. t: two walkers in lockstep; the first stamp of the other side is the apex ---
        tick += 2;
        const uint64_t mark_s = tick, mark_t = tick + 1;
        int64_t a = s, b = t, apex = -1;
        stamp[a] = mark_s;
        stamp[b] = mark_t;
        while (apex < 0) {
            if (a >= 0) {
                const int64_t up = parent[a];
                if (up >= 0) {
                    if (stamp[up] == mark_t) apex = up;
                    stamp[up] = mark_s;
                }
                a = up;
            }
            if (apex < 0 && b >= 0) {
                const int64_t up = parent[b];
                if (up >= 0) {
                    if (stamp[up] == mark_s) apex = up;
                    stamp[up] = mark_t;
                }
                b = up;
            }
            if (a < 0 && b < 0 && apex < 0) return fail(HM_EINVAL, "sparsify: entering edge joins two components");
        }
        // edges from s up to the apex (in path order), then from t up to the apex (reverse path order)
        from_s.clear();
        from_t.clear();
        for (int64_t x = s; x != apex; x = parent[x]) from_s.push_back({up_edge[x], x < n_source});
        for (int64_t x = t; x != apex; x = parent[x]) from_t.push_back({up_edge[x], x >= n_source});

        // --- direction, step and leaving edge ---
        double sum_forward = 0.0, sum_backward = 0.0;  // path costs by crossing direction, in path order
        for (const PathEdge& pe : from_s) (pe.forward ? sum_forward : sum_backward) += costs[pe.edge];
        for (size_t q = from_t.size(); q-- > 0;) (from_t[q].forward ? sum_forward : sum_backward) += costs[from_t[q].edge];
        const double gain = costs[k] - sum_forward + sum_backward;
        const double dir = gain <= 0.0 ? 1.0 : -1.0;
        const bool losing_forward = dir > 0.0;
        double step = std::numeric_limits<double>::infinity();
        int64_t leaving = -1;
        bool leaving_on_s = true;
        for (const PathEdge& pe : from_s)
            if (pe.forward == losing_forward && values[pe.edge] < step) {
                step = values[pe.edge];
                leaving = pe.edge;
                leaving_on_s = true;
            }
        for (size_t q = from_t.size(); q-- > 0;)
            if (from_t[q].forward == losing_forward && values[from_t[q].edge] < step) {
                step = values[from_t[q].edge];
                leaving = from_t[q].edge;
                leaving_on_s = false;
            }
        if (dir < 0.0 && flow_e < step) step = flow_e;
        if (!std::isfinite(step)) return fail(HM_EINVAL, "sparsify: cycle without a bounded step");
        if (step < 0.0) step = 0.0;

        // --- push: forward edges lose dir * step, backward edges gain it ---
        for (const PathEdge& pe : from_s) set_flow(pe.edge, values[pe.edge] + (pe.forward ? -dir : dir) * step);
        for (const PathEdge& pe : from_t) set_flow(pe.edge, values[pe.edge] + (pe.forward ? -dir : dir) * step);
        flow_e += dir * step;
        if (flow_e > zero_tolerance) {
            // exchange: the leaving edge drops to zero; the side it cut off hangs from e
            if (leaving < 0) return fail(HM_EINVAL, "sparsify: no leaving edge on the cycle");
            set_flow(leaving, 0.0);
            int64_t x = leaving_on_s ? s : t;
            int64_t new_parent = leaving_on_s ? t : s, new_edge = k;
            for (;;) {
                const int64_t old_parent = parent[x], old_edge = up_edge[x];
                parent[x] = new_parent;
                up_edge[x] = new_edge;
                if (old_edge == leaving) break;
                new_parent = x;
                new_edge = old_edge;
                x = old_parent;
            }
            values[k] = flow_e;
            ++forest_positive;
            ++exchanges;
        } else {
            values[k] = 0.0;
        }
        ++cycles;
    }

    int64_t out = 0;
    for (int64_t k = 0; k < e; ++k) {
        if (!std::isfinite(values[k]) || values[k] < -zero_tolerance)
            return fail(HM_EINVAL, "sparsify: edge %lld ended with an invalid flow", (long long)k);
        if (values[k] <= zero_tolerance) values[k] = 0.0;
        else ++out;
    }
    stats[0] = out;
    stats[1] = cycles;
    // the reference reports the link-cut operations it performs: two per cycle (evert and access of the path)
    // and four more per exchange (cut, re-initialise, evert, link); the same count follows from the cycle and
    // exchange counts
    stats[2] = 2 * cycles + 4 * exchanges;
    return HM_OK;
}
