// Support sparsification by cycle cancelling (host code; see hm_sparsify_support in include/helloot_hip.h).
//
// Behaviour follows the reference's sparsifier (restricted_ot/support_sparsification.py:52,
// _native/support_sparsifier/support_sparsifier_lct.cpp:378-555):
//   * a spanning forest of the positive edges, built in edge order by union-find;
//   * the other positive edges enter in edge order; entering edge e = (s, t) closes the cycle e + tree path
//     s .. t. Along that path (from s) the edges alternate: pushing +theta on e takes theta from the edges at
//     even positions and gives it to those at odd positions, at cost theta * (c_e - C_even + C_odd). The push
//     goes the way that does not increase the cost, by the largest step that keeps every flow >= 0. When e
//     stays positive, the first edge (in path order) that reached zero leaves the forest and e takes its place;
//     otherwise e drops to zero;
//   * every time enough cycles have been cancelled to possibly reach the target, the exact positive count is
//     taken (a degenerate step removes nothing) and the work stops once it is at most the target.
//
// The forest is a link-cut tree over vertex nodes and edge nodes (vertices 1..V, edge slots V+1..): each
// splay tree holds one path, in order, and aggregates over the edge nodes of its subtree, by the parity of
// their position within the subtree: cost sums, the minimum flow and the node that first attains it, and a
// pending flow addition. Reversing a subtree whose edge count is even swaps the two parities.
#include <cmath>
#include <cstdint>
#include <limits>
#include <numeric>
#include <vector>

#include "../../include/helloot_hip.h"

namespace hm {
int fail(int code, const char* fmt, ...);
}

namespace {

constexpr double kInf = std::numeric_limits<double>::infinity();

struct Node {
    int32_t ch[2] = {0, 0};
    int32_t up = 0;        // splay parent, or path parent when this node roots its splay tree
    int32_t edges = 0;     // edge nodes in the subtree
    bool flip = false;     // children's subtrees still to be reversed
    bool edge = false;
    bool pending = false;  // add[] still to be passed to the children
    double flow = 0.0, cost = 0.0;
    double sum[2] = {0.0, 0.0};    // cost sums by parity
    double low[2] = {kInf, kInf};  // minimum flow by parity
    int32_t at[2] = {0, 0};        // first node with that minimum
    double add[2] = {0.0, 0.0};    // addition by parity, already applied to this node's aggregates
};

class Forest {
  public:
    explicit Forest(int64_t nodes) : n_(static_cast<size_t>(nodes + 1)) {}

    void vertex(int32_t x) {
        n_[x] = Node{};
    }
    void edge_node(int32_t x, double flow, double cost) {
        n_[x] = Node{};
        n_[x].edge = true;
        n_[x].flow = flow;
        n_[x].cost = cost;
        pull(x);
    }
    // expose the path a .. b as one splay tree rooted at b (a first in order)
    int32_t expose(int32_t a, int32_t b) {
        evert(a);
        access(b);
        return b;
    }
    // attach isolated edge node x between the trees of a and b
    void link_between(int32_t a, int32_t x, int32_t b) {
        evert(a);
        n_[a].up = x;
        n_[x].up = b;
    }
    // cut edge node x out of the exposed path: its two sides become separate trees
    bool cut_exposed(int32_t x) {
        splay(x);
        const int32_t l = n_[x].ch[0], r = n_[x].ch[1];
        if (!l || !r) return false;
        n_[l].up = 0;
        n_[r].up = 0;
        n_[x].ch[0] = n_[x].ch[1] = 0;
        n_[x].up = 0;
        pull(x);
        return true;
    }
    void add_along(int32_t root, const double a[2]) { apply_add(root, a); }
    const Node& at(int32_t x) const { return n_[x]; }
    double flow(int32_t x) const { return n_[x].flow; }

    // pass every pending flip and addition down so each node's flow is current
    void settle() {
        std::vector<int32_t> stack;
        for (int32_t x = 1; x < static_cast<int32_t>(n_.size()); ++x) {
            if (!splay_root(x)) continue;
            stack.push_back(x);
            while (!stack.empty()) {
                const int32_t y = stack.back();
                stack.pop_back();
                push(y);
                for (int c = 0; c < 2; ++c)
                    if (n_[y].ch[c]) stack.push_back(n_[y].ch[c]);
            }
        }
    }

  private:
    int32_t edges(int32_t x) const { return x ? n_[x].edges : 0; }
    bool splay_root(int32_t x) const {
        const int32_t p = n_[x].up;
        return !p || (n_[p].ch[0] != x && n_[p].ch[1] != x);
    }

    // fold child segment c (its parity shifted by `offset` edges) into x's aggregates
    void fold(Node& x, const Node& c, int64_t offset) {
        for (int r = 0; r < 2; ++r) {
            const int s = static_cast<int>((offset + r) & 1);
            x.sum[s] += c.sum[r];
            if (c.low[r] < x.low[s]) {
                x.low[s] = c.low[r];
                x.at[s] = c.at[r];
            }
        }
    }

    void pull(int32_t x) {
        Node& v = n_[x];
        const int32_t l = v.ch[0], r = v.ch[1];
        v.edges = edges(l) + (v.edge ? 1 : 0) + edges(r);
        v.sum[0] = v.sum[1] = 0.0;
        v.low[0] = v.low[1] = kInf;
        v.at[0] = v.at[1] = 0;
        if (l) fold(v, n_[l], 0);
        if (v.edge) {
            const int s = edges(l) & 1;
            v.sum[s] += v.cost;
            if (v.flow < v.low[s]) {
                v.low[s] = v.flow;
                v.at[s] = x;
            }
        }
        if (r) fold(v, n_[r], edges(l) + (v.edge ? 1 : 0));
    }

    void apply_add(int32_t x, const double a[2]) {
        if (!x || (a[0] == 0.0 && a[1] == 0.0)) return;
        Node& v = n_[x];
        for (int r = 0; r < 2; ++r) {
            if (v.low[r] < kInf) v.low[r] += a[r];
            v.add[r] += a[r];
        }
        v.pending = true;
        if (v.edge) v.flow += a[edges(v.ch[0]) & 1];
    }

    void apply_flip(int32_t x) {
        if (!x) return;
        Node& v = n_[x];
        const int32_t t = v.ch[0];
        v.ch[0] = v.ch[1];
        v.ch[1] = t;
        if ((v.edges & 1) == 0) {  // position k -> edges-1-k changes parity iff edges is even
            for (double* a : {v.sum, v.low, v.add}) {
                const double t0 = a[0];
                a[0] = a[1];
                a[1] = t0;
            }
            const int32_t t1 = v.at[0];
            v.at[0] = v.at[1];
            v.at[1] = t1;
        }
        v.flip = !v.flip;
    }

    void push(int32_t x) {
        Node& v = n_[x];
        if (v.flip) {
            apply_flip(v.ch[0]);
            apply_flip(v.ch[1]);
            v.flip = false;
        }
        if (v.pending) {
            apply_add(v.ch[0], v.add);
            const int64_t off = edges(v.ch[0]) + (v.edge ? 1 : 0);
            const double shifted[2] = {v.add[off & 1], v.add[(off + 1) & 1]};
            apply_add(v.ch[1], shifted);
            v.add[0] = v.add[1] = 0.0;
            v.pending = false;
        }
    }

    void rotate(int32_t x) {
        const int32_t p = n_[x].up, g = n_[p].up;
        const int d = n_[p].ch[1] == x ? 1 : 0;
        const int32_t b = n_[x].ch[d ^ 1];
        if (!splay_root(p)) n_[g].ch[n_[g].ch[1] == p ? 1 : 0] = x;
        n_[x].up = g;
        n_[x].ch[d ^ 1] = p;
        n_[p].up = x;
        n_[p].ch[d] = b;
        if (b) n_[b].up = p;
        pull(p);
        pull(x);
    }

    void splay(int32_t x) {
        path_.clear();
        for (int32_t y = x;; y = n_[y].up) {
            path_.push_back(y);
            if (splay_root(y)) break;
        }
        for (size_t i = path_.size(); i-- > 0;) push(path_[i]);
        while (!splay_root(x)) {
            const int32_t p = n_[x].up;
            if (!splay_root(p)) {
                const int32_t g = n_[p].up;
                rotate((n_[g].ch[0] == p) == (n_[p].ch[0] == x) ? p : x);
            }
            rotate(x);
        }
    }

    void access(int32_t x) {
        int32_t below = 0;
        for (int32_t y = x; y; y = n_[y].up) {
            splay(y);
            n_[y].ch[1] = below;
            pull(y);
            below = y;
        }
        splay(x);
    }

    void evert(int32_t x) {
        access(x);
        apply_flip(x);
    }

    std::vector<Node> n_;
    std::vector<int32_t> path_;
};

struct UnionFind {
    std::vector<int64_t> p;
    std::vector<uint8_t> rank;
    explicit UnionFind(int64_t n) : p(static_cast<size_t>(n)), rank(static_cast<size_t>(n), 0) {
        std::iota(p.begin(), p.end(), 0);
    }
    int64_t root(int64_t x) {
        while (p[x] != x) {
            p[x] = p[p[x]];
            x = p[x];
        }
        return x;
    }
    bool join(int64_t a, int64_t b) {
        a = root(a);
        b = root(b);
        if (a == b) return false;
        if (rank[a] < rank[b]) std::swap(a, b);
        p[b] = a;
        if (rank[a] == rank[b]) ++rank[a];
        return true;
    }
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
    if (2 * V + 1 >= static_cast<int64_t>(std::numeric_limits<int32_t>::max()))
        return fail(HM_EINVAL, "sparsify: too many vertices");

    // vertices: source i -> 1 + i, target j -> 1 + n_source + j
    UnionFind uf(V);
    std::vector<int64_t> tree, entering;
    int64_t nnz = 0;
    for (int64_t k = 0; k < e; ++k) {
        if (rows[k] < 0 || rows[k] >= n_source || cols[k] < 0 || cols[k] >= n_target)
            return fail(HM_EINVAL, "sparsify: edge %lld has an endpoint out of range", (long long)k);
        if (!std::isfinite(values[k]) || values[k] < -zero_tolerance || !std::isfinite(costs[k]))
            return fail(HM_EINVAL, "sparsify: edge %lld has a negative or non-finite flow or cost", (long long)k);
        if (values[k] <= zero_tolerance) {
            values[k] = 0.0;
            continue;
        }
        ++nnz;
        if (uf.join(rows[k], n_source + cols[k])) tree.push_back(k);
        else entering.push_back(k);
    }
    int64_t cycles = 0, tree_ops = 0;
    if (nnz <= target_nnz || entering.empty()) {
        stats[0] = nnz;
        stats[1] = 0;
        stats[2] = 0;
        return HM_OK;
    }
    Forest f(V + static_cast<int64_t>(tree.size()));
    for (int32_t x = 1; x <= static_cast<int32_t>(V); ++x) f.vertex(x);
    std::vector<int64_t> slot_edge(tree);  // tree slot s (node V + 1 + s) -> edge id
    for (size_t s = 0; s < tree.size(); ++s) {
        const int64_t k = tree[s];
        const int32_t x = static_cast<int32_t>(V + 1 + static_cast<int64_t>(s));
        f.edge_node(x, values[k], costs[k]);
        f.link_between(static_cast<int32_t>(1 + rows[k]), x, static_cast<int32_t>(1 + n_source + cols[k]));
    }
    int64_t check_at = nnz - target_nnz;  // cycles after which the target can first be reached
    for (size_t pos = 0; pos < entering.size(); ++pos) {
        if (cycles >= check_at) {
            f.settle();
            int64_t count = static_cast<int64_t>(entering.size() - pos);
            for (size_t s = 0; s < slot_edge.size(); ++s)
                count += f.flow(static_cast<int32_t>(V + 1 + static_cast<int64_t>(s))) > zero_tolerance ? 1 : 0;
            if (count <= target_nnz) break;
            check_at = cycles + (count - target_nnz);
        }
        const int64_t k = entering[pos];
        double flow_e = values[k];
        if (flow_e <= zero_tolerance) continue;
        const int32_t s_node = static_cast<int32_t>(1 + rows[k]);
        const int32_t t_node = static_cast<int32_t>(1 + n_source + cols[k]);
        const int32_t root = f.expose(s_node, t_node);
        tree_ops += 2;
        const Node& path = f.at(root);
        // +theta on e: even positions (from the source) give theta, odd positions take it
        const double gain = costs[k] - path.sum[0] + path.sum[1];
        const double dir = gain <= 0.0 ? 1.0 : -1.0;
        const int losing = dir > 0.0 ? 0 : 1;
        double step = path.low[losing];
        const int32_t leaving = path.at[losing];
        if (dir < 0.0 && flow_e < step) step = flow_e;
        if (!std::isfinite(step)) return fail(HM_EINVAL, "sparsify: cycle without a bounded step");
        if (step < -zero_tolerance) return fail(HM_EINVAL, "sparsify: a tree flow became negative");
        if (step < 0.0) step = 0.0;
        const double delta[2] = {-dir * step, dir * step};
        f.add_along(root, delta);
        flow_e += dir * step;
        if (flow_e > zero_tolerance) {
            // the first edge on the losing side that reached zero leaves; e takes over its tree slot
            if (leaving <= static_cast<int32_t>(V)) return fail(HM_EINVAL, "sparsify: no leaving edge");
            const size_t slot = static_cast<size_t>(leaving - V - 1);
            if (!f.cut_exposed(leaving)) return fail(HM_EINVAL, "sparsify: leaving edge not on the path");
            values[slot_edge[slot]] = 0.0;
            slot_edge[slot] = k;
            f.edge_node(leaving, flow_e, costs[k]);
            f.link_between(s_node, leaving, t_node);
            tree_ops += 4;
        } else {
            values[k] = 0.0;
        }
        ++cycles;
    }
    f.settle();
    for (size_t s = 0; s < slot_edge.size(); ++s) {
        const double v = f.flow(static_cast<int32_t>(V + 1 + static_cast<int64_t>(s)));
        if (!std::isfinite(v) || v < -zero_tolerance) return fail(HM_EINVAL, "sparsify: invalid flow after cancelling");
        values[slot_edge[s]] = v > zero_tolerance ? v : 0.0;
    }
    int64_t out = 0;
    for (int64_t k = 0; k < e; ++k) {
        if (values[k] <= zero_tolerance) values[k] = 0.0;
        else ++out;
    }
    stats[0] = out;
    stats[1] = cycles;
    stats[2] = tree_ops;
    return HM_OK;
}
