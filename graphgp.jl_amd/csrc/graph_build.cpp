// graph_build.cpp — host construction of the refinement graph (declared in graphgp_graph.h).
//
// Restates the reference's CPU build_graph (src/graph_build.jl:254-288):
//   1. heap-order ("special order") k-d tree, one global pass per tree level
//      (build_tree_special, src/tree_special.jl:165-227);
//   2. stackless preceding k-nearest-neighbour query (src/tree_special.jl:231-332);
//   3. depth relaxation and stable reordering by depth (src/graph_build.jl:69-107, 160-200);
//   4. lattice quantization (src/graph_build.jl:231-242) and level offsets (:213-221).
// Each step keeps the reference's tie-breaking so the graph matches it point for point.
// Per-level sorts run as a counting sort by node id followed by independent per-node sorts.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <numeric>
#include <vector>
#include <omp.h>

#include "../../include/graphgp_graph.h"

struct ggp_built_graph {
    int64_t N = 0, n0 = 0, K = 0;
    int32_t D = 0;
    std::vector<uint32_t> coords;
    std::vector<int64_t> neighbors, offsets, indices;
    double scale = 1.0;
};

namespace {

inline int flevel(int64_t x) { return 63 - __builtin_clzll((unsigned long long)x); }

inline int64_t sp_parent(int64_t c) {
    if (c == 0) return -1;
    const int level = flevel(c + 1);
    const int64_t n_above = (int64_t(1) << level) - 1;
    const int64_t npl = int64_t(1) << (level - 1);
    return c < n_above + npl ? c - npl : c - 2 * npl;
}
inline int64_t sp_left(int64_t c) { return c + (int64_t(1) << flevel(c + 1)); }
inline int64_t sp_right(int64_t c) { return c + 2 * (int64_t(1) << flevel(c + 1)); }

// build_tree_special (src/tree_special.jl:165-227). pts is N x D row-major, rewritten in tree
// order; perm[tree_pos] = original index; split[node] = split dimension.
void build_tree(std::vector<double>& pts, int64_t N, int D, std::vector<int64_t>& perm,
                std::vector<int>& split) {
    const int n_levels = N > 0 ? flevel(N) + 1 : 0;
    std::vector<int64_t> nodes(N, 0), nodes_s(N), perm_s(N), order(N), cnt(N + 1);
    std::vector<double> pts_s(pts.size()), seg_max((size_t)N * D), seg_min((size_t)N * D),
        pad(N);
    perm.resize(N);
    std::iota(perm.begin(), perm.end(), 0);
    split.assign(N, -1);
    const double inf = std::numeric_limits<double>::infinity();
    for (int level = 0; level < n_levels; ++level) {
        const int64_t n_above = (int64_t(1) << level) - 1;
        const int64_t n_level = int64_t(1) << level;
        std::fill(seg_max.begin(), seg_max.end(), -inf);
        std::fill(seg_min.begin(), seg_min.end(), inf);
        for (int64_t i = 0; i < N; ++i) {
            const int64_t s = nodes[i];
            for (int d = 0; d < D; ++d) {
                const double v = pts[(size_t)i * D + d];
                if (v > seg_max[(size_t)s * D + d]) seg_max[(size_t)s * D + d] = v;
                if (v < seg_min[(size_t)s * D + d]) seg_min[(size_t)s * D + d] = v;
            }
        }
#pragma omp parallel for schedule(static)
        for (int64_t c = n_above; c < N; ++c) {
            int bestd = 0;
            double bestr = -inf;
            for (int d = 0; d < D; ++d) {
                const double r = seg_max[(size_t)c * D + d] - seg_min[(size_t)c * D + d];
                if (r > bestr) { bestr = r; bestd = d; }
            }
            split[c] = bestd;
        }
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < N; ++i) pad[i] = pts[(size_t)i * D + split[nodes[i]]];
        // Stable order by (node, pad, position): counting sort by node keeps position order,
        // then a stable sort by pad inside each node's run.
        std::fill(cnt.begin(), cnt.end(), 0);
        for (int64_t i = 0; i < N; ++i) cnt[nodes[i] + 1]++;
        for (int64_t s = 0; s < N; ++s) cnt[s + 1] += cnt[s];
        {
            std::vector<int64_t> pos(cnt.begin(), cnt.end() - 1);
            for (int64_t i = 0; i < N; ++i) order[pos[nodes[i]]++] = i;
        }
#pragma omp parallel for schedule(dynamic, 64)
        for (int64_t s = 0; s < N; ++s) {
            const int64_t lo = cnt[s], hi = cnt[s + 1];
            if (hi - lo > 1)
                std::stable_sort(order.begin() + lo, order.begin() + hi,
                                 [&](int64_t a, int64_t b) { return pad[a] < pad[b]; });
        }
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < N; ++i) {
            const int64_t p = order[i];
            for (int d = 0; d < D; ++d) pts_s[(size_t)i * D + d] = pts[(size_t)p * D + d];
            nodes_s[i] = nodes[p];
            perm_s[i] = perm[p];
        }
        pts.swap(pts_s);
        perm.swap(perm_s);
        nodes.swap(nodes_s);
        const int64_t n_remaining = N - n_above;
        const int64_t q = n_remaining / n_level, r = n_remaining % n_level;
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < N; ++i) {
            const int64_t s = nodes[i];
            if (i < n_above) { nodes_s[i] = s; continue; }
            const int64_t ii = s - n_above;
            const int64_t mid = (ii < r ? ii * (q + 1) + (q + 1) / 2
                                        : r * (q + 1) + (ii - r) * q + q / 2) + n_above;
            nodes_s[i] = i == mid ? s : (i < mid ? s + n_level : s + 2 * n_level);
        }
        nodes.swap(nodes_s);
    }
}

// _sp_query_one! (src/tree_special.jl:231-300) for one query node.
void query_one(const double* pts, const int* split, int64_t query, int64_t max_index, int k,
               int D, double* cand_d, int64_t* cand_i) {
    const double inf = std::numeric_limits<double>::infinity();
    for (int j = 0; j < k; ++j) { cand_d[j] = inf; cand_i[j] = -1; }
    double square_radius = inf;
    const double* qp = pts + (size_t)query * D;
    int64_t current = 0, previous = -1;
    while (current != -1) {
        const int64_t parent = sp_parent(current);
        if (previous == parent) {
            const double* cp = pts + (size_t)current * D;
            double sq = 0.0;
            for (int d = 0; d < D; ++d) {
                const double dv = qp[d] - cp[d];
                sq += dv * dv;
            }
            int wpos = 0;
            double wval = cand_d[0];
            for (int j = 1; j < k; ++j)
                if (cand_d[j] > wval) { wval = cand_d[j]; wpos = j; }
            if (sq < wval) {
                cand_d[wpos] = sq;
                cand_i[wpos] = current;
                double m = cand_d[0];
                for (int j = 1; j < k; ++j) if (cand_d[j] > m) m = cand_d[j];
                square_radius = m;
            } else {
                square_radius = wval;
            }
        }
        const int sd = split[current];
        const double split_distance = qp[sd] - pts[(size_t)current * D + sd];
        const int64_t near = split_distance < 0 ? sp_left(current) : sp_right(current);
        const int64_t far = split_distance < 0 ? sp_right(current) : sp_left(current);
        const bool far_in_range = split_distance * split_distance <= square_radius;
        int64_t nxt;
        if (previous == near || (previous == parent && near >= max_index))
            nxt = (far < max_index && far_in_range) ? far : parent;
        else
            nxt = previous == parent ? near : parent;
        previous = current;
        current = nxt;
    }
}

}  // namespace

extern "C" {

int ggp_build_graph(const double* points, int64_t N, int32_t D, int64_t n0, int64_t k,
                    int32_t lattice_bits, int32_t nthreads, ggp_built_graph** out) {
    if (!out || !points || N < 2 || D < 1 || k < 1 || n0 < k || n0 >= N || lattice_bits < 1 ||
        lattice_bits > 30)
        return 7;
    if (nthreads > 0) omp_set_num_threads(nthreads);
    std::vector<double> pts(points, points + (size_t)N * D);
    std::vector<int64_t> perm;
    std::vector<int> split;
    build_tree(pts, N, D, perm, split);
    const int64_t M = N - n0;
    std::vector<int64_t> nbr((size_t)M * k);
#pragma omp parallel
    {
        std::vector<double> cd(k);
        std::vector<int64_t> ci(k);
        std::vector<int> ord(k);
#pragma omp for schedule(dynamic, 256)
        for (int64_t m = n0; m < N; ++m) {
            query_one(pts.data(), split.data(), m, m, (int)k, D, cd.data(), ci.data());
            std::iota(ord.begin(), ord.end(), 0);
            std::stable_sort(ord.begin(), ord.end(), [&](int a, int b) {
                return cd[a] != cd[b] ? cd[a] < cd[b] : ci[a] < ci[b];
            });
            for (int64_t j = 0; j < k; ++j) nbr[(size_t)(m - n0) * k + j] = ci[ord[j]];
        }
    }
    // compute_depths (src/graph_build.jl:69-93): neighbours precede, one ordered pass.
    std::vector<int64_t> depth(N, 0);
    for (int64_t m = 0; m < M; ++m) {
        int64_t mx = 0;
        for (int64_t j = 0; j < k; ++j) {
            const int64_t q = nbr[(size_t)m * k + j];
            if (q >= 0 && depth[q] > mx) mx = depth[q];
        }
        depth[n0 + m] = mx + 1;
    }
    // order_by_depth (src/graph_build.jl:160-200): stable sort by depth.
    std::vector<int64_t> sp(N), inv(N);
    std::iota(sp.begin(), sp.end(), 0);
    std::stable_sort(sp.begin(), sp.end(), [&](int64_t a, int64_t b) { return depth[a] < depth[b]; });
    for (int64_t i = 0; i < N; ++i) inv[sp[i]] = i;
    int64_t n0_new = 0;
    for (int64_t i = 0; i < N; ++i) n0_new += depth[i] == 0;
    ggp_built_graph* g = new ggp_built_graph();
    g->N = N; g->n0 = n0_new; g->K = k; g->D = D;
    std::vector<double> spts((size_t)N * D);
    g->indices.resize(N);
    std::vector<int64_t> sdepth(N);
    for (int64_t i = 0; i < N; ++i) {
        for (int d = 0; d < D; ++d) spts[(size_t)i * D + d] = pts[(size_t)sp[i] * D + d];
        g->indices[i] = perm[sp[i]];
        sdepth[i] = depth[sp[i]];
    }
    g->neighbors.assign((size_t)(N - n0_new) * k, 0);
    for (int64_t m_old = 0; m_old < M; ++m_old) {
        const int64_t m_new = inv[n0 + m_old] - n0_new;
        if (m_new < 0) continue;
        for (int64_t j = 0; j < k; ++j) {
            const int64_t q = nbr[(size_t)m_old * k + j];
            if (q < 0) continue;
            g->neighbors[(size_t)m_new * k + j] = inv[q];
        }
    }
    // quantize_to_lattice (src/graph_build.jl:231-242), ties to even like round(Int64, x).
    const double lmax = (double)((int64_t(1) << lattice_bits) - 1);
    std::vector<double> origin(D, std::numeric_limits<double>::infinity()), hi(D, -std::numeric_limits<double>::infinity());
    for (int64_t i = 0; i < N; ++i)
        for (int d = 0; d < D; ++d) {
            origin[d] = std::min(origin[d], spts[(size_t)i * D + d]);
            hi[d] = std::max(hi[d], spts[(size_t)i * D + d]);
        }
    double extent = 0.0;
    for (int d = 0; d < D; ++d) extent = std::max(extent, hi[d] - origin[d]);
    const double scale = extent > 0 ? extent / lmax : 1.0 / lmax;
    g->scale = scale;
    g->coords.resize((size_t)N * D);
    for (int64_t i = 0; i < N; ++i)
        for (int d = 0; d < D; ++d) {
            const double c = std::nearbyint((spts[(size_t)i * D + d] - origin[d]) / scale);
            g->coords[(size_t)i * D + d] = (uint32_t)std::min(std::max(c, 0.0), lmax);
        }
    // _compute_offsets (src/graph_build.jl:213-221)
    const int64_t maxd = sdepth.empty() ? 0 : sdepth.back();
    int64_t idx = 0;
    for (int64_t d = 0; d <= maxd; ++d) {
        while (idx < N && sdepth[idx] <= d) ++idx;
        g->offsets.push_back(idx);
    }
    *out = g;
    return 0;
}

int ggp_built_graph_shape(const ggp_built_graph* g, int64_t* N, int64_t* n0, int64_t* k,
                          int32_t* D, int64_t* n_offsets) {
    if (!g) return 7;
    if (N) *N = g->N;
    if (n0) *n0 = g->n0;
    if (k) *k = g->K;
    if (D) *D = g->D;
    if (n_offsets) *n_offsets = (int64_t)g->offsets.size();
    return 0;
}

int ggp_built_graph_copy(const ggp_built_graph* g, uint32_t* coords, int64_t* neighbors,
                         int64_t* offsets, int64_t* indices, double* scale) {
    if (!g) return 7;
    if (coords) std::memcpy(coords, g->coords.data(), g->coords.size() * 4);
    if (neighbors) std::memcpy(neighbors, g->neighbors.data(), g->neighbors.size() * 8);
    if (offsets) std::memcpy(offsets, g->offsets.data(), g->offsets.size() * 8);
    if (indices) std::memcpy(indices, g->indices.data(), g->indices.size() * 8);
    if (scale) *scale = g->scale;
    return 0;
}

void ggp_built_graph_free(ggp_built_graph* g) { delete g; }

}  // extern "C"
