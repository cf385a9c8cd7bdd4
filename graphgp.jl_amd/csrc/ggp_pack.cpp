// ggp_pack.cpp — host-side validation and repacking of a problem's graph (see ggp_pack.h).
#include "ggp_pack.h"

#include <algorithm>

#include "../../include/graphgp_hip.h"

namespace ggp {

namespace {
int pfail(std::string* err, int code, const char* msg) {
    if (err) *err = msg;
    return code;
}
}  // namespace

int check_graph_host(const uint32_t* coords, const int64_t* nbrs, const int64_t* offs,
                     int64_t n_off, const int64_t* indices, int64_t n0, int64_t k, int64_t N,
                     int32_t D, std::string* err) {
    if (N < 1 || n0 < 1 || n0 > N) return pfail(err, GGP_ERR_GRAPH, "need 1 <= n0 <= N");
    if (N > INT32_MAX) return pfail(err, GGP_ERR_ARG, "N must fit in int32");
    if (n0 > 16384) return pfail(err, GGP_ERR_ARG, "n0 above 16384 is not supported");
    const int64_t M = N - n0;
    if ((uint64_t)M * (uint64_t)k >= (1ull << 32)) return pfail(err, GGP_ERR_ARG, "M*k must be < 2^32");
    if (!coords || (M > 0 && !nbrs) || !offs) return pfail(err, GGP_ERR_ARG, "null input array");
    // check_graph (src/graph_build.jl:20-57)
    if (n_off < 1) return pfail(err, GGP_ERR_GRAPH, "offsets is empty");
    if (offs[0] != n0) return pfail(err, GGP_ERR_GRAPH, "offsets[0] must equal n0");
    for (int64_t b = 1; b < n_off; ++b)
        if (offs[b] < offs[b - 1]) return pfail(err, GGP_ERR_GRAPH, "offsets must be non-decreasing");
    if (offs[n_off - 1] > N) return pfail(err, GGP_ERR_GRAPH, "offsets[end] must be <= N");
    {
        int64_t b = 1;
        for (int64_t m = 0; m < M; ++m) {
            const int64_t p = n0 + m;
            while (b < n_off && offs[b] <= p) ++b;
            const int64_t prev_end = b < n_off ? offs[b - 1] : offs[n_off - 1];
            for (int64_t j = 0; j < k; ++j) {
                const int64_t q = nbrs[m * k + j];
                if (q < 0 || q >= N) return pfail(err, GGP_ERR_GRAPH, "neighbour index out of range");
                if (q >= p)
                    return pfail(err, GGP_ERR_GRAPH, "neighbour does not precede its point (not topological)");
                if (b < n_off && q >= prev_end)
                    return pfail(err, GGP_ERR_GRAPH, "neighbour in its own depth level; neighbours must be in earlier levels");
            }
        }
    }
    if (indices) {
        std::vector<char> seen((size_t)N, 0);
        for (int64_t i = 0; i < N; ++i) {
            if (indices[i] < 0 || indices[i] >= N || seen[(size_t)indices[i]])
                return pfail(err, GGP_ERR_GRAPH, "indices must be a permutation of 0..N-1");
            seen[(size_t)indices[i]] = 1;
        }
    }
    for (int64_t i = 0; i < N * D; ++i)
        if (coords[i] >= (1u << 25)) return pfail(err, GGP_ERR_ARG, "lattice coordinates must be < 2^25");
    return 0;
}

int pack_graph(const uint32_t* coords, const int64_t* nbrs, const int64_t* offs, int64_t n_off,
               const int64_t* indices, int64_t n0, int64_t k, int64_t N, int32_t D, bool relabel,
               PackedGraph* out, std::string* err) {
    PackedGraph& P = *out;
    const int64_t M = N - n0;
    // Internal order: inside every refined depth level the points are ordered along a Morton
    // curve of their lattice coordinates, so that the points a chunk of lanes handles are
    // neighbours in space and their gathers (neighbour coordinates and values, consumers) share
    // cache lines. The dense block and any points past the last level keep their positions. No
    // result depends on this order: per-point arithmetic is unchanged and every list keeps the
    // reference's order; ops translate at their boundary (i2t: internal -> tree position).
    std::vector<int32_t>& i2t = P.i2t;
    i2t.assign((size_t)N, 0);
    std::vector<int32_t> t2i((size_t)N);
    for (int64_t i = 0; i < N; ++i) i2t[(size_t)i] = (int32_t)i;
    P.relabel = relabel && M > 0;
    if (P.relabel) {
        uint32_t cmax = 0;
        for (int64_t i = 0; i < N * D; ++i) cmax = std::max(cmax, coords[i]);
        int cbits = 0;
        while (cbits < 32 && (cmax >> cbits) != 0) ++cbits;
        const int per = 63 / D;
        const int drop = std::max(0, cbits - per);
        std::vector<uint64_t> key((size_t)N, 0);
        for (int64_t i = n0; i < N; ++i) {
            uint64_t kk = 0;
            for (int b = per - 1; b >= 0; --b)
                for (int d = 0; d < D; ++d)
                    kk = (kk << 1) | ((coords[i * D + d] >> (b + drop)) & 1u);
            key[(size_t)i] = kk;
        }
        for (int64_t b = 1; b < n_off; ++b) {
            const int64_t lo = offs[b - 1], hi = offs[b];
            std::stable_sort(i2t.begin() + lo, i2t.begin() + hi,
                             [&](int32_t a, int32_t c) { return key[(size_t)a] < key[(size_t)c]; });
        }
    }
    for (int64_t i = 0; i < N; ++i) t2i[(size_t)i2t[(size_t)i]] = (int32_t)i;
    // neighbours: int32 structure of arrays, internal indices
    P.nsoa.assign((size_t)(M * k), 0);
    for (int64_t m = 0; m < M; ++m) {
        const int64_t mt = i2t[(size_t)(n0 + m)] - n0;  // tree index of internal m
        for (int64_t j = 0; j < k; ++j)
            P.nsoa[(size_t)(j * M + m)] = t2i[(size_t)nbrs[mt * k + j]];
    }
    // reverse neighbour list over the points that lie in a level, consumers by decreasing tree
    // position (entries m*k + j with internal m), indexed by internal q
    const int64_t mlev = std::max<int64_t>(0, offs[n_off - 1] - n0);
    std::vector<int64_t> rptr((size_t)N + 1, 0);
    for (int64_t m = 0; m < mlev; ++m)
        for (int64_t j = 0; j < k; ++j) rptr[(size_t)t2i[(size_t)nbrs[m * k + j]] + 1]++;
    for (int64_t q = 0; q < N; ++q) rptr[(size_t)q + 1] += rptr[(size_t)q];
    std::vector<uint32_t> revl((size_t)std::max<int64_t>(rptr[(size_t)N], 1));
    {
        std::vector<int64_t> pos(rptr.begin(), rptr.end() - 1);
        for (int64_t m = mlev - 1; m >= 0; --m) {
            const int64_t mi = t2i[(size_t)(n0 + m)] - n0;
            for (int64_t j = 0; j < k; ++j) {
                const int64_t q = t2i[(size_t)nbrs[m * k + j]];
                revl[(size_t)pos[(size_t)q]++] = (uint32_t)(mi * k + j);
            }
        }
    }
    P.rcnt.assign((size_t)N, 0);
    for (int64_t q = 0; q < N; ++q) P.rcnt[(size_t)q] = (uint32_t)(rptr[(size_t)q + 1] - rptr[(size_t)q]);
    // Chunk lists of the one-launch sweeps (within one level each, topological order).
    P.fwd.clear();
    P.revc.clear();
    for (int64_t b = 1; b < n_off; ++b)
        for (int64_t s0 = offs[b - 1]; s0 < offs[b]; s0 += kPackBlock)
            P.fwd.push_back(Chunk{(int)(s0 - n0), (int)std::min<int64_t>(kPackBlock, offs[b] - s0), 0, 0});
    // Reverse chunks: the fewest lanes per point (2^lg) that keep every lane at kPackRevSlots
    // list entries or fewer (at most 64 lanes; longer lists take several rounds).
    std::vector<uint32_t>& rev = P.rev;
    rev.clear();
    for (int64_t b = n_off - 1; b >= 0; --b) {
        const int64_t lo = b == 0 ? 0 : offs[b - 1], hi = b == 0 ? n0 : offs[b];
        for (int64_t s0 = lo; s0 < hi;) {
            int lg = 0;
            int64_t np = 0, maxc = 0;
            for (;; ++lg) {
                np = std::min<int64_t>(kPackBlock >> lg, hi - s0);
                maxc = 0;
                for (int64_t q = s0; q < s0 + np; ++q) maxc = std::max<int64_t>(maxc, P.rcnt[(size_t)q]);
                if (((maxc + (1 << lg) - 1) >> lg) <= kPackRevSlots || lg == 6) break;
            }
            const int64_t nslots = (maxc + (1 << lg) - 1) >> lg;
            // every chunk's entries start at a multiple of kPackBlock: the chunk stores its base
            // in units of kPackBlock, which holds 2^31 * kPackBlock entries
            const int64_t base = (int64_t)rev.size();
            if ((base >> kPackBaseShift) + nslots >= ((int64_t)1 << 31))
                return pfail(err, GGP_ERR_ARG, "reverse neighbour lists too large");
            rev.resize((size_t)(base + nslots * kPackBlock), kPackRevNone);
            for (int64_t i = 0; i < np; ++i) {
                const int64_t q = s0 + i;
                for (int64_t u = 0; u < (int64_t)P.rcnt[(size_t)q]; ++u) {
                    const int64_t lane = (i << lg) + (u & ((1 << lg) - 1));
                    rev[(size_t)(base + (u >> lg) * kPackBlock + lane)] = revl[(size_t)(rptr[(size_t)q] + u)];
                }
            }
            P.revc.push_back(Chunk{(int)s0, (int)(np | ((int64_t)lg << 16)),
                                   (int)(base >> kPackBaseShift), (int)nslots});
            s0 += np;
        }
    }
    if (rev.empty()) rev.push_back(kPackRevNone);
    // original position of each internal position
    P.idx32.clear();
    if (indices || P.relabel) {
        P.idx32.resize((size_t)N);
        for (int64_t i = 0; i < N; ++i)
            P.idx32[(size_t)i] = indices ? (int32_t)indices[i2t[(size_t)i]] : i2t[(size_t)i];
    }
    P.coords.assign((size_t)(N * D), 0);
    for (int64_t i = 0; i < N; ++i)
        for (int d = 0; d < D; ++d)
            P.coords[(size_t)(i * D + d)] = coords[(int64_t)i2t[(size_t)i] * D + d];
    P.i2tm.assign((size_t)std::max<int64_t>(M, 1), 0);
    for (int64_t m = 0; m < M; ++m) P.i2tm[(size_t)m] = i2t[(size_t)(n0 + m)] - (int32_t)n0;
    return 0;
}

}  // namespace ggp
