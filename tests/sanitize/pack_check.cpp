// pack_check — runs the host code of ggp_graph_create (check_graph_host, pack_graph) and the
// host graph builder (ggp_build_graph) on graph files the tests write, under the sanitizers of
// the build, and checks the invariants of the packed layout. Prints "ok" and exits 0 when every
// check holds.
//
//   pack_check graph <file>   file: int64 N, D, n0, k, n_off, has_indices; uint32 coords[N*D];
//                             int64 neighbors[(N-n0)*k]; int64 offsets[n_off];
//                             int64 indices[N] (if has_indices)
//   pack_check build <file>   file: int64 N, D, n0, k; double points[N*D]; builds the graph and
//                             packs it
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "../../include/graphgp_graph.h"
#include "../../include/graphgp_hip.h"
#include "ggp_pack.h"

using namespace ggp;

static int bad(const char* what) {
    std::fprintf(stderr, "FAIL: %s\n", what);
    return 1;
}

template <typename T>
static bool read_vec(FILE* f, std::vector<T>& v, size_t n) {
    v.resize(n);
    return n == 0 || std::fread(v.data(), sizeof(T), n, f) == n;
}

// Invariants of one packing of a validated graph.
static int check_pack(const std::vector<uint32_t>& coords, const std::vector<int64_t>& nbrs,
                      const std::vector<int64_t>& offs, const int64_t* indices, int64_t N,
                      int64_t D, int64_t n0, int64_t k, bool relabel) {
    PackedGraph P;
    std::string err;
    const int rc = pack_graph(coords.data(), nbrs.data(), offs.data(), (int64_t)offs.size(),
                              indices, n0, k, N, (int32_t)D, relabel, &P, &err);
    if (rc) return bad(err.c_str());
    const int64_t M = N - n0, n_off = (int64_t)offs.size();
    // internal order: a permutation that keeps every point inside its level
    std::vector<int32_t> t2i((size_t)N, -1);
    for (int64_t i = 0; i < N; ++i) {
        const int32_t t = P.i2t[(size_t)i];
        if (t < 0 || t >= N || t2i[(size_t)t] != -1) return bad("i2t is not a permutation");
        t2i[(size_t)t] = (int32_t)i;
    }
    std::vector<int64_t> level((size_t)N, n_off);  // level of each tree position (0: dense)
    for (int64_t i = 0; i < n0; ++i) level[(size_t)i] = 0;
    for (int64_t b = 1; b < n_off; ++b)
        for (int64_t p = offs[b - 1]; p < offs[b]; ++p) level[(size_t)p] = b;
    for (int64_t i = 0; i < N; ++i)
        if (level[(size_t)i] != level[(size_t)P.i2t[(size_t)i]]) return bad("relabel crosses a level");
    for (int64_t m = 0; m < M; ++m)
        if (P.i2tm[(size_t)m] != P.i2t[(size_t)(n0 + m)] - n0) return bad("i2tm");
    // neighbours: the tree table through the internal order
    if ((int64_t)P.nsoa.size() != M * k) return bad("nsoa size");
    for (int64_t m = 0; m < M; ++m) {
        const int64_t mt = P.i2t[(size_t)(n0 + m)] - n0;
        for (int64_t j = 0; j < k; ++j)
            if (P.nsoa[(size_t)(j * M + m)] != t2i[(size_t)nbrs[(size_t)(mt * k + j)]])
                return bad("nsoa entry");
    }
    // reverse lists: q's list holds every (m, j) with nbr (m, j) = q, consumers decreasing
    const int64_t last = offs[(size_t)(n_off - 1)];
    std::vector<int64_t> seen((size_t)(M * k), 0);
    std::vector<char> covered((size_t)N, 0);
    int64_t prev_level = n_off + 1;
    for (const Chunk& c : P.revc) {
        const int lg = c.y >> 16, np = c.y & 0xffff;
        const int64_t base = (int64_t)c.z << kPackBaseShift, nslots = c.w;
        if (np < 1 || np > (kPackBlock >> lg)) return bad("reverse chunk size");
        if (base < 0 || base + nslots * kPackBlock > (int64_t)P.rev.size()) return bad("reverse chunk range");
        const int64_t lv = level[(size_t)P.i2t[(size_t)c.x]];
        if (lv > prev_level) return bad("reverse chunks out of topological order");
        prev_level = lv;
        for (int i = 0; i < np; ++i) {
            const int64_t q = c.x + i;
            if (q >= N || covered[(size_t)q]) return bad("reverse chunk coverage");
            covered[(size_t)q] = 1;
            if (level[(size_t)P.i2t[(size_t)q]] != lv) return bad("reverse chunk spans levels");
            const int64_t cnt = P.rcnt[(size_t)q];
            if (((cnt + (1 << lg) - 1) >> lg) > nslots) return bad("list longer than the chunk's slots");
            int64_t prev_consumer = N;
            for (int64_t u = 0; u < cnt; ++u) {
                const int64_t lane = ((int64_t)i << lg) + (u & ((1 << lg) - 1));
                const uint32_t e = P.rev[(size_t)(base + (u >> lg) * kPackBlock + lane)];
                if (e == kPackRevNone || (int64_t)e >= M * k) return bad("list entry");
                const int64_t m = e / k, j = e % k;
                if (P.nsoa[(size_t)(j * M + m)] != q) return bad("list entry is not a consumer");
                const int64_t consumer_tree = P.i2t[(size_t)(n0 + m)];
                if (consumer_tree > prev_consumer) return bad("consumers not by decreasing position");
                prev_consumer = consumer_tree;
                seen[(size_t)e]++;
            }
        }
    }
    for (int64_t q = 0; q < last; ++q)
        if (!covered[(size_t)q]) return bad("a point of a level is in no reverse chunk");
    for (int64_t m = 0; m < M; ++m)
        if (P.i2t[(size_t)(n0 + m)] < last)
            for (int64_t j = 0; j < k; ++j)
                if (seen[(size_t)(m * k + j)] != 1) return bad("a consumer entry is missing or repeated");
    // forward chunks: every refined point of a level exactly once, level by level
    std::vector<char> fcov((size_t)(M > 0 ? M : 1), 0);
    int64_t plv = 0;
    for (const Chunk& c : P.fwd) {
        if (c.y < 1 || c.y > kPackBlock) return bad("forward chunk size");
        const int64_t lv = level[(size_t)(n0 + c.x)];
        if (lv < plv) return bad("forward chunks out of order");
        plv = lv;
        for (int i = 0; i < c.y; ++i) {
            const int64_t m = c.x + i;
            if (m >= M || fcov[(size_t)m] || level[(size_t)(n0 + m)] != lv) return bad("forward chunk coverage");
            fcov[(size_t)m] = 1;
        }
    }
    for (int64_t m = 0; m < M; ++m)
        if ((n0 + m < last) != (bool)fcov[(size_t)m]) return bad("forward chunks miss a point");
    // original positions and coordinates in internal order
    if (!P.idx32.empty()) {
        std::vector<char> hit((size_t)N, 0);
        for (int64_t i = 0; i < N; ++i) {
            const int64_t o = P.idx32[(size_t)i];
            const int64_t want = indices ? indices[P.i2t[(size_t)i]] : P.i2t[(size_t)i];
            if (o != want || hit[(size_t)o]) return bad("idx32");
            hit[(size_t)o] = 1;
        }
    } else if (indices || P.relabel) {
        return bad("idx32 missing");
    }
    for (int64_t i = 0; i < N; ++i)
        for (int64_t d = 0; d < D; ++d)
            if (P.coords[(size_t)(i * D + d)] != coords[(size_t)(P.i2t[(size_t)i] * D + d)])
                return bad("coords");
    return 0;
}

static int check_graph_file(const char* path) {
    FILE* f = std::fopen(path, "rb");
    if (!f) return bad("cannot open the graph file");
    int64_t hdr[6];
    if (std::fread(hdr, sizeof(int64_t), 6, f) != 6) return bad("header");
    const int64_t N = hdr[0], D = hdr[1], n0 = hdr[2], k = hdr[3], n_off = hdr[4], has_idx = hdr[5];
    std::vector<uint32_t> coords;
    std::vector<int64_t> nbrs, offs, idx;
    if (!read_vec(f, coords, (size_t)(N * D)) || !read_vec(f, nbrs, (size_t)((N - n0) * k)) ||
        !read_vec(f, offs, (size_t)n_off) || (has_idx && !read_vec(f, idx, (size_t)N)))
        return bad("short graph file");
    std::fclose(f);
    std::string err;
    const int64_t* ip = has_idx ? idx.data() : nullptr;
    if (int rc = check_graph_host(coords.data(), nbrs.data(), offs.data(), n_off, ip, n0, k, N,
                                  (int32_t)D, &err)) {
        std::printf("rejected %d %s\n", rc, err.c_str());
        return 0;  // a rejection is a result too: the test compares the code
    }
    for (bool relabel : {true, false})
        if (int rc = check_pack(coords, nbrs, offs, ip, N, D, n0, k, relabel)) return rc;
    std::printf("ok\n");
    return 0;
}

static int check_build_file(const char* path) {
    FILE* f = std::fopen(path, "rb");
    if (!f) return bad("cannot open the points file");
    int64_t hdr[4];
    if (std::fread(hdr, sizeof(int64_t), 4, f) != 4) return bad("header");
    const int64_t N = hdr[0], D = hdr[1], n0 = hdr[2], k = hdr[3];
    std::vector<double> pts;
    if (!read_vec(f, pts, (size_t)(N * D))) return bad("short points file");
    std::fclose(f);
    ggp_built_graph* g = nullptr;
    if (ggp_build_graph(pts.data(), N, (int32_t)D, n0, k, 21, 0, &g) != 0) return bad("build");
    int64_t gN, gn0, gk, noff;
    int32_t gD;
    ggp_built_graph_shape(g, &gN, &gn0, &gk, &gD, &noff);
    std::vector<uint32_t> coords((size_t)(gN * gD));
    std::vector<int64_t> nbrs((size_t)((gN - gn0) * gk)), offs((size_t)noff), idx((size_t)gN);
    double scale = 0;
    ggp_built_graph_copy(g, coords.data(), nbrs.data(), offs.data(), idx.data(), &scale);
    ggp_built_graph_free(g);
    std::string err;
    if (int rc = check_graph_host(coords.data(), nbrs.data(), offs.data(), noff, idx.data(), gn0,
                                  gk, gN, gD, &err)) {
        std::fprintf(stderr, "built graph rejected (%d): %s\n", rc, err.c_str());
        return 1;
    }
    for (bool relabel : {true, false})
        if (int rc = check_pack(coords, nbrs, offs, idx.data(), gN, gD, gn0, gk, relabel)) return rc;
    std::printf("ok %lld levels\n", (long long)(noff - 1));
    return 0;
}

int main(int argc, char** argv) {
    if (argc != 3) return bad("usage: pack_check graph|build <file>");
    const std::string mode = argv[1];
    if (mode == "graph") return check_graph_file(argv[2]);
    if (mode == "build") return check_build_file(argv[2]);
    return bad("unknown mode");
}
