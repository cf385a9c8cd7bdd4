// ggp_pack.h — host-side validation and repacking of a problem's graph for the device (the work
// of ggp_graph_create before any upload). Plain C++ with no HIP dependency, so it also builds
// with the host compiler alone (the sanitizer build of the tests).
#pragma once
#include <stdint.h>

#include <string>
#include <vector>

namespace ggp {

constexpr int kPackBlock = 256;    // lanes per chunk of the one-launch sweeps (= kBlock)
constexpr int kPackRevSlots = 16;  // reverse sweep: list entries per lane fetched together
constexpr uint32_t kPackRevNone = 0xffffffffu;
constexpr int kPackBaseShift = 8;  // reverse chunk bases are stored in units of 2^8 = kPackBlock
static_assert((1 << kPackBaseShift) == kPackBlock, "chunk bases are multiples of the chunk width");

// One work chunk of a sweep, in the layout of the device's int4.
struct alignas(16) Chunk {
    int x, y, z, w;
};

// The device layout of a graph (ggp_internal.h, struct Graph), built on the host.
struct PackedGraph {
    bool relabel = false;               // internal order differs from tree order
    std::vector<int32_t> i2t;           // N: tree position of each internal position
    std::vector<int32_t> i2tm;          // max(M, 1): the same for refined indices
    std::vector<int32_t> nsoa;          // K*M: nbr[j*M + m], internal indices
    std::vector<uint32_t> rcnt;         // N: consumers of each internal position
    std::vector<uint32_t> rev;          // reverse lists, lane-major per reverse chunk
    std::vector<Chunk> fwd, revc;       // sweep chunks in topological order (revc: {first
                                        // position, points | lg << 16, base / kPackBlock, slots})
    std::vector<int32_t> idx32;         // N original positions (empty: identity)
    std::vector<uint32_t> coords;       // N*D, internal order
};

// check_graph (src/graph_build.jl:20-57) on the host arrays of ggp_graph_create, and the
// argument limits of the library. Returns 0 or a GGP_ERR_* status with *err set.
int check_graph_host(const uint32_t* coords, const int64_t* nbrs, const int64_t* offs,
                     int64_t n_off, const int64_t* indices, int64_t n0, int64_t k, int64_t N,
                     int32_t D, std::string* err);

// The device layout of a validated graph: the internal order (every refined level along a
// Morton curve of its lattice coordinates when `relabel`), the int32 structure-of-arrays
// neighbour table, the reverse-neighbour lists and the sweep chunks. Returns 0 or a GGP_ERR_*
// status with *err set.
int pack_graph(const uint32_t* coords, const int64_t* nbrs, const int64_t* offs, int64_t n_off,
               const int64_t* indices, int64_t n0, int64_t k, int64_t N, int32_t D, bool relabel,
               PackedGraph* out, std::string* err);

}  // namespace ggp
