// ggp_graph_gpu.hip — the refinement graph built on the GPU (ggp_build_graph_device in
// include/graphgp_hip.h).
//
// The same pipeline as the host builder (graph_build.cpp) and the reference's CPU build_graph
// (src/graph_build.jl:254-288), with its tie-breaking, so the two builders return the same
// graph bit for bit:
//   1. heap-order ("special order") k-d tree (build_tree_special, src/tree_special.jl:165-227),
//      one pass per tree level. At level L the points still unplaced lie in 2^L contiguous
//      segments whose sizes follow from N and L alone. Per level: segment extents and split
//      dimension (a wavefront per segment chunk), the order (segment, split coordinate,
//      position) by two stable radix sorts (coordinate first, then segment), and one scatter
//      that places each segment's median at its node position and the two halves at the
//      children's segments of the next level.
//   2. stackless preceding k-nearest-neighbour query (src/tree_special.jl:231-332), one lane per
//      refined point, candidates in registers;
//   3. depths by relaxation to the fixed point of depth[p] = 1 + max depth[neighbours]
//      (compute_depths, src/graph_build.jl:69-93), then a stable radix sort by depth
//      (order_by_depth, src/graph_build.jl:160-200);
//   4. lattice quantization (src/graph_build.jl:231-242) and level offsets (:213-221).
// Coordinates stay in double throughout, and every comparison and distance is the host
// builder's expression (-ffp-contract=off on both sides).
#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <limits>
#include <string>
#include <vector>

#include "../../include/graphgp_hip.h"
#include "ggp_internal.h"

namespace {

using ggp::set_error;

constexpr int kGbBlock = 256;
constexpr int64_t kChunk = 2048;  // positions per wavefront in the segment-extent pass

// Level L of the tree: nodes [n_above, n_above + n_level); the n_rem unplaced points form
// n_level segments in node order, the first r of q+1 points, the rest of q.
struct Geom {
    int64_t n_above, n_level, q, r;
};
__host__ __device__ inline Geom geom(int L, int64_t N) {
    Geom g;
    g.n_level = (int64_t)1 << L;
    g.n_above = g.n_level - 1;
    const int64_t rem = N - g.n_above;
    g.q = rem / g.n_level;
    g.r = rem % g.n_level;
    return g;
}
__host__ __device__ inline int64_t seg_start(const Geom& g, int64_t ii) {
    return g.n_above + (ii < g.r ? ii * (g.q + 1) : g.r * (g.q + 1) + (ii - g.r) * g.q);
}
__host__ __device__ inline int64_t seg_size(const Geom& g, int64_t ii) {
    return ii < g.r ? g.q + 1 : g.q;
}
// Segment of position i >= n_above (positions past the first r segments exist only if q > 0).
__device__ inline int64_t seg_of(const Geom& g, int64_t i) {
    const int64_t t = i - g.n_above, big = g.r * (g.q + 1);
    return t < big ? t / (g.q + 1) : g.r + (t - big) / g.q;
}

// ---- 1. tree -------------------------------------------------------------------------------
// Segment extents per dimension; split = the first dimension of largest extent. A wavefront
// covers kChunk positions of one segment; with one chunk per segment it writes the split
// itself, otherwise per-chunk extents for k_tree_split.
// One (segment, chunk) task of k_tree_extent on one wavefront.
template <int D>
__device__ inline void extent_task(const double* __restrict__ pts, const Geom& g, int gps,
                                   int64_t w, int lane, double* __restrict__ pmin,
                                   double* __restrict__ pmax, int8_t* __restrict__ split) {
    const int64_t ii = w / gps;
    const int c = (int)(w % gps);
    const int64_t s0 = seg_start(g, ii), end = s0 + seg_size(g, ii);
    const int64_t lo = s0 + c * kChunk, hi = std::min(end, lo + kChunk);
    double mn[D], mx[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        mn[d] = INFINITY;
        mx[d] = -INFINITY;
    }
    for (int64_t i = lo + lane; i < hi; i += 64)
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const double v = pts[i * D + d];
            mn[d] = fmin(mn[d], v);
            mx[d] = fmax(mx[d], v);
        }
#pragma unroll
    for (int d = 0; d < D; ++d)
        for (int o = 32; o > 0; o >>= 1) {
            mn[d] = fmin(mn[d], __shfl_xor(mn[d], o, 64));
            mx[d] = fmax(mx[d], __shfl_xor(mx[d], o, 64));
        }
    if (lane != 0) return;
    if (gps == 1) {
        int bd = 0;
        double br = -INFINITY;
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const double r = mx[d] - mn[d];
            if (r > br) { br = r; bd = d; }
        }
        split[g.n_above + ii] = (int8_t)bd;
    } else {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            pmin[w * D + d] = mn[d];
            pmax[w * D + d] = mx[d];
        }
    }
}

template <int D>
__global__ void __launch_bounds__(kGbBlock)
k_tree_extent(const double* __restrict__ pts, Geom g, int64_t nseg, int gps,
              double* __restrict__ pmin, double* __restrict__ pmax, int8_t* __restrict__ split) {
    const int lane = threadIdx.x & 63;
    // one wavefront per (segment, chunk) task, grid-stride: a deep level of a large build has
    // more tasks than a launch may hold wavefronts (at most 2^32 work-items per dimension)
    const int64_t wstride = ((int64_t)gridDim.x * blockDim.x) >> 6;
    for (int64_t w = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6; w < nseg * gps;
         w += wstride)  // uniform per wavefront
        extent_task<D>(pts, g, gps, w, lane, pmin, pmax, split);
}

template <int D>
__global__ void k_tree_split(const double* __restrict__ pmin, const double* __restrict__ pmax,
                             Geom g, int64_t nseg, int gps, int8_t* __restrict__ split) {
    const int64_t ii = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (ii >= nseg) return;
    int bd = 0;
    double br = -INFINITY;
#pragma unroll
    for (int d = 0; d < D; ++d) {
        double mn = INFINITY, mx = -INFINITY;
        for (int c = 0; c < gps; ++c) {
            mn = fmin(mn, pmin[(ii * gps + c) * D + d]);
            mx = fmax(mx, pmax[(ii * gps + c) * D + d]);
        }
        const double r = mx - mn;
        if (r > br) { br = r; bd = d; }
    }
    split[g.n_above + ii] = (int8_t)bd;
}

// Order-preserving unsigned key of a double; -0 and +0 map to one key (the host builder's
// comparison `<` treats them as equal, so their order is decided by position).
__device__ inline uint64_t order_key(double x) {
    const double y = x == 0.0 ? 0.0 : x;
    const uint64_t u = (uint64_t)__double_as_longlong(y);
    return (u >> 63) ? ~u : (u | (1ull << 63));
}

template <int D>
__global__ void k_tree_keys(const double* __restrict__ pts, Geom g, int64_t n_items,
                            const int8_t* __restrict__ split, uint64_t* __restrict__ key,
                            int32_t* __restrict__ val) {
    const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= n_items) return;
    const int64_t i = g.n_above + j;
    const int d = split[g.n_above + seg_of(g, i)];
    key[j] = order_key(pts[i * D + d]);
    val[j] = (int32_t)i;
}

__global__ void k_tree_segkeys(Geom g, int64_t n_items, const int32_t* __restrict__ val,
                               uint32_t* __restrict__ key) {
    const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j < n_items) key[j] = (uint32_t)seg_of(g, val[j]);
}

// Place the sorted segment contents: the median (position start + size/2) at its node
// position, the lower half at the left child's segment, the upper half at the right child's
// (children s + 2^L and s + 2^(L+1), src/tree_special.jl:165-227). Placed positions are
// copied through.
template <int D>
__global__ void k_tree_place(Geom g, Geom gn, int64_t N, const int32_t* __restrict__ src_of,
                             const double* __restrict__ pa, const int32_t* __restrict__ perm_a,
                             double* __restrict__ pb, int32_t* __restrict__ perm_b) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= N) return;
    int64_t src, dest;
    if (t < g.n_above) {
        src = dest = t;
    } else {
        src = src_of[t - g.n_above];
        const int64_t ii = seg_of(g, t);
        const int64_t start = seg_start(g, ii), mid = start + seg_size(g, ii) / 2;
        if (t == mid)
            dest = g.n_above + ii;
        else if (t < mid)
            dest = seg_start(gn, ii) + (t - start);
        else
            dest = seg_start(gn, ii + g.n_level) + (t - mid - 1);
    }
#pragma unroll
    for (int d = 0; d < D; ++d) pb[dest * D + d] = pa[src * D + d];
    perm_b[dest] = perm_a[src];
}

// ---- 2. preceding k-nearest neighbours (_sp_query_one!, src/tree_special.jl:231-300) --------
__device__ inline int flevel(int64_t x) { return 63 - __clzll((unsigned long long)x); }
__device__ inline int64_t sp_parent(int64_t c) {
    if (c == 0) return -1;
    const int level = flevel(c + 1);
    const int64_t n_above = ((int64_t)1 << level) - 1;
    const int64_t npl = (int64_t)1 << (level - 1);
    return c < n_above + npl ? c - npl : c - 2 * npl;
}
__device__ inline int64_t sp_left(int64_t c) { return c + ((int64_t)1 << flevel(c + 1)); }
__device__ inline int64_t sp_right(int64_t c) { return c + 2 * ((int64_t)1 << flevel(c + 1)); }

// Candidates live in registers: every loop over them is unrolled to KM with a run-time bound
// k <= KM, and the slot to replace is selected, never indexed.
template <int D, int KM>
__global__ void __launch_bounds__(kGbBlock)
k_knn(const double* __restrict__ pts, const int8_t* __restrict__ split, int64_t N, int64_t n0,
      int k, int32_t* __restrict__ nbr) {
    const int64_t m = n0 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (m >= N) return;
    double cd[KM];
    int32_t ci[KM];
#pragma unroll
    for (int j = 0; j < KM; ++j) { cd[j] = INFINITY; ci[j] = -1; }
    double qp[D];
#pragma unroll
    for (int d = 0; d < D; ++d) qp[d] = pts[m * D + d];
    double square_radius = INFINITY;
    const int64_t max_index = m;
    int64_t current = 0, previous = -1;
    while (current != -1) {
        const int64_t parent = sp_parent(current);
        if (previous == parent) {
            double sq = 0.0;
#pragma unroll
            for (int d = 0; d < D; ++d) {
                const double dv = qp[d] - pts[current * D + d];
                sq += dv * dv;
            }
            int wpos = 0;
            double wval = cd[0];
#pragma unroll
            for (int j = 1; j < KM; ++j)
                if (j < k && cd[j] > wval) { wval = cd[j]; wpos = j; }
            if (sq < wval) {
#pragma unroll
                for (int j = 0; j < KM; ++j)
                    if (j == wpos) { cd[j] = sq; ci[j] = (int32_t)current; }
                double mx = cd[0];
#pragma unroll
                for (int j = 1; j < KM; ++j)
                    if (j < k && cd[j] > mx) mx = cd[j];
                square_radius = mx;
            } else {
                square_radius = wval;
            }
        }
        const int sd = split[current];
        double qs = qp[0];
#pragma unroll
        for (int d = 1; d < D; ++d)
            if (d == sd) qs = qp[d];
        const double split_distance = qs - pts[current * D + sd];
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
    // ascending (distance, index): a transposition network over the unrolled slots
#pragma unroll
    for (int pass = 0; pass < KM; ++pass)
#pragma unroll
        for (int j = pass & 1; j + 1 < KM; j += 2)
            if (j + 1 < k) {
                const bool sw = cd[j] > cd[j + 1] || (cd[j] == cd[j + 1] && ci[j] > ci[j + 1]);
                const double a = cd[j], b = cd[j + 1];
                const int32_t x = ci[j], y = ci[j + 1];
                cd[j] = sw ? b : a;
                cd[j + 1] = sw ? a : b;
                ci[j] = sw ? y : x;
                ci[j + 1] = sw ? x : y;
            }
    int32_t* out = nbr + (m - n0) * k;
#pragma unroll
    for (int j = 0; j < KM; ++j)
        if (j < k) out[j] = ci[j];
}

// ---- 3. depths and the order by depth --------------------------------------------------------
// depth[n0+m] = 1 + max(0, depth[neighbours]) (compute_depths, src/graph_build.jl:69-93) in one
// pass: refined points in position order (neighbours precede their point), 256 per chunk,
// chunks taken by ticket, so a chunk only waits for chunks already taken by running
// workgroups. Depths start at -1 (pending) and are published once. A wavefront retries its
// lanes whose inputs are still pending, so no lane ever waits for a lane of its own
// wavefront; later wavefronts only wait for earlier ones. Bounded: past the limit the
// wavefront sets *err and stops.
constexpr int kDepthSpinLimit = 1 << 22;
__global__ void __launch_bounds__(kGbBlock)
k_depth_flow(const int32_t* __restrict__ nbr, int64_t n0, int64_t M, int k, int32_t* depth,
             int* ticket, int* err) {
    __shared__ int s_c;
    const int64_t nchunks = (M + kGbBlock - 1) / kGbBlock;
    for (;;) {
        __syncthreads();
        if (threadIdx.x == 0) s_c = atomicAdd(ticket, 1);
        __syncthreads();
        const int c = __builtin_amdgcn_readfirstlane(s_c);
        if (c >= nchunks) break;
        const int64_t m = (int64_t)c * kGbBlock + threadIdx.x;
        bool done = m >= M;
        for (int spins = 0;; ++spins) {
            if (!done) {
                int32_t mx = 0;
                bool ready = true;
                for (int j = 0; j < k; ++j) {
                    const int32_t d = __hip_atomic_load(&depth[nbr[m * k + j]], __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT);
                    ready = ready && d >= 0;
                    mx = d > mx ? d : mx;
                }
                if (ready) {
                    __hip_atomic_store(&depth[n0 + m], mx + 1, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                    done = true;
                }
            }
            if (__all(done)) break;
            if (spins > kDepthSpinLimit) {
                if (!done) atomicOr(err, 1);
                break;
            }
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "agent");
            __builtin_amdgcn_s_sleep(1);
        }
    }
}

__global__ void k_iota(int32_t* __restrict__ x, int64_t n, int64_t base) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] = (int32_t)(base + i);
}

__global__ void k_fill_i32(int32_t* __restrict__ x, int32_t v, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] = v;
}

template <int D>
__global__ void k_depth_gather(int64_t N, const int32_t* __restrict__ sp,
                               const double* __restrict__ pts, const int32_t* __restrict__ perm,
                               const uint32_t* __restrict__ depth, double* __restrict__ spts,
                               int64_t* __restrict__ indices, uint32_t* __restrict__ sdepth,
                               int32_t* __restrict__ inv) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N) return;
    const int64_t s = sp[i];
#pragma unroll
    for (int d = 0; d < D; ++d) spts[i * D + d] = pts[s * D + d];
    indices[i] = perm[s];
    sdepth[i] = depth[s];
    inv[s] = (int32_t)i;
}

__global__ void k_nbr_remap(const int32_t* __restrict__ nbr, const int32_t* __restrict__ inv,
                            int64_t n0, int64_t M, int k, int64_t* __restrict__ out) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;  // M*k may pass 2^32
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < M * k; t += stride) {
        const int64_t m_old = t / k, j = t % k;
        const int64_t m_new = inv[n0 + m_old] - n0;
        out[m_new * k + j] = inv[nbr[t]];
    }
}

// ---- 4. lattice and offsets -----------------------------------------------------------------
template <int D>
__global__ void __launch_bounds__(kGbBlock)
k_bbox(const double* __restrict__ pts, int64_t N, double* __restrict__ part) {
    __shared__ double s[kGbBlock / 64][2 * D];
    double mn[D], mx[D];
#pragma unroll
    for (int d = 0; d < D; ++d) { mn[d] = INFINITY; mx[d] = -INFINITY; }
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < N;
         i += (int64_t)gridDim.x * blockDim.x)
#pragma unroll
        for (int d = 0; d < D; ++d) {
            mn[d] = fmin(mn[d], pts[i * D + d]);
            mx[d] = fmax(mx[d], pts[i * D + d]);
        }
#pragma unroll
    for (int d = 0; d < D; ++d)
        for (int o = 32; o > 0; o >>= 1) {
            mn[d] = fmin(mn[d], __shfl_xor(mn[d], o, 64));
            mx[d] = fmax(mx[d], __shfl_xor(mx[d], o, 64));
        }
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (lane == 0)
#pragma unroll
        for (int d = 0; d < D; ++d) { s[w][d] = mn[d]; s[w][D + d] = mx[d]; }
    __syncthreads();
    if (threadIdx.x == 0)
#pragma unroll
        for (int d = 0; d < D; ++d) {
            double a = s[0][d], b = s[0][D + d];
            for (int q = 1; q < kGbBlock / 64; ++q) { a = fmin(a, s[q][d]); b = fmax(b, s[q][D + d]); }
            part[blockIdx.x * 2 * D + d] = a;
            part[blockIdx.x * 2 * D + D + d] = b;
        }
}

struct Origin {
    double o[4];
};

// round(Int64, (x - origin) / scale), ties to even, clamped to the lattice.
template <int D>
__global__ void k_quantize(const double* __restrict__ spts, int64_t N, Origin org, double scale,
                           double lmax, uint32_t* __restrict__ coords) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;  // N*D may pass 2^32
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < N * D; t += stride) {
        const int d = (int)(t % D);
        const double c = rint((spts[t] - org.o[d]) / scale);
        coords[t] = (uint32_t)fmin(fmax(c, 0.0), lmax);
    }
}

__global__ void k_level_ends(const uint32_t* __restrict__ sdepth, int64_t N,
                             int64_t* __restrict__ offs) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N) return;
    if (i == N - 1 || sdepth[i] != sdepth[i + 1]) offs[sdepth[i]] = i + 1;
}

inline unsigned nblocks(int64_t n) { return (unsigned)((n + kGbBlock - 1) / kGbBlock); }
// Grid of a grid-stride kernel: at most 2^20 workgroups (2^28 work-items).
inline unsigned nblocks_capped(int64_t n) {
    return (unsigned)std::min<int64_t>((n + kGbBlock - 1) / kGbBlock, (int64_t)1 << 20);
}

// ---- the pipeline --------------------------------------------------------------------------
struct Bufs {
    std::vector<void*> owned;
    ~Bufs() {
        for (void* p : owned) (void)hipFree(p);
    }
    template <typename T>
    T* get(size_t n) {
        void* p = nullptr;
        if (hipMalloc(&p, std::max<size_t>(n, 1) * sizeof(T)) != hipSuccess) return nullptr;
        owned.push_back(p);
        return static_cast<T*>(p);
    }
};

#define GB_HC(x)                                                                               \
    do {                                                                                       \
        hipError_t e_ = (x);                                                                   \
        if (e_ != hipSuccess)                                                                  \
            return set_error(GGP_ERR_HIP, std::string(#x) + ": " + hipGetErrorString(e_));    \
    } while (0)
#define GB_ALLOC(p, T, n)                                                                      \
    T* p = bufs.get<T>(n);                                                                     \
    if (!p) return set_error(GGP_ERR_HIP, "hipMalloc failed in the graph build")

template <int D, int KM>
int build(const double* points, int64_t N, int64_t n0, int k, int lattice_bits, uint32_t* coords,
          int64_t* neighbors, int64_t* indices, int64_t* offsets_host, int64_t offsets_cap,
          int64_t* n_offsets, double* scale_out, hipStream_t st) {
    Bufs bufs;
    const int64_t M = N - n0;
    const int n_levels = 64 - __builtin_clzll((unsigned long long)N);  // floor(log2 N) + 1
    GB_ALLOC(pa, double, N * D);
    GB_ALLOC(pb, double, N * D);
    GB_ALLOC(perm_a, int32_t, N);
    GB_ALLOC(perm_b, int32_t, N);
    GB_ALLOC(split, int8_t, N);
    GB_ALLOC(key64a, uint64_t, N);
    GB_ALLOC(key64b, uint64_t, N);
    GB_ALLOC(val_a, int32_t, N);
    GB_ALLOC(val_b, int32_t, N);
    // 32-bit keys reuse the 64-bit key buffers
    uint32_t* key32a = reinterpret_cast<uint32_t*>(key64a);
    uint32_t* key32b = reinterpret_cast<uint32_t*>(key64b);
    const int64_t max_parts = (N + kChunk - 1) / kChunk + 1;
    GB_ALLOC(pmin, double, max_parts * D);
    GB_ALLOC(pmax, double, max_parts * D);
    size_t tmp_bytes = 0, t2 = 0;
    GB_HC(hipcub::DeviceRadixSort::SortPairs(nullptr, tmp_bytes, key64a, key64b, val_a, val_b,
                                             (int)N, 0, 64, st));
    GB_HC(hipcub::DeviceRadixSort::SortPairs(nullptr, t2, key32a, key32b, val_a, val_b, (int)N,
                                             0, 32, st));
    tmp_bytes = std::max(tmp_bytes, t2);
    GB_ALLOC(tmp, unsigned char, tmp_bytes);

    GB_HC(hipMemcpyAsync(pa, points, (size_t)N * D * sizeof(double), hipMemcpyDeviceToDevice, st));
    hipLaunchKernelGGL(k_iota, dim3(nblocks(N)), dim3(kGbBlock), 0, st, perm_a, N, (int64_t)0);

    // 1. tree: level L places the medians of its 2^L segments
    for (int L = 0; L < n_levels; ++L) {
        const Geom g = geom(L, N), gn = geom(L + 1, N);
        const int64_t n_items = N - g.n_above;
        const int64_t nseg = g.q > 0 ? g.n_level : g.r;
        const int gps = (int)((g.q + 1 + kChunk - 1) / kChunk);
        hipLaunchKernelGGL((k_tree_extent<D>), dim3(nblocks_capped(nseg * gps * 64)), dim3(kGbBlock), 0,
                           st, pa, g, nseg, gps, pmin, pmax, split);
        if (gps > 1)
            hipLaunchKernelGGL((k_tree_split<D>), dim3(nblocks(nseg)), dim3(kGbBlock), 0, st,
                               pmin, pmax, g, nseg, gps, split);
        const int32_t* src_of;
        if (g.q + (g.r > 0 ? 1 : 0) <= 1) {
            // every segment holds at most one point: each is its own median
            hipLaunchKernelGGL(k_iota, dim3(nblocks(n_items)), dim3(kGbBlock), 0, st, val_b,
                               n_items, g.n_above);
            src_of = val_b;
        } else {
            // order (segment, split coordinate, position): stable sort by the coordinate, then
            // a stable sort by segment
            hipLaunchKernelGGL((k_tree_keys<D>), dim3(nblocks(n_items)), dim3(kGbBlock), 0, st,
                               pa, g, n_items, split, key64a, val_a);
            size_t tb = tmp_bytes;
            GB_HC(hipcub::DeviceRadixSort::SortPairs(tmp, tb, key64a, key64b, val_a, val_b,
                                                     (int)n_items, 0, 64, st));
            src_of = val_b;
            if (nseg > 1) {
                hipLaunchKernelGGL(k_tree_segkeys, dim3(nblocks(n_items)), dim3(kGbBlock), 0, st,
                                   g, n_items, val_b, key32a);
                tb = tmp_bytes;
                GB_HC(hipcub::DeviceRadixSort::SortPairs(tmp, tb, key32a, key32b, val_b, val_a,
                                                         (int)n_items, 0, L + 1, st));
                src_of = val_a;
            }
        }
        hipLaunchKernelGGL((k_tree_place<D>), dim3(nblocks(N)), dim3(kGbBlock), 0, st, g, gn, N,
                           src_of, pa, perm_a, pb, perm_b);
        std::swap(pa, pb);
        std::swap(perm_a, perm_b);
    }

    // 2. neighbours (tree positions), M x k
    GB_ALLOC(nbr, int32_t, M * k);
    hipLaunchKernelGGL((k_knn<D, KM>), dim3(nblocks(M)), dim3(kGbBlock), 0, st, pa, split, N, n0,
                       k, nbr);

    // 3. depths, then the stable order by depth
    GB_ALLOC(depth, int32_t, N);
    GB_ALLOC(sync2, int, 2);  // ticket, error
    hipLaunchKernelGGL(k_fill_i32, dim3(nblocks(N)), dim3(kGbBlock), 0, st, depth, -1, N);
    hipLaunchKernelGGL(k_fill_i32, dim3(nblocks(n0)), dim3(kGbBlock), 0, st, depth, 0, n0);
    hipLaunchKernelGGL(k_fill_i32, dim3(1), dim3(kGbBlock), 0, st, sync2, 0, 2);
    {
        int dev = 0, ncu = 256;
        if (hipGetDevice(&dev) == hipSuccess)
            (void)hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
        const unsigned nwg = (unsigned)std::max<int64_t>(1, std::min<int64_t>(ncu, (M + kGbBlock - 1) / kGbBlock));
        hipLaunchKernelGGL(k_depth_flow, dim3(nwg), dim3(kGbBlock), 0, st, nbr, n0, M, k, depth,
                           sync2, sync2 + 1);
    }
    int derr = 0;
    GB_HC(hipMemcpyAsync(&derr, sync2 + 1, sizeof(int), hipMemcpyDeviceToHost, st));
    GB_HC(hipStreamSynchronize(st));
    if (derr) return set_error(GGP_ERR_HIP, "graph build: a depth wait ran past its bound");
    hipLaunchKernelGGL(k_iota, dim3(nblocks(N)), dim3(kGbBlock), 0, st, val_a, N, (int64_t)0);
    {
        size_t tb = tmp_bytes;
        GB_HC(hipcub::DeviceRadixSort::SortPairs(tmp, tb, reinterpret_cast<uint32_t*>(depth),
                                                 key32b, val_a, val_b, (int)N, 0, 32, st));
    }
    GB_ALLOC(inv, int32_t, N);
    hipLaunchKernelGGL((k_depth_gather<D>), dim3(nblocks(N)), dim3(kGbBlock), 0, st, N, val_b, pa,
                       perm_a, reinterpret_cast<const uint32_t*>(depth), pb, indices, key32a, inv);
    if (M > 0)
        hipLaunchKernelGGL(k_nbr_remap, dim3(nblocks_capped(M * k)), dim3(kGbBlock), 0, st, nbr, inv, n0,
                           M, k, neighbors);

    // 4. lattice: bounding box, step, rounding; level ends from the sorted depths
    const unsigned nb_box = (unsigned)std::min<int64_t>(1024, nblocks(N));
    GB_ALLOC(part, double, (size_t)nb_box * 2 * D);
    hipLaunchKernelGGL((k_bbox<D>), dim3(nb_box), dim3(kGbBlock), 0, st, pb, N, part);
    std::vector<double> hpart((size_t)nb_box * 2 * D);
    GB_HC(hipMemcpyAsync(hpart.data(), part, hpart.size() * sizeof(double), hipMemcpyDeviceToHost,
                         st));
    uint32_t last_depth = 0;
    GB_HC(hipMemcpyAsync(&last_depth, key32a + (N - 1), sizeof(uint32_t), hipMemcpyDeviceToHost,
                         st));
    GB_HC(hipStreamSynchronize(st));
    const double lmax = (double)((int64_t(1) << lattice_bits) - 1);
    Origin org{};
    double extent = 0.0;
    for (int d = 0; d < D; ++d) {
        double lo = std::numeric_limits<double>::infinity(), hi = -lo;
        for (unsigned b = 0; b < nb_box; ++b) {
            lo = std::min(lo, hpart[(size_t)b * 2 * D + d]);
            hi = std::max(hi, hpart[(size_t)b * 2 * D + D + d]);
        }
        org.o[d] = lo;
        extent = std::max(extent, hi - lo);
    }
    const double scale = extent > 0 ? extent / lmax : 1.0 / lmax;
    hipLaunchKernelGGL((k_quantize<D>), dim3(nblocks_capped(N * D)), dim3(kGbBlock), 0, st, pb, N, org,
                       scale, lmax, coords);
    const int64_t n_off = (int64_t)last_depth + 1;
    if (n_off > offsets_cap)
        return set_error(GGP_ERR_ARG, "graph build: offsets_host holds fewer than the " +
                                          std::to_string(n_off) + " level ends");
    GB_ALLOC(doffs, int64_t, n_off);
    hipLaunchKernelGGL(k_fill_i32, dim3(nblocks(2 * n_off)), dim3(kGbBlock), 0, st,
                       reinterpret_cast<int32_t*>(doffs), -1, 2 * n_off);
    hipLaunchKernelGGL(k_level_ends, dim3(nblocks(N)), dim3(kGbBlock), 0, st, key32a, N, doffs);
    GB_HC(hipMemcpyAsync(offsets_host, doffs, n_off * sizeof(int64_t), hipMemcpyDeviceToHost, st));
    GB_HC(hipStreamSynchronize(st));
    GB_HC(hipGetLastError());
    for (int64_t d = 0; d < n_off; ++d)  // a depth with no points ends where the previous one did
        if (offsets_host[d] < 0) offsets_host[d] = d > 0 ? offsets_host[d - 1] : 0;
    *n_offsets = n_off;
    *scale_out = scale;
    return 0;
}

template <int D>
int build_k(const double* points, int64_t N, int64_t n0, int k, int lattice_bits,
            uint32_t* coords, int64_t* neighbors, int64_t* indices, int64_t* offsets_host,
            int64_t offsets_cap, int64_t* n_offsets, double* scale, hipStream_t st) {
#define GB_K(KM)                                                                               \
    return build<D, KM>(points, N, n0, k, lattice_bits, coords, neighbors, indices,            \
                        offsets_host, offsets_cap, n_offsets, scale, st)
    if (k <= 8) GB_K(8);
    if (k <= 16) GB_K(16);
    GB_K(32);
#undef GB_K
}

}  // namespace

extern "C" int ggp_build_graph_device(const double* points, int64_t N, int32_t D, int64_t n0,
                                      int64_t k, int32_t lattice_bits, uint32_t* coords,
                                      int64_t* neighbors, int64_t* indices,
                                      int64_t* offsets_host, int64_t offsets_cap,
                                      int64_t* n_offsets, double* scale, void* stream) {
    if (!points || !coords || !indices || !offsets_host || !n_offsets || !scale ||
        (N > n0 && !neighbors))
        return set_error(GGP_ERR_ARG, "graph build: null argument");
    if (N < 2 || N >= ((int64_t)1 << 31) || k < 1 || k > 32 || n0 < k || n0 >= N ||
        lattice_bits < 1 || lattice_bits > 30)
        return set_error(GGP_ERR_ARG, "graph build: need 1 <= k <= 32, k <= n0 < N < 2^31 and "
                                      "1 <= lattice_bits <= 30");
    hipStream_t st = static_cast<hipStream_t>(stream);
    switch (D) {
        case 1: return build_k<1>(points, N, n0, (int)k, lattice_bits, coords, neighbors, indices, offsets_host, offsets_cap, n_offsets, scale, st);
        case 2: return build_k<2>(points, N, n0, (int)k, lattice_bits, coords, neighbors, indices, offsets_host, offsets_cap, n_offsets, scale, st);
        case 3: return build_k<3>(points, N, n0, (int)k, lattice_bits, coords, neighbors, indices, offsets_host, offsets_cap, n_offsets, scale, st);
        case 4: return build_k<4>(points, N, n0, (int)k, lattice_bits, coords, neighbors, indices, offsets_host, offsets_cap, n_offsets, scale, st);
        default: return set_error(GGP_ERR_D, "graph build: D must be 1 to 4");
    }
}
