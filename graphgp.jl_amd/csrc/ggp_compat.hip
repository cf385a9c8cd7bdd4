// ggp_compat.hip — stateless entry points with the reference's accelerator signatures
// (gpcuda_refine_logdet_f32 / gpcuda_refine_inv_f32, csrc/graphgp_capi.cu:70-94), taking the
// integer lattice (coords + scale) instead of float positions.
//
// They launch the factor pass of the problem-handle path on the caller's arrays as they are:
// point-major uint32 coords in tree order and the reference's int64 point-major neighbour table
// (read directly by the factor kernels, no repack), over all M = N - n0 refined points in one
// launch. The covariance table is prepared on the device (segment entries, O(1) cell index and
// its step bound) by one small kernel into a scratch buffer, exactly as ggp_set_cov_iso prepares
// it on the host, so both paths evaluate the same lookups. The logdet terms are summed in double
// per workgroup and then in a fixed order; out[0] receives that sum rounded to T.
//
// Scratch (bytes from offset 0): [TabParams | TabEnt x (nb-1) | uint16 cell index x (U+1) |
// double partial sums x nblk], each part 256-byte aligned. The entry points allocate it
// stream-ordered (hipMallocAsync / hipFreeAsync) on the caller's stream; nothing else is
// allocated and nothing is synchronized. gphip_refine_logdet_f32_noalloc instead uses a fixed
// 64 KiB device array of this file (tables of at most 2048 bins): every byte a call reads is
// written earlier in the same call, so nothing needs clearing, and calls that overlap on one
// device race on it.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>
#include <string>

#include "../../include/graphgp_hip.h"
#include "ggp_internal.h"

namespace ggp {
namespace {

constexpr int kCompatMaxBlocks = 2048;  // workgroups of the factor launch (partial sums)
constexpr int kCompatMaxCells = 4096;   // cells of the O(1) segment index in LDS
constexpr int kCompatMinLdsCells = 512;  // fewer: the table stays in global memory

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

template <typename T>
struct CompatLayout {
    size_t tab, acc, part, total;
    int ucells_max;
};

// The cell count of the O(1) index as ggp_set_cov_iso chooses it: what the LDS budget leaves
// beside the table (and a histogram), or, when that is too little, a table in global memory
// (*global set) with a finer index there.
template <typename T>
int cells_for(int64_t nb, int64_t k, size_t lds_max, bool* global) {
    const size_t entb = (size_t)(nb - 1) * sizeof(TabEnt<T>);
    const size_t slack = lds_slack<T>(k);
    const size_t hist = (size_t)nb * 8;
    const size_t budget = lds_max > entb + hist + slack ? lds_max - entb - hist - slack : 0;
    const int64_t cells = std::min<int64_t>(kCompatMaxCells, (int64_t)(budget / 2) - 1);
    *global = cells < kCompatMinLdsCells;
    if (*global) return (int)std::min<int64_t>(65536, std::max<int64_t>(4096, 4 * nb));
    return (int)cells;
}

template <typename T>
CompatLayout<T> layout(int64_t nb, int ucells_max, int nblk) {
    CompatLayout<T> L;
    L.ucells_max = ucells_max;
    L.tab = align256(sizeof(TabParams<T>));
    L.acc = align256(L.tab + (size_t)(nb - 1) * sizeof(TabEnt<T>));
    L.part = align256(L.acc + (size_t)(ucells_max + 1) * sizeof(uint16_t));
    L.total = align256(L.part + (size_t)nblk * sizeof(double));
    return L;
}

// 1 + #{i in [2, nb-2] : bins[i] <= v}: for a strictly increasing table, the largest lo >= 1
// with bins[lo] <= v among lo <= nb-2 (the host scan of ggp_set_cov_iso), by binary search.
template <typename T>
__device__ inline int64_t lo_of(const T* __restrict__ bins, int64_t nb, T v) {
    int64_t a = 2, b = nb - 1;  // search [a, b) for the first bins[i] > v
    while (a < b) {
        const int64_t mid = (a + b) >> 1;
        if (bins[mid] <= v) a = mid + 1; else b = mid;
    }
    return 1 + (a - 2 > 0 ? a - 2 : 0);
}

// The table as ggp_set_cov_iso prepares it (segment entries with the reference's inline slope,
// src/interp.jl:30; cell index; step bound), built by one workgroup from device bins / vals.
template <typename T>
__global__ void __launch_bounds__(256) k_table_prep(const T* __restrict__ bins,
                                                    const T* __restrict__ vals, int64_t nb,
                                                    int umax, TabParams<T>* __restrict__ Pout,
                                                    TabEnt<T>* __restrict__ tab,
                                                    uint16_t* __restrict__ acc) {
    using U = typename num<T>::bits_t;
    __shared__ int s_shift, s_ucells;
    __shared__ int s_steps[256];
    const int tid = threadIdx.x;
    const U base = num<T>::bits(bins[1]);
    const U top_all = num<T>::bits(bins[nb - 1]);
    const U range = top_all - base;
    if (tid == 0) {
        int shift = 0;
        while ((int64_t)(range >> shift) + 1 > umax) ++shift;
        s_shift = shift;
        s_ucells = (int)((range >> shift) + 1);
    }
    for (int64_t i = tid; i + 1 < nb; i += blockDim.x) {
        TabEnt<T> e;
        e.x0 = bins[i];
        e.y0 = vals[i];
        e.x1 = bins[i + 1];
        e.slope = (vals[i + 1] - vals[i]) / (bins[i + 1] - bins[i]);
        tab[i] = e;
    }
    __syncthreads();
    const int shift = s_shift, ucells = s_ucells;
    int steps = 0;
    if (tid == 0) acc[0] = 0;
    for (int c = tid; c < ucells; c += blockDim.x) {
        const U lo_bits = base + ((U)c << shift);
        T cm;
        U hi_bits = base + (((U)c + 1) << shift) - 1;
        hi_bits = hi_bits < top_all - 1 ? hi_bits : top_all - 1;
        if constexpr (sizeof(T) == 4) cm = __uint_as_float(lo_bits);
        else cm = __longlong_as_double((long long)lo_bits);
        T vmax;
        if constexpr (sizeof(T) == 4) vmax = __uint_as_float(hi_bits);
        else vmax = __longlong_as_double((long long)hi_bits);
        const int64_t a = min(lo_of(bins, nb, cm), nb - 2);
        const int64_t b = min(lo_of(bins, nb, vmax), nb - 2);
        acc[c + 1] = (uint16_t)a;
        steps = max(steps, (int)(b > a ? b - a : 0));
    }
    s_steps[tid] = steps;
    __syncthreads();
    if (tid == 0) {
        int sm = 0;
        for (int i = 0; i < (int)blockDim.x; ++i) sm = max(sm, s_steps[i]);
        TabParams<T> P{};
        P.steps = sm;
        P.b0 = bins[0];
        P.b1 = bins[1];
        P.bl = bins[nb - 1];
        P.v0 = vals[0];
        P.vl = vals[nb - 1];
        P.base = base;
        P.shift = shift;
        P.ucells = ucells;
        P.nb = (int)nb;
        *Pout = P;
    }
}

// out[0] = T(sum of the n partial sums), in index order.
template <typename T>
__global__ void k_sum_partials(const double* __restrict__ part, int n, T* __restrict__ out) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    double s = 0.0;
    for (int i = 0; i < n; ++i) s += part[i];
    out[0] = (T)s;
}

struct DevInfo {
    int ncu = 0;
    size_t lds = 0;
};

// Compute units and LDS budget of the current device (attribute queries only).
int dev_info(DevInfo& d) {
    int dev = 0, ncu = 0, lds = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
        return set_error(GGP_ERR_HIP, "device attribute query failed");
    d.ncu = std::max(1, ncu);
    d.lds = std::min<size_t>((size_t)lds, 65536);
    return 0;
}

enum CompatOp { C_LOGDET, C_INV };

struct CompatArgs {
    const uint32_t* coords;
    double scale;
    const int64_t* nbr;
    const void* bins;
    const void* vals;
    const void* values;
    void* out;
    int64_t n0, k, N, nb, D;
};

int check(const CompatArgs& a, int op) {
    if (a.D < 2 || a.D > 4) return set_error(GGP_ERR_D, "ndim must be 2, 3 or 4");
    if (a.k < 1 || a.k > kMaxK) return set_error(GGP_ERR_K, "k must be in 1..31");
    if (a.N < 1 || a.n0 < 1 || a.n0 > a.N || a.N > INT32_MAX)
        return set_error(GGP_ERR_ARG, "need 1 <= n0 <= n_points < 2^31");
    if (a.nb < 2 || a.nb > 65535) return set_error(GGP_ERR_ARG, "n_cov must be in 2..65535");
    if (!(a.scale > 0) || !(a.scale < 1e300)) return set_error(GGP_ERR_ARG, "scale must be finite and > 0");
    if (!a.coords || !a.bins || !a.vals || !a.out || (a.N > a.n0 && !a.nbr) ||
        (op == C_INV && !a.values))
        return set_error(GGP_ERR_ARG, "null argument");
    return 0;
}

// Workgroups of the factor launch: the handle path's grid for this k, at most kCompatMaxBlocks.
unsigned factor_blocks(int64_t M, int64_t k, int ncu) {
    const bool reg = register_block_k(k);
    const int64_t ppb = reg ? kBlock : kWidePts;
    const int64_t want = reg ? (int64_t)ncu * 4 : (int64_t)ncu * 8;
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>({want, (M + ppb - 1) / ppb,
                                                              (int64_t)kCompatMaxBlocks}));
}

// Scratch bytes one call needs (0 on a rejected argument, with the error set).
template <typename T>
size_t scratch_bytes(const CompatArgs& a, const DevInfo& d, int* cells_out, unsigned* nblk_out,
                     bool* global) {
    const int cells = cells_for<T>(a.nb, a.k, d.lds, global);
    const unsigned nblk = factor_blocks(a.N - a.n0, a.k, d.ncu);
    *cells_out = cells;
    *nblk_out = nblk;
    return layout<T>(a.nb, cells, (int)nblk).total;
}

// Enqueue the table preparation and the factor pass (and for the logdet the final sum) on
// stream `st`, using `scratch` (at least scratch_bytes bytes).
template <typename T>
int enqueue(const CompatArgs& a, int op, unsigned char* scratch, int cells, unsigned nblk,
            bool global, hipStream_t st) {
    const CompatLayout<T> L = layout<T>(a.nb, cells, (int)nblk);
    Table<T> tb;
    tb.global = global;
    tb.params = reinterpret_cast<TabParams<T>*>(scratch);
    tb.tab = reinterpret_cast<TabEnt<T>*>(scratch + L.tab);
    tb.acc = reinterpret_cast<uint16_t*>(scratch + L.acc);
    tb.P.nb = (int)a.nb;
    tb.P.ucells = cells;  // the staging size the launch reserves; the kernel reads the real P
    double* part = reinterpret_cast<double*>(scratch + L.part);
    hipLaunchKernelGGL((k_table_prep<T>), dim3(1), dim3(256), 0, st, (const T*)a.bins,
                       (const T*)a.vals, a.nb, cells, tb.params, tb.tab, tb.acc);
    const int64_t M = a.N - a.n0;
    if (M > 0) {
        Graph g;
        g.N = a.N;
        g.n0 = a.n0;
        g.M = M;
        g.K = a.k;
        g.D = (int)a.D;
        g.scale = a.scale;
        g.coords = const_cast<uint32_t*>(a.coords);
        g.nbr64 = a.nbr;
        if (op == C_LOGDET)
            launch_factor<T>(g, tb, F_TERMS, nullptr, nullptr, nullptr, part, nullptr, nullptr,
                             nblk, st);
        else
            launch_factor<T>(g, tb, F_INV, nullptr, nullptr, nullptr, nullptr,
                             (const T*)a.values, (T*)a.out, nblk, st);
    }
    if (op == C_LOGDET)
        hipLaunchKernelGGL((k_sum_partials<T>), dim3(1), dim3(64), 0, st, part,
                           M > 0 ? (int)nblk : 0, (T*)a.out);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(GGP_ERR_HIP, std::string("launch: ") + hipGetErrorString(e));
    return 0;
}

// ---- the allocation-free variant --------------------------------------------------------------
// One file-scope device array serves every call on a device (each device holds its own copy
// until the process ends). Host code never passes the array's name: its device address is taken
// once per device with hipGetSymbolAddress and kept here.
constexpr size_t kNoAllocBytes = 64 * 1024;
constexpr int64_t kNoAllocMaxBins = 2048;  // f32 table that, with the index and partial sums, fits
constexpr int kMaxDevices = 64;
__device__ __align__(256) unsigned char scratch[kNoAllocBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_of_device(unsigned char** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return set_error(GGP_ERR_HIP, "hipGetDevice failed");
    if (dev < 0 || dev >= kMaxDevices) return set_error(GGP_ERR_HIP, "device ordinal out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return set_error(GGP_ERR_HIP, std::string("hipGetSymbolAddress(scratch): ") +
                                              hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = static_cast<unsigned char*>(g_scratch_ptr[dev]);
    return 0;
}

template <typename T>
int run_noalloc(const CompatArgs& a, int op, hipStream_t st) {
    if (int rc = check(a, op)) return rc;
    if (a.nb > kNoAllocMaxBins)
        return set_error(GGP_ERR_ARG, "n_cov above 2048: the allocation-free entry point's fixed "
                                      "scratch holds tables of at most 2048 bins");
    DevInfo d;
    if (int rc = dev_info(d)) return rc;
    int cells = 0;
    unsigned nblk = 0;
    bool global = false;
    const size_t bytes = scratch_bytes<T>(a, d, &cells, &nblk, &global);
    if (bytes > kNoAllocBytes)
        return set_error(GGP_ERR_ARG, "problem needs more scratch than the allocation-free entry "
                                      "point's fixed 64 KiB");
    unsigned char* p = nullptr;
    if (int rc = scratch_of_device(&p)) return rc;
    return enqueue<T>(a, op, p, cells, nblk, global, st);
}

template <typename T>
int run_alloc(const CompatArgs& a, int op, hipStream_t st) {
    if (int rc = check(a, op)) return rc;
    DevInfo d;
    if (int rc = dev_info(d)) return rc;
    int cells = 0;
    unsigned nblk = 0;
    bool global = false;
    const size_t bytes = scratch_bytes<T>(a, d, &cells, &nblk, &global);
    void* p = nullptr;
    hipError_t e = hipMallocAsync(&p, bytes, st);
    if (e != hipSuccess) return set_error(GGP_ERR_HIP, std::string("hipMallocAsync: ") + hipGetErrorString(e));
    const int rc = enqueue<T>(a, op, static_cast<unsigned char*>(p), cells, nblk, global, st);
    e = hipFreeAsync(p, st);
    if (rc) return rc;
    if (e != hipSuccess) return set_error(GGP_ERR_HIP, std::string("hipFreeAsync: ") + hipGetErrorString(e));
    return 0;
}

}  // namespace
}  // namespace ggp

using ggp::CompatArgs;

extern "C" {

int gphip_refine_logdet_f32(const uint32_t* coords, float scale, const int64_t* neighbors,
                            const float* cov_bins, const float* cov_vals, float* out, int64_t n0,
                            int64_t k, int64_t n_points, int64_t n_cov, int64_t ndim,
                            void* stream) {
    const CompatArgs a{coords, (double)scale, neighbors, cov_bins, cov_vals, nullptr, out,
                       n0, k, n_points, n_cov, ndim};
    return ggp::run_alloc<float>(a, ggp::C_LOGDET, (hipStream_t)stream);
}

int gphip_refine_logdet_f32_noalloc(const uint32_t* coords, float scale,
                                    const int64_t* neighbors, const float* cov_bins,
                                    const float* cov_vals, float* out, int64_t n0, int64_t k,
                                    int64_t n_points, int64_t n_cov, int64_t ndim, void* stream) {
    const CompatArgs a{coords, (double)scale, neighbors, cov_bins, cov_vals, nullptr, out,
                       n0, k, n_points, n_cov, ndim};
    return ggp::run_noalloc<float>(a, ggp::C_LOGDET, (hipStream_t)stream);
}

int gphip_refine_inv_f32(const uint32_t* coords, float scale, const int64_t* neighbors,
                         const float* cov_bins, const float* cov_vals, const float* values,
                         float* xi, int64_t n0, int64_t k, int64_t n_points, int64_t n_cov,
                         int64_t ndim, void* stream) {
    const CompatArgs a{coords, (double)scale, neighbors, cov_bins, cov_vals, values, xi,
                       n0, k, n_points, n_cov, ndim};
    return ggp::run_alloc<float>(a, ggp::C_INV, (hipStream_t)stream);
}

int gphip_refine_logdet_f64(const uint32_t* coords, double scale, const int64_t* neighbors,
                            const double* cov_bins, const double* cov_vals, double* out,
                            int64_t n0, int64_t k, int64_t n_points, int64_t n_cov,
                            int64_t ndim, void* stream) {
    const CompatArgs a{coords, scale, neighbors, cov_bins, cov_vals, nullptr, out,
                       n0, k, n_points, n_cov, ndim};
    return ggp::run_alloc<double>(a, ggp::C_LOGDET, (hipStream_t)stream);
}

int gphip_refine_inv_f64(const uint32_t* coords, double scale, const int64_t* neighbors,
                         const double* cov_bins, const double* cov_vals, const double* values,
                         double* xi, int64_t n0, int64_t k, int64_t n_points, int64_t n_cov,
                         int64_t ndim, void* stream) {
    const CompatArgs a{coords, scale, neighbors, cov_bins, cov_vals, values, xi,
                       n0, k, n_points, n_cov, ndim};
    return ggp::run_alloc<double>(a, ggp::C_INV, (hipStream_t)stream);
}

}  // extern "C"
