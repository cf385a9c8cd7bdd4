// ggp_internal.h — shared declarations of libgraphgp_hip (not part of the public ABI).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "ggp_point.h"

namespace ggp {

constexpr int kBlock = 256;    // threads per workgroup of the per-point kernels
constexpr int kTile = 32;      // dense-layer tile edge
constexpr int kWideBlock = 256;  // threads per workgroup of the group-per-point kernels (k <= 31)
constexpr int kWidePts = kWideBlock / 32;  // points per workgroup pass there (32 lanes each)
constexpr int kWideXch = 144;    // exchange area per point there, in elements of T
// Static LDS of one workgroup of those kernels: per point its rows' coordinates (32 x 4 words),
// the pivots' reciprocals and a seed vector (2 x 32 T) and the exchange area; plus the block
// reduction.
template <typename T>
constexpr size_t wide_static_lds() {
    return (size_t)kWidePts * (32 * 4 * sizeof(uint32_t) + (64 + kWideXch) * sizeof(T)) + 64;
}
constexpr int kRevSlots = 16;    // reverse sweep: list entries per lane fetched together
constexpr uint32_t kRevNone = 0xffffffffu;

// Records msg as ggp_last_error() of this thread and returns code.
int set_error(int code, const std::string& msg);

// Device-resident graph (the reference's GraphGPProblem arrays after to_backend).
struct Graph {
    int64_t N = 0, n0 = 0, M = 0, K = 0;
    int D = 0;
    double scale = 0;
    uint32_t* coords = nullptr;    // N*D point-major
    int32_t* nbr = nullptr;        // K*M, nbr[j*M + m]
    // The stateless entry points' view of a caller's graph: neighbours in the reference's
    // layout (int64, nbr64[m*K + j]) instead of nbr; only the factor pass reads it.
    const int64_t* nbr64 = nullptr;
    int32_t* idx = nullptr;        // N, original position of each internal position, or null
    // Internal order = tree order with every refined level sorted along a Morton curve.
    int32_t* i2t = nullptr;        // N, tree position of each internal position, or null
    int32_t* i2tm = nullptr;       // M, the same for refined indices (i2t[n0+m] - n0), or null
    // Consumers of each point (the transpose of the neighbour table), m*K + j each, listed by
    // decreasing consumer position. rcnt[q] = number of consumers of q. The lists are stored
    // per reverse-sweep chunk: a point of the chunk uses 2^lg lanes, entry u of its list sits
    // on lane (i << lg) + (u mod 2^lg) at slot u >> lg, and slot t of lane l is
    // rev[base + t*kBlock + l] (unused slots hold kRevNone).
    uint32_t* rcnt = nullptr;      // N
    uint32_t* rev = nullptr;
    std::vector<int64_t> offsets;  // host copy, offsets[0] = n0
    // Work lists of the one-launch sweeps: chunks of one level each, in topological order.
    // fwd: {first refined index m, points, 0, 0}; rev: {first position q, points | lg << 16,
    // base / kBlock, slots}, latest level first, the dense block last.
    int4* fwd_chunks = nullptr;
    int4* rev_chunks = nullptr;
    int n_fwd_chunks = 0, n_rev_chunks = 0;
    int* sweep_ticket = nullptr;   // [forward, reverse], zeroed before each sweep
    int* sweep_err = nullptr;      // bit 2: a wait ran past its bound
    int sweep_wgs = 1024;          // workgroups of a sweep launch
};

// Device-resident covariance table prepared for O(1) segment lookup.
template <typename T>
struct Table {
    TabEnt<T>* tab = nullptr;   // nb-1 entries
    TabParams<T>* params = nullptr;  // device copy of P
    uint16_t* acc = nullptr;    // ucells+1 entries
    TabParams<T> P{};
    // The table (entries + cell index) and the d/dvals histogram do not fit the LDS budget: the
    // per-point kernels then read the table from global memory and accumulate the histogram
    // with f64 atomics into their own global row (every k runs on the group-per-point
    // kernels, which have this form).
    bool global = false;
    std::vector<T> bins, vals;  // host copies
    AnisoArgs<T> aniso{};        // device arrays of the anisotropic table (grid == null: isotropic)
    std::vector<T> aniso_host;   // host copy: [sb, zb, grid]
};

enum FactorMode { F_MV = 1, F_TERMS = 2, F_INV = 4 };
// Seeds of the pullback (low two bits); P_PTS sends Abar to the point positions instead of the
// table histogram (with P_LOGDET or P_INVLOSS).
enum PullMode { P_LOGDET = 0, P_INVLOSS = 1, P_GENVALS = 2, P_PTS = 4 };

// Launchers of the per-point kernels for one (T, K); defined in ggp_point_kernels.h and
// instantiated per (T, K) by ggp_inst.hip.
template <typename T, int K>
struct PointK {
    static void factor(const Graph& g, const Table<T>& tb, int mode, T* mv, T* sd, T* terms,
                       double* partial, const T* values, T* xi_out, unsigned nblk,
                       hipStream_t st);
    static void pullback(const Graph& g, const Table<T>& tb, int mode, const T* v, const T* xi,
                         const T* vb, double* hist_partial, double* scalar_partial,
                         unsigned nblk, hipStream_t st);
    static void sweep_fwd(const Graph& g, T* v, const T* xi, int64_t xi_off, const T* mv,
                          const T* sd, bool two_pass, T* out, const int32_t* oidx,
                          hipStream_t st);
    static void sweep_rev(const Graph& g, T* vb, const T* vbar, T* xg, const T* mv, const T* sd,
                          T* xout, const int32_t* oidx, hipStream_t st);
};
// The same launchers for any k <= 31 (group-per-point kernels, ggp_wide.h).
template <typename T>
struct WideK {
    static void factor(const Graph& g, const Table<T>& tb, int mode, T* mv, T* sd, T* terms,
                       double* partial, const T* values, T* xi_out, unsigned nblk,
                       hipStream_t st);
    static void pullback(const Graph& g, const Table<T>& tb, int mode, const T* v, const T* xi,
                         const T* vb, double* hist_partial, double* scalar_partial,
                         unsigned nblk, hipStream_t st);
    static void sweep_fwd(const Graph& g, T* v, const T* xi, int64_t xi_off, const T* mv,
                          const T* sd, bool two_pass, T* out, const int32_t* oidx,
                          hipStream_t st);
    static void sweep_rev(const Graph& g, T* vb, const T* vbar, T* xg, const T* mv, const T* sd,
                          T* xout, const int32_t* oidx, hipStream_t st);
};
extern template struct WideK<float>;
extern template struct WideK<double>;
// Per-dimension factor/pullback launchers behind WideK (ggp_wide.hip, one object per (T, D)).
template <typename T, int D>
struct WideD {
    static void factor(const Graph& g, const Table<T>& tb, int mode, T* mv, T* sd, T* terms,
                       double* partial, const T* values, T* xi_out, unsigned nblk,
                       hipStream_t st);
    static void pullback(const Graph& g, const Table<T>& tb, int mode, const T* v, const T* xi,
                         const T* vb, double* hist_partial, double* scalar_partial,
                         unsigned nblk, hipStream_t st);
};
// The pullback with the table in global memory (ggp_wide.hip, part 2), behind WideD.
template <typename T, int D>
struct WideG {
    static void pullback(const Graph& g, const Table<T>& tb, int mode, const T* v, const T* xi,
                         const T* vb, double* hist_partial, double* scalar_partial,
                         unsigned nblk, hipStream_t st);
};
extern template struct WideG<float, 2>;
extern template struct WideG<float, 3>;
extern template struct WideG<float, 4>;
extern template struct WideG<double, 2>;
extern template struct WideG<double, 3>;
extern template struct WideG<double, 4>;
extern template struct WideD<float, 2>;
extern template struct WideD<float, 3>;
extern template struct WideD<float, 4>;
extern template struct WideD<double, 2>;
extern template struct WideD<double, 3>;
extern template struct WideD<double, 4>;
constexpr int kMaxK = 31;  // largest neighbour count (group-per-point path)
inline bool register_block_k(int64_t k) { return k == 4 || k == 8 || k == 10 || k == 16; }
// LDS the per-point kernels of neighbour count k need beside the table and the histogram: the
// reductions, and for the group-per-point kernels their per-point areas.
template <typename T>
inline size_t lds_slack(int64_t k) {
    return register_block_k(k) ? 512 + (size_t)4 * 2 * 64 * sizeof(T) : 512 + wide_static_lds<T>();
}

extern template struct PointK<float, 4>;
extern template struct PointK<float, 8>;
extern template struct PointK<float, 10>;
extern template struct PointK<float, 16>;
extern template struct PointK<double, 4>;
extern template struct PointK<double, 8>;
extern template struct PointK<double, 10>;
extern template struct PointK<double, 16>;

// Dispatch over k (ggp_kernels.hip).
template <typename T>
void launch_factor(const Graph& g, const Table<T>& tb, int mode, T* mv, T* sd, T* terms,
                   double* partial, const T* values, T* xi_out, unsigned nblk, hipStream_t st);
template <typename T>
void launch_pullback(const Graph& g, const Table<T>& tb, int mode, const T* v, const T* xi,
                     const T* vb, double* hist_partial, double* scalar_partial, unsigned nblk,
                     hipStream_t st);
// Whole sweeps, one launch each: the forward apply over every level (v[n0:end] is written) and
// the reverse gather (vb and xg of every position in a level or the dense block).
// prepared: launch_sweep_prep already ran for this sweep (else the sweep prepares itself).
// out / xout (optional): every value the sweep produces (v, or xg = std * vb) is also stored at
// out[oidx[position]] (the op's original-order output, so no separate scatter is needed); a null
// oidx is the identity map, as in launch_scatter.
template <typename T>
void launch_sweep_fwd(const Graph& g, T* v, const T* xi, int64_t xi_off, const T* mv,
                      const T* sd, bool two_pass, bool prepared, hipStream_t st,
                      T* out = nullptr, const int32_t* oidx = nullptr);
template <typename T>
void launch_sumsq_half(const T* x, int64_t n, double* out, hipStream_t st);
template <typename T>
void launch_sweep_rev(const Graph& g, T* vb, const T* vbar, T* xg, const T* mv, const T* sd,
                      bool prepared, hipStream_t st, T* xout = nullptr,
                      const int32_t* oidx = nullptr);
// Pending markers for the next forward (v) and/or reverse (vb) sweep, tickets zeroed.
template <typename T>
void launch_sweep_prep(const Graph& g, T* v, T* vb, hipStream_t st);
// p[0:n] = the pending marker of the sweeps (a NaN no arithmetic produces).
template <typename T>
void launch_fill_pending(T* p, int64_t n, hipStream_t st);
template <typename T>
void launch_reduce_hist(T* d_out, const double* partial, int nw, int nb, const double* extra,
                        hipStream_t st);
void launch_reduce_scalar(double* out, const double* in, int n, const double* add,
                          hipStream_t st);
template <typename T>
void launch_gather(T* out, const T* in, const int32_t* idx, int64_t n, hipStream_t st);
template <typename T>
void launch_scatter(T* out, const T* in, const int32_t* idx, int64_t n, hipStream_t st);
template <typename T>
void launch_fill(T* p, T v, int64_t n, hipStream_t st);
template <typename T>
void launch_copy(T* dst, const T* src, int64_t n, hipStream_t st);
// Rows of out (N x D, tree order) = dp (+ dpd on the first n_dense entries), rounded to T
// once; map: internal -> tree position, or null.
template <typename T>
void launch_points_out(T* out, const double* dp, const double* dpd, int64_t N, int D,
                       int64_t n_dense, const int32_t* map, hipStream_t st);

// Self-check of the f32 square roots (sqrt_rn_f32 in its range, sqrt_rn_any_f32 everywhere) over
// bit patterns [b0, b0 + count).
void launch_sqrt_check(uint32_t b0, uint32_t count, unsigned long long* bad, hipStream_t st);
// Self-check of div_rcp against the IEEE division (f32: divisor bit patterns [b0, b0 + count);
// f64: count random divisors), `per` numerators per divisor.
void launch_div_check(int f64, uint64_t b0, uint64_t count, uint32_t per, uint64_t seed,
                      unsigned long long* bad, hipStream_t st);

// Dense first layer (ggp_dense.hip). Matrices are n x n row-major; L lower.
// zero_info / zero_sync (optional): zeroed by the same launch (*zero_info and the flag part of
// a dense_potrf sync workspace), so that dense_potrf(..., zeroed = true) can follow directly.
template <typename T>
void dense_assemble(const Graph& g, const Table<T>& tb, T* A, T diag_add, hipStream_t st,
                    int* zero_info = nullptr, int* zero_sync = nullptr);
// Cholesky in place (lower), one persistent launch of at most max_wg workgroups; sync is a
// workspace of dense_sync_ints(n) ints. *info: bit 0 = non-positive pivot, bit 1 = a wait ran
// past its bound (the result is then invalid).
template <typename T>
void dense_potrf(T* A, int n, int* info, int* sync, int max_wg, hipStream_t st,
                 bool zeroed = false);
int dense_sync_ints(int n);
// y = L x and y = L^T x; out (optional): y[i] also stored at out[oidx[i]] (null oidx: out[i]).
template <typename T>
void dense_trmv(const T* L, int n, const T* x, T* y, hipStream_t st, T* out = nullptr,
                const int32_t* oidx = nullptr);
template <typename T>
void dense_trmv_t(const T* L, int n, const T* x, T* y, hipStream_t st, T* out = nullptr,
                  const int32_t* oidx = nullptr);
// Triangular solves x = L \ b and x = L^T \ b. sync: nt + 1 ints of scratch (nt = ceil(n/32)),
// zeroed by the solve itself; *info bit 1 reports a wait past its bound.
template <typename T>
void dense_trsv(const T* L, int n, const T* b, T* x, int* sync, int* info, hipStream_t st);
template <typename T>
void dense_trsv_t(const T* L, int n, const T* b, T* x, int* sync, int* info, hipStream_t st);
template <typename T>
void dense_logdiag(const T* L, int n, double* out, hipStream_t st);
// Dense cotangent pipelines (f64 internally). Each writes d/dvals of the dense term, accumulated
// per workgroup into hist_partial[nw][nb]; returns nw through *nw_out.
template <typename T>
void dense_grad_logdet(const Graph& g, const Table<T>& tb, const T* L, double* W, double* C,
                       double* hist_partial, int nw, hipStream_t st);
// W = L^-1 (f64, lower); S is n x n scratch.
template <typename T>
void dense_inverse(const T* L, int n, double* W, double* S, hipStream_t st);
// inverse_ready: W already holds L^-1 (dense_inverse ran on this stream or was waited for).
template <typename T>
void dense_grad_generate(const Graph& g, const Table<T>& tb, const T* L, const T* vb,
                         const T* xi, double* W, double* C, double* Q, double* u,
                         double* hist_partial, int nw, bool inverse_ready, hipStream_t st);
template <typename T>
void dense_grad_invloss(const Graph& g, const Table<T>& tb, const T* alpha, double* hist_partial,
                        int nw, hipStream_t st);
template <typename T>
size_t dense_scatter_lds(const Table<T>& tb);
// d/dpoints of the dense term into dpd (n0 x D, f64, overwritten).
template <typename T>
void dense_grad_points_logdet(const Graph& g, const Table<T>& tb, const T* L, double* W,
                              double* C, double* dpd, hipStream_t st);
template <typename T>
void dense_grad_points_invloss(const Graph& g, const Table<T>& tb, const T* alpha, double* dpd,
                               hipStream_t st);

}  // namespace ggp
