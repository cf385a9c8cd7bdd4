// ggp_api.cpp — the C ABI of libgraphgp_hip (declared in include/graphgp_hip.h).
//
// Each op runs as: a fully parallel factor pass over all refined points (mean_vec, std — the
// value-independent part of every per-point kernel of the reference) on the main stream, the
// dense first layer on a side stream at the same time, then the sequential depth-level sweeps
// and the parallel adjoint passes. Ops return after the work is done; a failed dense
// factorization is detected there and retried with escalating jitter, as src/dense.jl:46-67.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/graphgp_hip.h"
#include "ggp_internal.h"
#include "ggp_pack.h"

using namespace ggp;

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

#define HC(x)                                                                                  \
    do {                                                                                       \
        hipError_t e_ = (x);                                                                   \
        if (e_ != hipSuccess)                                                                  \
            return fail(GGP_ERR_HIP, std::string(#x) + ": " + hipGetErrorString(e_));         \
    } while (0)

bool supported_k(int64_t k) { return k >= 1 && k <= kMaxK; }
bool supported_d(int64_t d) { return d >= 2 && d <= 4; }

}  // namespace

int ggp::set_error(int code, const std::string& msg) { return fail(code, msg); }

struct ggp_graph {
    int dtype = GGP_F32;
    int dev = 0;
    int ncu = 256;
    size_t lds_max = 65536;
    Graph g;
    Table<float> tf;
    Table<double> td;
    bool has_cov = false;
    unsigned nblk_factor = 1024, nblk_pull = 512;
    int nw_dense = 256;
    hipStream_t s_main = nullptr, s_side = nullptr;
    hipStream_t s_rev = nullptr;  // generate_grad_vals: the reverse sweep beside the forward chain
    hipEvent_t ev_fork = nullptr, ev_join = nullptr, ev_user = nullptr;
    hipEvent_t ev_fac = nullptr, ev_rev = nullptr;
    // workspaces (element type T = dtype)
    void *mv = nullptr, *sd = nullptr, *v = nullptr, *xt = nullptr, *vb = nullptr,
         *vbt = nullptr, *xg = nullptr, *A = nullptr, *tmp = nullptr;
    double* scal_partial = nullptr;  // nblk_factor (>= nblk_pull) doubles
    // Status block, one device allocation mirrored by one pinned host block so that an op
    // fetches all of it with one copy: [0, 64) scalars, [64, 80) info, [80, 96) sweep errors.
    void* dstat = nullptr;
    void* hstat = nullptr;
    double* dscal = nullptr;         // 8 doubles (dstat + 0)
    double* hscal = nullptr;         // host mirror of dscal
    int* info = nullptr;             // dstat + 64
    int* hinfo = nullptr;            // host mirror of info
    int* herr = nullptr;             // host mirror of the sweep error flags (dstat + 80)
    int* dsync = nullptr;            // dense Cholesky task counter and tile flags
    double* hist = nullptr;          // (pull_blocks + nw_dense) x nb
    int hist_nb = 0;
    unsigned hist_rows = 0;
    double *W = nullptr, *C = nullptr, *Q = nullptr, *u = nullptr;  // dense f64 scratch (lazy)
    double *dp = nullptr, *dpd = nullptr;  // d/dpoints accumulators, N x D and n0 x D (lazy)
    std::vector<void*> owned;
    // optional HIP-event timers around the main kernels (ggp_kernel_timers)
    int timing = 0;  // bit t: timer kTimerNames[t] is on
    hipEvent_t tev[2 * 8] = {};
    bool tpending[8] = {};
    double tms[8] = {};
    int64_t tcnt[8] = {};
};

namespace {

constexpr int64_t kMinLdsCells = 512;     // fewer cells of LDS index than this: table in global
constexpr unsigned kGlobalPullBlocks = 256;

template <typename T> Table<T>& table(ggp_graph* h);
template <> Table<float>& table<float>(ggp_graph* h) { return h->tf; }
template <> Table<double>& table<double>(ggp_graph* h) { return h->td; }

bool table_global(const ggp_graph* h) { return h->dtype == GGP_F32 ? h->tf.global : h->td.global; }

// Workgroups (and histogram rows) of the adjoint pass. With the table in global memory each row
// is zeroed and accumulated by atomics and every row is reduced, so fewer rows are used.
unsigned pull_blocks(const ggp_graph* h, bool global) {
    return global ? std::min<unsigned>(h->nblk_pull, kGlobalPullBlocks) : h->nblk_pull;
}
unsigned pull_blocks(const ggp_graph* h) { return pull_blocks(h, table_global(h)); }

constexpr size_t kStatBytes = 96;

int dmalloc(ggp_graph* h, void** p, size_t bytes) {
    if (bytes == 0) bytes = 16;
    hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess) {
        *p = nullptr;
        return fail(GGP_ERR_HIP, std::string("hipMalloc: ") + hipGetErrorString(e));
    }
    h->owned.push_back(*p);
    return 0;
}

// Release a buffer of the handle (set_cov replacing a table; every op has finished by then:
// ops return after their work is done).
void dfree(ggp_graph* h, void* p) {
    if (!p) return;
    auto it = std::find(h->owned.begin(), h->owned.end(), p);
    if (it != h->owned.end()) {
        h->owned.erase(it);
        (void)hipFree(p);
    }
}

void free_all(ggp_graph* h) {
    for (void* p : h->owned) (void)hipFree(p);
    h->owned.clear();
    if (h->hstat) (void)hipHostFree(h->hstat);
    if (h->s_main) (void)hipStreamDestroy(h->s_main);
    if (h->s_side) (void)hipStreamDestroy(h->s_side);
    if (h->s_rev) (void)hipStreamDestroy(h->s_rev);
    if (h->ev_fac) (void)hipEventDestroy(h->ev_fac);
    if (h->ev_rev) (void)hipEventDestroy(h->ev_rev);
    if (h->ev_fork) (void)hipEventDestroy(h->ev_fork);
    if (h->ev_join) (void)hipEventDestroy(h->ev_join);
    if (h->ev_user) (void)hipEventDestroy(h->ev_user);
    for (int i = 0; i < 16; ++i)
        if (h->tev[i]) (void)hipEventDestroy(h->tev[i]);
}

// ---- covariance table ----------------------------------------------------------------------
template <typename T> struct Bits;
template <> struct Bits<float> {
    using U = uint32_t;
    static U of(float x) { U u; std::memcpy(&u, &x, 4); return u; }
    static float from(U u) { float x; std::memcpy(&x, &u, 4); return x; }
};
template <> struct Bits<double> {
    using U = uint64_t;
    static U of(double x) { U u; std::memcpy(&u, &x, 8); return u; }
    static double from(U u) { double x; std::memcpy(&x, &u, 8); return x; }
};

// O(1) segment index of a strictly increasing axis (nb >= 2) over the bit patterns of
// [bins[1], bins[nb-1]] in at most umax cells: acc[c+1] is the largest lo <= nb-2 with bins[lo]
// <= the smallest value of cell c (acc[0] = 0); steps is the most forward steps the search takes
// from acc[cell] for any r < bins[nb-1] (the kernels use one unconditional step when <= 1).
template <typename T>
struct CellIndex {
    std::vector<uint16_t> acc;
    typename Bits<T>::U base = 0;
    int shift = 0, ucells = 0, steps = 0;
};
template <typename T>
CellIndex<T> cell_index(const T* bins, int64_t nb, int64_t umax) {
    using U = typename Bits<T>::U;
    CellIndex<T> ci;
    ci.base = Bits<T>::of(bins[1]);
    const U range = Bits<T>::of(bins[nb - 1]) - ci.base;
    while ((int64_t)(range >> ci.shift) + 1 > umax) ++ci.shift;
    ci.ucells = (int)((range >> ci.shift) + 1);
    ci.acc.assign((size_t)ci.ucells + 1, 0);
    int64_t lo = 1;
    for (int c = 0; c < ci.ucells; ++c) {
        const T cm = Bits<T>::from(ci.base + ((U)c << ci.shift));
        while (lo + 1 <= nb - 2 && bins[lo + 1] <= cm) ++lo;
        ci.acc[(size_t)c + 1] = (uint16_t)std::min<int64_t>(lo, nb - 2);
    }
    const U top_all = Bits<T>::of(bins[nb - 1]) - 1;
    for (int c = 0; c < ci.ucells; ++c) {
        const U top = std::min<U>(ci.base + (((U)c + 1) << ci.shift) - 1, top_all);
        const T vmax = Bits<T>::from(top);
        int64_t hi = ci.acc[(size_t)c + 1];
        const int64_t lo0 = hi;
        while (hi + 1 <= nb - 2 && bins[hi + 1] <= vmax) ++hi;
        ci.steps = std::max<int>(ci.steps, (int)(hi - lo0));
    }
    return ci;
}

template <typename T>
int set_cov(ggp_graph* h, const T* bins, const T* vals, int64_t nb) {
    if (nb < 2) return fail(GGP_ERR_ARG, "nbins must be >= 2");
    if (nb > 65535) return fail(GGP_ERR_ARG, "nbins must be < 65536");
    for (int64_t i = 0; i < nb; ++i) {
        if (!std::isfinite(bins[i]) || !std::isfinite(vals[i]))
            return fail(GGP_ERR_ARG, "bins and vals must be finite");
        if (i > 0 && !(bins[i] > bins[i - 1]))
            return fail(GGP_ERR_ARG, "bins must be strictly increasing");
    }
    if (!(bins[0] >= T(0))) return fail(GGP_ERR_ARG, "bins[0] must be >= 0");
    Table<T>& tb = table<T>(h);
    // Segment entries; slope evaluated exactly as src/interp.jl:30 does inline.
    std::vector<TabEnt<T>> ent((size_t)nb - 1);
    for (int64_t i = 0; i + 1 < nb; ++i) {
        ent[i].x0 = bins[i];
        ent[i].y0 = vals[i];
        ent[i].x1 = bins[i + 1];
        volatile T dy = vals[i + 1] - vals[i];
        volatile T dx = bins[i + 1] - bins[i];
        ent[i].slope = dy / dx;
    }
    // Cell index over bit patterns from bins[1] to bins[nb-1].
    const size_t entb = (size_t)(nb - 1) * sizeof(TabEnt<T>);
    const size_t slack = lds_slack<T>(h->g.K);
    size_t budget = h->lds_max > entb + (size_t)nb * 8 + slack ? h->lds_max - entb - (size_t)nb * 8 - slack : 0;
    int64_t umax = std::min<int64_t>(4096, (int64_t)(budget / 2) - 1);
    // Too little LDS left for a useful cell index: the table stays in global memory (the
    // reference's lookups read it there for any nbins, src/interp.jl:10-34; its gradients fall
    // back to global atomics beyond its shared-memory histogram, src/grad.jl:107-116), with a
    // finer index there.
    const bool global = umax < kMinLdsCells;
    if (global) umax = std::min<int64_t>(65536, std::max<int64_t>(4096, 4 * nb));
    const CellIndex<T> ci = cell_index(bins, nb, umax);
    const std::vector<uint16_t>& acc = ci.acc;
    const int ucells = ci.ucells;
    TabParams<T> P{};
    P.steps = ci.steps;
    P.b0 = bins[0];
    P.b1 = bins[1];
    P.bl = bins[nb - 1];
    P.v0 = vals[0];
    P.vl = vals[nb - 1];
    P.base = ci.base;
    P.shift = ci.shift;
    P.ucells = ucells;
    P.nb = (int)nb;
    const bool realloc_tab = !tb.tab || tb.P.nb != (int)nb || tb.P.ucells != ucells;
    if (realloc_tab) {  // the previous table's buffers are released (ops have finished)
        dfree(h, tb.tab);
        dfree(h, tb.acc);
        tb.tab = nullptr;
        tb.acc = nullptr;
        if (dmalloc(h, (void**)&tb.tab, entb)) return GGP_ERR_HIP;
        if (dmalloc(h, (void**)&tb.acc, acc.size() * sizeof(uint16_t))) return GGP_ERR_HIP;
        if (!tb.params && dmalloc(h, (void**)&tb.params, sizeof(TabParams<T>))) return GGP_ERR_HIP;
    }
    HC(hipMemcpy(tb.tab, ent.data(), entb, hipMemcpyHostToDevice));
    HC(hipMemcpy(tb.acc, acc.data(), acc.size() * sizeof(uint16_t), hipMemcpyHostToDevice));
    HC(hipMemcpy(tb.params, &P, sizeof(P), hipMemcpyHostToDevice));
    tb.P = P;
    tb.global = global;
    tb.bins.assign(bins, bins + nb);
    tb.vals.assign(vals, vals + nb);
    dfree(h, const_cast<T*>(tb.aniso.sb));  // an anisotropic table set before
    tb.aniso = AnisoArgs<T>{};
    tb.aniso_host.clear();
    const unsigned rows = pull_blocks(h, global) + (unsigned)h->nw_dense;
    if (h->hist_nb != (int)nb || h->hist_rows != rows) {
        dfree(h, h->hist);
        h->hist = nullptr;
        if (dmalloc(h, (void**)&h->hist, (size_t)rows * (size_t)nb * sizeof(double)))
            return GGP_ERR_HIP;
        h->hist_nb = (int)nb;
        h->hist_rows = rows;
    }
    h->has_cov = true;
    return 0;
}

// ---- kernel timers ---------------------------------------------------------------------------
enum Timer { TM_FACTOR = 0, TM_PULLBACK = 1, TM_SWEEP_FWD = 2, TM_SWEEP_REV = 3, TM_DENSE = 4,
             TM_OP = 5, TM_POTRF = 6, TM_COUNT = 7 };
const char* const kTimerNames[TM_COUNT] = {"factor", "pullback", "sweep_fwd", "sweep_rev",
                                           "dense", "op", "potrf"};

inline void tstart(ggp_graph* h, int t, hipStream_t st) {
    if (h->timing >> t & 1) (void)hipEventRecord(h->tev[2 * t], st);
}
inline void tstop(ggp_graph* h, int t, hipStream_t st) {
    if (h->timing >> t & 1) {
        (void)hipEventRecord(h->tev[2 * t + 1], st);
        h->tpending[t] = true;
    }
}
void tcollect(ggp_graph* h) {
    if (!h->timing) return;
    for (int t = 0; t < TM_COUNT; ++t)
        if (h->tpending[t]) {
            float ms = 0.f;
            if (hipEventElapsedTime(&ms, h->tev[2 * t], h->tev[2 * t + 1]) == hipSuccess) {
                h->tms[t] += ms;
                h->tcnt[t] += 1;
            }
            h->tpending[t] = false;
        }
}

// Anisotropic table (src/aniso.jl:22-37, src/types.jl:15-20). The grid is used as given
// (build_anisotropic_covariance's jitter already applied by the caller).
template <typename T>
int set_cov_aniso(ggp_graph* h, const T* sb, int64_t ns, const T* zb, int64_t nz, const T* grid,
                  double alpha) {
    if (ns < 1 || nz < 1 || ns > 65536 || nz > 65536) return fail(GGP_ERR_ARG, "bad aniso grid size");
    if (!(std::isfinite(alpha) && alpha > 0)) return fail(GGP_ERR_ARG, "alpha must be finite and > 0");
    for (int64_t i = 1; i < ns; ++i)
        if (!(sb[i] > sb[i - 1])) return fail(GGP_ERR_ARG, "spatial_bins must be strictly increasing");
    for (int64_t i = 1; i < nz; ++i)
        if (!(zb[i] > zb[i - 1])) return fail(GGP_ERR_ARG, "z_bins must be strictly increasing");
    if (h->g.D < 2) return fail(GGP_ERR_D, "anisotropic covariance needs D >= 2");
    if (!(sb[0] >= T(0)) || !(zb[0] >= T(0))) return fail(GGP_ERR_ARG, "aniso axes must start at >= 0");
    Table<T>& tb = table<T>(h);
    std::vector<T> host;
    host.insert(host.end(), sb, sb + ns);
    host.insert(host.end(), zb, zb + nz);
    host.insert(host.end(), grid, grid + ns * nz);
    for (const T& x : host)
        if (!std::isfinite(x)) return fail(GGP_ERR_ARG, "aniso table must be finite");
    // O(1) cell indices of the two axes (the reference's _frac_index binary search,
    // src/aniso.jl:43-57, finds the same segment); an axis of one entry never needs one
    const CellIndex<T> si = ns >= 2 ? cell_index(sb, ns, std::max<int64_t>(64, 4 * ns)) : CellIndex<T>{};
    const CellIndex<T> zi = nz >= 2 ? cell_index(zb, nz, std::max<int64_t>(64, 4 * nz)) : CellIndex<T>{};
    std::vector<uint16_t> idx(si.acc);
    if (idx.empty()) idx.push_back(0);
    const size_t zoff = idx.size();
    idx.insert(idx.end(), zi.acc.begin(), zi.acc.end());
    if (idx.size() == zoff) idx.push_back(0);
    const size_t tbytes = host.size() * sizeof(T);
    T* dev = nullptr;
    dfree(h, const_cast<T*>(tb.aniso.sb));  // the previous anisotropic table
    tb.aniso = AnisoArgs<T>{};
    if (dmalloc(h, (void**)&dev, tbytes + idx.size() * sizeof(uint16_t))) return GGP_ERR_HIP;
    HC(hipMemcpy(dev, host.data(), tbytes, hipMemcpyHostToDevice));
    uint16_t* didx = reinterpret_cast<uint16_t*>(reinterpret_cast<char*>(dev) + tbytes);
    HC(hipMemcpy(didx, idx.data(), idx.size() * sizeof(uint16_t), hipMemcpyHostToDevice));
    tb.aniso.sb = dev;
    tb.aniso.zb = dev + ns;
    tb.aniso.grid = dev + ns + nz;
    tb.aniso.sacc = didx;
    tb.aniso.zacc = didx + zoff;
    tb.aniso.si.base = si.base;
    tb.aniso.si.shift = si.shift;
    tb.aniso.si.ucells = si.ucells;
    tb.aniso.zi.base = zi.base;
    tb.aniso.zi.shift = zi.shift;
    tb.aniso.zi.ucells = zi.ucells;
    tb.aniso.ns = (int)ns;
    tb.aniso.nz = (int)nz;
    tb.aniso.alpha = (T)alpha;
    // staged in LDS by the assembling kernels when the axes and indices fit the budget
    const size_t sbytes = aniso_stage_bytes<T>((int)ns, (int)nz, si.ucells, zi.ucells);
    tb.aniso.lds = sbytes + lds_slack<T>(h->g.K) <= h->lds_max ? (int)sbytes : 0;
    tb.aniso_host = host;
    tb.global = false;
    // the isotropic table is not used by an anisotropic problem
    tb.vals.assign(1, grid[0]);
    h->has_cov = true;
    return 0;
}

bool is_aniso(ggp_graph* h) {
    return h->dtype == GGP_F32 ? h->tf.aniso.grid != nullptr : h->td.aniso.grid != nullptr;
}

// ---- stream plumbing -------------------------------------------------------------------------
int enter(ggp_graph* h, hipStream_t user) {
    HC(hipSetDevice(h->dev));
    HC(hipEventRecord(h->ev_user, user));
    HC(hipStreamWaitEvent(h->s_main, h->ev_user, 0));
    tstart(h, TM_OP, h->s_main);
    return 0;
}
int fork(ggp_graph* h) {
    HC(hipEventRecord(h->ev_fork, h->s_main));
    HC(hipStreamWaitEvent(h->s_side, h->ev_fork, 0));
    return 0;
}
int join(ggp_graph* h) {
    HC(hipEventRecord(h->ev_join, h->s_side));
    HC(hipStreamWaitEvent(h->s_main, h->ev_join, 0));
    return 0;
}
// Drain the main stream, release the user stream, and fetch info + scalars.
int finish(ggp_graph* h, hipStream_t user) {
    HC(hipMemcpyAsync(h->hstat, h->dstat, kStatBytes, hipMemcpyDeviceToHost, h->s_main));
    HC(hipGetLastError());
    tstop(h, TM_OP, h->s_main);
    HC(hipEventRecord(h->ev_user, h->s_main));
    HC(hipStreamWaitEvent(user, h->ev_user, 0));
    // Poll the op's last event rather than block in hipStreamSynchronize: a blocking wait
    // returns to the host tens of microseconds after the stream drains, a poll within one or two.
    for (;;) {
        const hipError_t q = hipEventQuery(h->ev_user);
        if (q == hipSuccess) break;
        if (q != hipErrorNotReady) return fail(GGP_ERR_HIP, std::string("op: ") + hipGetErrorString(q));
    }
    tcollect(h);
    if (h->herr[0] & 4) {
        h->herr[0] = 0;
        (void)hipMemset(h->g.sweep_err, 0, sizeof(int));
        return fail(GGP_ERR_HIP, "level sweep: a wait for an input value timed out");
    }
    return 0;
}

template <typename T> T* tp(void* p) { return static_cast<T*>(p); }

// K(0, 0) of the anisotropic table on the host, evaluated as aniso_lookup does (src/aniso.jl:66-84):
// both fractional indices are 0, so the result is grid[0][0] combined with zero weights.
template <typename T>
T dense_aniso_diag(const Table<T>& tb) {
    const int nz = tb.aniso.nz, ns = tb.aniso.ns;
    const T* g = tb.aniso_host.data() + ns + nz;
    const int i1 = ns > 1 ? 1 : 0, j1 = nz > 1 ? 1 : 0;
    volatile T one = T(1), zero = T(0);
    return (g[0] * (one - zero) + g[i1 * nz] * zero) * (one - zero) + (g[j1] * (one - zero) + g[i1 * nz + j1] * zero) * zero;
}

// Workgroups of the dense factor's persistent launch: the walker plus helpers. The helpers take
// tasks in dependency order and wait in place for their inputs, so their number sets how far
// ahead of the walker the partial sums get started; half the CUs keeps every step's inputs
// ready at n0 = 1000 (a quarter left the walker waiting on late partial sums).
int dense_wgs(const ggp_graph* h) {
    static const int env = std::getenv("GGP_DENSE_WGS") ? std::atoi(std::getenv("GGP_DENSE_WGS")) : 0;
    return std::max(1, env > 0 ? env : h->ncu / 2);
}

// Dense factor with jitter escalation (src/dense.jl:46-67), synchronous; used after the first
// in-op attempt reported a non-positive pivot.
template <typename T>
int dense_retry(ggp_graph* h) {
    if (*h->hinfo & 2) return fail(GGP_ERR_HIP, "dense factorization: a tile wait timed out");
    const Table<T>& tb = table<T>(h);
    const int n = (int)h->g.n0;
    T dmean = T(0);
    const T d0 = tb.aniso.grid ? dense_aniso_diag(tb) : tb.vals[0];
    for (int i = 0; i < n; ++i) dmean += d0;  // every diagonal entry is K(0)
    dmean = dmean / T(n > 1 ? n : 1);
    T e = T(1e-9);
    while (e <= T(1e-2)) {
        launch_fill<int>(h->info, 0, 1, h->s_main);
        dense_assemble<T>(h->g, tb, tp<T>(h->A), e * dmean, h->s_main);
        dense_potrf<T>(tp<T>(h->A), n, h->info, h->dsync, dense_wgs(h), h->s_main);
        HC(hipMemcpyAsync(h->hinfo, h->info, sizeof(int), hipMemcpyDeviceToHost, h->s_main));
        HC(hipStreamSynchronize(h->s_main));
        if (*h->hinfo == 0) return 0;
        if (*h->hinfo & 2) return fail(GGP_ERR_HIP, "dense factorization: a tile wait timed out");
        e *= T(10);
    }
    return fail(GGP_ERR_NOT_PD,
                "dense first-layer covariance is not positive definite even with 1e-2 relative "
                "jitter; increase the kernel jitter or reduce n0");
}

template <typename T>
void dense_factor_async(ggp_graph* h, hipStream_t st) {
    tstart(h, TM_DENSE, st);
    dense_assemble<T>(h->g, table<T>(h), tp<T>(h->A), T(0), st, h->info, h->dsync);
    tstart(h, TM_POTRF, st);
    dense_potrf<T>(tp<T>(h->A), (int)h->g.n0, h->info, h->dsync, dense_wgs(h), st, true);
    tstop(h, TM_POTRF, st);
    tstop(h, TM_DENSE, st);
}

// Factor / pullback launches bracketed by the timers.
template <typename T>
void factor_t(ggp_graph* h, int mode, T* mv, T* sd, T* terms, double* partial, const T* values,
              T* xi_out) {
    tstart(h, TM_FACTOR, h->s_main);
    launch_factor<T>(h->g, table<T>(h), mode, mv, sd, terms, partial, values, xi_out,
                     h->nblk_factor, h->s_main);
    tstop(h, TM_FACTOR, h->s_main);
}
template <typename T>
void pullback_t(ggp_graph* h, int mode, const T* v, const T* xi, const T* vb) {
    tstart(h, TM_PULLBACK, h->s_main);
    launch_pullback<T>(h->g, table<T>(h), mode, v, xi, vb, h->hist, h->scal_partial, pull_blocks(h),
                       h->s_main);
    tstop(h, TM_PULLBACK, h->s_main);
}

int ensure_dense64(ggp_graph* h) {
    if (h->W) return 0;
    const size_t nn = (size_t)h->g.n0 * (size_t)h->g.n0 * sizeof(double);
    if (dmalloc(h, (void**)&h->W, nn) || dmalloc(h, (void**)&h->C, nn) ||
        dmalloc(h, (void**)&h->Q, nn) || dmalloc(h, (void**)&h->u, (size_t)h->g.n0 * 8))
        return GGP_ERR_HIP;
    return 0;
}

int check_ready(ggp_graph* h) {
    if (!h) return fail(GGP_ERR_ARG, "null handle");
    if (!h->has_cov) return fail(GGP_ERR_NO_COV, "no covariance table: call ggp_set_cov_iso first");
    return 0;
}

// Forward sweep over all depth levels (src/api.jl:126-137), one launch; xi indexed as
// xi[xi_off + m].
template <typename T>
void sweep_forward(ggp_graph* h, T* v, const T* xi, int64_t xi_off, hipStream_t st,
                   bool prepared = false, T* out = nullptr, const int32_t* oidx = nullptr) {
    const Graph& g = h->g;
    tstart(h, TM_SWEEP_FWD, st);
    launch_sweep_fwd<T>(g, v, xi, xi_off, tp<T>(h->mv), tp<T>(h->sd),
                        table<T>(h).aniso.grid != nullptr, prepared, st, out, oidx);
    tstop(h, TM_SWEEP_FWD, st);
}

// Reverse sweep, latest level first, then the dense level (src/grad.jl:433-445, 483-489), one
// launch.
template <typename T>
void sweep_reverse(ggp_graph* h, T* vb, const T* vbar, T* xg, hipStream_t st,
                   bool prepared = false, T* xout = nullptr, const int32_t* oidx = nullptr) {
    const Graph& g = h->g;
    tstart(h, TM_SWEEP_REV, st);
    launch_sweep_rev<T>(g, vb, vbar, xg, tp<T>(h->mv), tp<T>(h->sd), prepared, st, xout, oidx);
    tstop(h, TM_SWEEP_REV, st);
}

// out[idx[i]] = x[i] for the positions past the last level (the products and sweeps store the
// rest of an op's original-order output themselves).
template <typename T>
void scatter_tail(ggp_graph* h, T* out, const T* x, hipStream_t st) {
    const Graph& g = h->g;
    const int64_t end = g.offsets.back();
    if (end >= g.N) return;
    if (g.idx) launch_scatter<T>(out, x + end, g.idx + end, g.N - end, st);
    else launch_scatter<T>(out + end, x + end, (const int32_t*)nullptr, g.N - end, st);  // identity
}

// Points past the last level are never refined by the reference (values stay zero).
template <typename T>
void zero_tail(ggp_graph* h, T* x, hipStream_t st) {
    const int64_t end = h->g.offsets.back();
    if (end < h->g.N) launch_fill<T>(x + end, T(0), h->g.N - end, st);
}

// ================================== ops ========================================================
template <typename T>
int op_generate(ggp_graph* h, const T* xi, T* out, hipStream_t user) {
    if (int rc = check_ready(h)) return rc;
    if (int rc = enter(h, user)) return rc;
    Graph& g = h->g;
    T *xt = tp<T>(h->xt), *v = tp<T>(h->v);
    // the dense factor is the longest chain: start it first; everything else on the main
    // stream overlaps it
    if (int rc = fork(h)) return rc;
    dense_factor_async<T>(h, h->s_side);
    launch_gather<T>(xt, xi, g.idx, g.N, h->s_main);
    launch_sweep_prep<T>(g, v, nullptr, h->s_main);
    zero_tail<T>(h, v, h->s_main);
    factor_t<T>(h, F_MV, tp<T>(h->mv), tp<T>(h->sd), nullptr, nullptr, nullptr, nullptr);
    if (int rc = join(h)) return rc;
    // L xi and the sweep also store their values at out[idx[i]] (original order)
    dense_trmv<T>(tp<T>(h->A), (int)g.n0, xt, v, h->s_main, out, g.idx);
    sweep_forward<T>(h, v, xt, g.n0, h->s_main, true, out, g.idx);
    scatter_tail<T>(h, out, v, h->s_main);
    if (int rc = finish(h, user)) return rc;
    if (*h->hinfo != 0) {
        if (int rc = dense_retry<T>(h)) return rc;
        dense_trmv<T>(tp<T>(h->A), (int)g.n0, xt, v, h->s_main);
        sweep_forward<T>(h, v, xt, g.n0, h->s_main);
        launch_scatter<T>(out, v, g.idx, g.N, h->s_main);
        HC(hipStreamSynchronize(h->s_main));
    }
    return 0;
}

template <typename T>
int op_generate_inv(ggp_graph* h, const T* values, T* xi_out, hipStream_t user) {
    if (int rc = check_ready(h)) return rc;
    if (int rc = enter(h, user)) return rc;
    Graph& g = h->g;
    T *vt = tp<T>(h->v), *xt = tp<T>(h->xt);
    if (int rc = fork(h)) return rc;
    dense_factor_async<T>(h, h->s_side);
    launch_gather<T>(vt, values, g.idx, g.N, h->s_main);
    factor_t<T>(h, F_INV, nullptr, nullptr, nullptr, nullptr, vt, xt + g.n0);
    if (int rc = join(h)) return rc;
    dense_trsv<T>(tp<T>(h->A), (int)g.n0, vt, xt, h->dsync, h->info, h->s_main);
    launch_scatter<T>(xi_out, xt, g.idx, g.N, h->s_main);
    if (int rc = finish(h, user)) return rc;
    if (*h->hinfo != 0) {
        if (int rc = dense_retry<T>(h)) return rc;
        dense_trsv<T>(tp<T>(h->A), (int)g.n0, vt, xt, h->dsync, h->info, h->s_main);
        launch_scatter<T>(xi_out, xt, g.idx, g.N, h->s_main);
        HC(hipStreamSynchronize(h->s_main));
    }
    return 0;
}

template <typename T>
int op_logdet(ggp_graph* h, bool dense, double* out, hipStream_t user) {
    if (int rc = check_ready(h)) return rc;
    if (int rc = enter(h, user)) return rc;
    Graph& g = h->g;
    launch_fill<double>(h->dscal, 0.0, 8, h->s_main);
    launch_fill<int>(h->info, 0, 1, h->s_main);
    if (dense) {
        if (int rc = fork(h)) return rc;
        dense_factor_async<T>(h, h->s_side);
        dense_logdiag<T>(tp<T>(h->A), (int)g.n0, h->dscal + 1, h->s_side);
    }
    if (g.M > 0) {
        factor_t<T>(h, F_TERMS, nullptr, nullptr, nullptr, h->scal_partial, nullptr,
                         nullptr);
        launch_reduce_scalar(h->dscal, h->scal_partial, (int)h->nblk_factor, nullptr, h->s_main);
    }
    if (dense)
        if (int rc = join(h)) return rc;
    if (int rc = finish(h, user)) return rc;
    if (dense && *h->hinfo != 0) {
        if (int rc = dense_retry<T>(h)) return rc;
        dense_logdiag<T>(tp<T>(h->A), (int)g.n0, h->dscal + 1, h->s_main);
        HC(hipMemcpyAsync(h->hscal, h->dscal, 8 * sizeof(double), hipMemcpyDeviceToHost, h->s_main));
        HC(hipStreamSynchronize(h->s_main));
    }
    *out = h->hscal[0] + (dense ? h->hscal[1] : 0.0);
    return 0;
}

// The refine_* ops take and return tree-order arrays: translate them to the internal order
// (x_int[i] = x_tree[map[i]]) and back. Without a relabelling (map null) the caller's array is
// used as is.
template <typename T>
const T* tree_in(const T* x, T* buf, const int32_t* map, int64_t n, hipStream_t st) {
    if (!map) return x;
    launch_gather<T>(buf, x, map, n, st);
    return buf;
}

template <typename T>
int op_refine_logdet_terms(ggp_graph* h, T* terms, hipStream_t user) {
    if (int rc = check_ready(h)) return rc;
    if (int rc = enter(h, user)) return rc;
    const Graph& g = h->g;
    if (g.M > 0) {
        T* out = g.i2tm ? tp<T>(h->xt) : terms;
        factor_t<T>(h, F_TERMS, nullptr, nullptr, out, h->scal_partial, nullptr, nullptr);
        if (g.i2tm) launch_scatter<T>(terms, out, g.i2tm, g.M, h->s_main);
    }
    return finish(h, user);
}

template <typename T>
int op_refine_inv(ggp_graph* h, const T* values, T* xi_ref, hipStream_t user) {
    if (int rc = check_ready(h)) return rc;
    if (int rc = enter(h, user)) return rc;
    const Graph& g = h->g;
    if (g.M > 0) {
        const T* vin = tree_in<T>(values, tp<T>(h->v), g.i2t, g.N, h->s_main);
        T* out = g.i2tm ? tp<T>(h->xt) : xi_ref;
        factor_t<T>(h, F_INV, nullptr, nullptr, nullptr, nullptr, vin, out);
        if (g.i2tm) launch_scatter<T>(xi_ref, out, g.i2tm, g.M, h->s_main);
    }
    return finish(h, user);
}

template <typename T>
int op_refine(ggp_graph* h, T* values, const T* xi_ref, hipStream_t user) {
    if (int rc = check_ready(h)) return rc;
    if (int rc = enter(h, user)) return rc;
    const Graph& g = h->g;
    if (g.M > 0) {
        T* v = g.i2t ? tp<T>(h->v) : values;
        const T* xr = tree_in<T>(xi_ref, tp<T>(h->xt), g.i2tm, g.M, h->s_main);
        if (g.i2t) launch_gather<T>(v, values, g.i2t, g.N, h->s_main);
        factor_t<T>(h, F_MV, tp<T>(h->mv), tp<T>(h->sd), nullptr, nullptr,
                         nullptr, nullptr);
        sweep_forward<T>(h, v, xr, 0, h->s_main);
        if (g.i2t) launch_scatter<T>(values, v, g.i2t, g.N, h->s_main);
    }
    return finish(h, user);
}

template <typename T>
int op_grad_xi(ggp_graph* h, const T* vbar, T* xbar, hipStream_t user) {
    if (int rc = check_ready(h)) return rc;
    if (int rc = enter(h, user)) return rc;
    Graph& g = h->g;
    T *vbt = tp<T>(h->vbt), *vb = tp<T>(h->vb), *xg = tp<T>(h->xg);
    if (int rc = fork(h)) return rc;
    dense_factor_async<T>(h, h->s_side);
    launch_gather<T>(vbt, vbar, g.idx, g.N, h->s_main);
    launch_sweep_prep<T>(g, nullptr, vb, h->s_main);
    zero_tail<T>(h, xg, h->s_main);
    factor_t<T>(h, F_MV, tp<T>(h->mv), tp<T>(h->sd), nullptr, nullptr, nullptr,
                     nullptr);
    // the sweep and L^T vb also store their values at xbar[idx[i]] (original order)
    sweep_reverse<T>(h, vb, vbt, xg, h->s_main, true, xbar, g.idx);
    if (int rc = join(h)) return rc;
    dense_trmv_t<T>(tp<T>(h->A), (int)g.n0, vb, xg, h->s_main, xbar, g.idx);
    scatter_tail<T>(h, xbar, xg, h->s_main);
    if (int rc = finish(h, user)) return rc;
    if (*h->hinfo != 0) {
        if (int rc = dense_retry<T>(h)) return rc;
        dense_trmv_t<T>(tp<T>(h->A), (int)g.n0, vb, xg, h->s_main);
        launch_scatter<T>(xbar, xg, g.idx, g.N, h->s_main);
        HC(hipStreamSynchronize(h->s_main));
    }
    return 0;
}

// Dense-layer cotangent for the op, enqueued on `st` into the dense rows of h->hist.
enum DenseGrad { DG_NONE, DG_LOGDET, DG_GENERATE, DG_INVLOSS };

template <typename T>
void dense_grad(ggp_graph* h, int kind, hipStream_t st, bool inverse_ready = false) {
    const Graph& g = h->g;
    const Table<T>& tb = table<T>(h);
    double* rows = h->hist + (size_t)pull_blocks(h) * h->hist_nb;
    const int n = (int)g.n0;
    if (kind == DG_LOGDET) {
        dense_logdiag<T>(tp<T>(h->A), n, h->dscal + 1, st);
        dense_grad_logdet<T>(g, tb, tp<T>(h->A), h->W, h->C, rows, h->nw_dense, st);
    } else if (kind == DG_GENERATE) {
        dense_grad_generate<T>(g, tb, tp<T>(h->A), tp<T>(h->vb), tp<T>(h->xt), h->W, h->C, h->Q,
                               h->u, rows, h->nw_dense, inverse_ready, st);
    } else if (kind == DG_INVLOSS) {
        // xi_dense = L \ y, alpha = L^-T xi_dense (src/dense.jl:229-240).
        T* xid = tp<T>(h->xt);
        T* alpha = tp<T>(h->tmp);
        dense_trsv<T>(tp<T>(h->A), n, tp<T>(h->v), xid, h->dsync, h->info, st);
        dense_trsv_t<T>(tp<T>(h->A), n, xid, alpha, h->dsync, h->info, st);
        launch_sumsq_half<T>(xid, n, h->dscal + 1, st);
        dense_grad_invloss<T>(g, tb, alpha, rows, h->nw_dense, st);
    }
}

// Shared driver of the four d/dvals ops.
//   mode: P_LOGDET / P_INVLOSS / P_GENVALS pullback; dense: which dense cotangent to add.
template <typename T>
int op_grad_vals(ggp_graph* h, int mode, int dkind, const T* in1, const T* in2, T* d_vals,
                 double* scalar_out, hipStream_t user) {
    if (int rc = check_ready(h)) return rc;
    if (is_aniso(h))
        return fail(GGP_ERR_ARG, "gradients w.r.t. the covariance table are defined for the "
                                 "isotropic table only (the anisotropic path is forward-only)");
    if (dkind != DG_NONE)
        if (int rc = ensure_dense64(h)) return rc;
    if (int rc = enter(h, user)) return rc;
    Graph& g = h->g;
    const Table<T>& tb = table<T>(h);
    const int nb = tb.P.nb;
    T *v = tp<T>(h->v), *xt = tp<T>(h->xt), *vb = tp<T>(h->vb), *vbt = tp<T>(h->vbt);
    launch_fill<double>(h->dscal, 0.0, 8, h->s_main);
    launch_fill<int>(h->info, 0, 1, h->s_main);
    const T* pull_v = nullptr;
    if (mode == P_GENVALS) {  // generate_grad_vals: forward field, then the reverse sweep
        if (int rc = fork(h)) return rc;
        dense_factor_async<T>(h, h->s_side);
        HC(hipEventRecord(h->ev_join, h->s_side));  // the factor is done
        launch_gather<T>(xt, in1, g.idx, g.N, h->s_main);
        launch_gather<T>(vbt, in2, g.idx, g.N, h->s_main);
        launch_sweep_prep<T>(g, v, vb, h->s_main);
        zero_tail<T>(h, v, h->s_main);
        factor_t<T>(h, F_MV, tp<T>(h->mv), tp<T>(h->sd), nullptr, nullptr, nullptr, nullptr);
        // The reverse sweep needs only mean_vec / std and the cotangent: it runs on its own
        // stream beside the dense factor and the forward chain.
        HC(hipEventRecord(h->ev_fac, h->s_main));
        HC(hipStreamWaitEvent(h->s_rev, h->ev_fac, 0));
        sweep_reverse<T>(h, vb, vbt, nullptr, h->s_rev, true);
        HC(hipEventRecord(h->ev_rev, h->s_rev));
        // L^-1 needs only the factor: it runs beside both sweeps (enqueued after the main
        // stream's first launches, which it does not hold up)
        dense_inverse<T>(tp<T>(h->A), (int)g.n0, h->W, h->C, h->s_side);
        // the forward sweep needs v[0:n0] = L xi[0:n0]: wait for the factor, not for the inverse
        HC(hipStreamWaitEvent(h->s_main, h->ev_join, 0));
        dense_trmv<T>(tp<T>(h->A), (int)g.n0, xt, v, h->s_main);
        sweep_forward<T>(h, v, xt, g.n0, h->s_main, true);
        HC(hipStreamWaitEvent(h->s_main, h->ev_rev, 0));
        pull_v = v;
        if (int rc = fork(h)) return rc;
        dense_grad<T>(h, DG_GENERATE, h->s_side, true);
    } else {
        if (mode == P_INVLOSS) {  // inverse loss: data (original order) or values (tree order)
            if (dkind == DG_INVLOSS) {
                launch_gather<T>(v, in1, g.idx, g.N, h->s_main);
                pull_v = v;
            } else {
                pull_v = tree_in<T>(in1, v, g.i2t, g.N, h->s_main);
            }
        }
        if (dkind != DG_NONE) {
            if (int rc = fork(h)) return rc;
            dense_factor_async<T>(h, h->s_side);
            dense_grad<T>(h, dkind, h->s_side);
        }
    }
    if (g.M > 0)
        pullback_t<T>(h, mode, pull_v, xt, vb);
    else
        launch_fill<double>(h->hist, 0.0, (int64_t)pull_blocks(h) * nb, h->s_main);
    if (mode != P_GENVALS && g.M > 0)
        launch_reduce_scalar(h->dscal, h->scal_partial, (int)pull_blocks(h), nullptr, h->s_main);
    if (dkind != DG_NONE)
        if (int rc = join(h)) return rc;
    const int rows = (int)pull_blocks(h) + (dkind != DG_NONE ? h->nw_dense : 0);
    launch_reduce_hist<T>(d_vals, h->hist, rows, nb, nullptr, h->s_main);
    if (int rc = finish(h, user)) return rc;
    if (dkind != DG_NONE && *h->hinfo != 0) {
        if (int rc = dense_retry<T>(h)) return rc;
        if (mode == P_GENVALS) {
            dense_trmv<T>(tp<T>(h->A), (int)g.n0, xt, v, h->s_main);
            sweep_forward<T>(h, v, xt, g.n0, h->s_main);
            sweep_reverse<T>(h, vb, vbt, nullptr, h->s_main);
            pullback_t<T>(h, mode, v, xt, vb);
        }
        dense_grad<T>(h, dkind, h->s_main);
        launch_reduce_hist<T>(d_vals, h->hist, rows, nb, nullptr, h->s_main);
        HC(hipMemcpyAsync(h->hscal, h->dscal, 8 * sizeof(double), hipMemcpyDeviceToHost, h->s_main));
        HC(hipStreamSynchronize(h->s_main));
    }
    if (scalar_out) *scalar_out = h->hscal[0] + (dkind != DG_NONE ? h->hscal[1] : 0.0);
    return 0;
}

// Shared driver of the four d/dpoints ops (src/grad.jl:168-377): the refinement pullback with
// Abar sent to the point positions (f64 atomics into h->dp), the dense term on the side stream
// into h->dpd, both rounded once into d_points (N x D, tree order).
//   mode: P_LOGDET / P_INVLOSS; dense: add the dense first layer.
template <typename T>
int op_grad_points(ggp_graph* h, int mode, bool dense, const T* in, T* d_points,
                   double* scalar_out, hipStream_t user) {
    if (int rc = check_ready(h)) return rc;
    if (is_aniso(h))
        return fail(GGP_ERR_ARG, "gradients w.r.t. the point positions are defined for the "
                                 "isotropic table only (the anisotropic path is forward-only)");
    if (!d_points) return fail(GGP_ERR_ARG, "null d_points");
    if (mode == P_INVLOSS && !in) return fail(GGP_ERR_ARG, "null values");
    Graph& g = h->g;
    const int64_t nd = g.N * g.D;
    if (!h->dp) {
        if (dmalloc(h, (void**)&h->dp, (size_t)nd * sizeof(double)) ||
            dmalloc(h, (void**)&h->dpd, (size_t)g.n0 * g.D * sizeof(double)))
            return GGP_ERR_HIP;
    }
    if (dense)
        if (int rc = ensure_dense64(h)) return rc;
    if (int rc = enter(h, user)) return rc;
    const Table<T>& tb = table<T>(h);
    T* v = tp<T>(h->v);
    launch_fill<double>(h->dscal, 0.0, 8, h->s_main);
    launch_fill<int>(h->info, 0, 1, h->s_main);
    launch_fill<double>(h->dp, 0.0, nd, h->s_main);
    const T* pull_v = nullptr;
    if (mode == P_INVLOSS) {
        if (dense) {  // data in the original order
            launch_gather<T>(v, in, g.idx, g.N, h->s_main);
            pull_v = v;
        } else {  // values in tree order
            pull_v = tree_in<T>(in, v, g.i2t, g.N, h->s_main);
        }
    }
    auto dense_part = [&](hipStream_t st) {
        const int n = (int)g.n0;
        if (mode == P_LOGDET) {
            dense_logdiag<T>(tp<T>(h->A), n, h->dscal + 1, st);
            dense_grad_points_logdet<T>(g, tb, tp<T>(h->A), h->W, h->C, h->dpd, st);
        } else {
            // xi_dense = L \ y, alpha = L^-T xi_dense (src/dense.jl:271-300)
            T* xid = tp<T>(h->xt);
            T* alpha = tp<T>(h->tmp);
            dense_trsv<T>(tp<T>(h->A), n, v, xid, h->dsync, h->info, st);
            dense_trsv_t<T>(tp<T>(h->A), n, xid, alpha, h->dsync, h->info, st);
            launch_sumsq_half<T>(xid, n, h->dscal + 1, st);
            dense_grad_points_invloss<T>(g, tb, alpha, h->dpd, st);
        }
    };
    if (dense) {
        if (int rc = fork(h)) return rc;
        dense_factor_async<T>(h, h->s_side);
        dense_part(h->s_side);
    }
    if (g.M > 0) {
        tstart(h, TM_PULLBACK, h->s_main);
        launch_pullback<T>(g, tb, mode | P_PTS, pull_v, nullptr, nullptr, h->dp, h->scal_partial,
                           pull_blocks(h), h->s_main);
        tstop(h, TM_PULLBACK, h->s_main);
        launch_reduce_scalar(h->dscal, h->scal_partial, (int)pull_blocks(h), nullptr, h->s_main);
    }
    if (dense)
        if (int rc = join(h)) return rc;
    const int64_t ndd = dense ? g.n0 * g.D : 0;
    launch_points_out<T>(d_points, h->dp, h->dpd, g.N, g.D, ndd, g.i2t, h->s_main);
    if (int rc = finish(h, user)) return rc;
    if (dense && *h->hinfo != 0) {
        if (int rc = dense_retry<T>(h)) return rc;
        launch_fill<double>(h->dscal + 1, 0.0, 1, h->s_main);
        dense_part(h->s_main);
        launch_points_out<T>(d_points, h->dp, h->dpd, g.N, g.D, ndd, g.i2t, h->s_main);
        HC(hipMemcpyAsync(h->hscal, h->dscal, 8 * sizeof(double), hipMemcpyDeviceToHost, h->s_main));
        HC(hipStreamSynchronize(h->s_main));
    }
    if (scalar_out) *scalar_out = h->hscal[0] + (dense ? h->hscal[1] : 0.0);
    return 0;
}

// ---- graph creation -----------------------------------------------------------------------
int create(ggp_graph** out, const uint32_t* coords, const int64_t* nbrs, const int64_t* offs,
           int64_t n_off, const int64_t* indices, int64_t n0, int64_t k, int64_t N, int32_t D,
           double scale, int32_t dtype) {
    if (!out) return fail(GGP_ERR_ARG, "null output handle");
    *out = nullptr;
    if (!supported_k(k)) return fail(GGP_ERR_K, "unsupported k (supported: 1 to 31)");
    if (!supported_d(D)) return fail(GGP_ERR_D, "unsupported D (supported: 2, 3, 4)");
    if (dtype != GGP_F32 && dtype != GGP_F64) return fail(GGP_ERR_ARG, "dtype must be GGP_F32 or GGP_F64");
    if (!(std::isfinite(scale) && scale > 0)) return fail(GGP_ERR_ARG, "scale must be finite and > 0");
    std::string err;
    if (int rc = check_graph_host(coords, nbrs, offs, n_off, indices, n0, k, N, D, &err))
        return fail(rc, err);
    const int64_t M = N - n0;

    ggp_graph* h = new ggp_graph();
    auto bail = [&](int rc) { free_all(h); delete h; return rc; };
    h->dtype = dtype;
    if (hipGetDevice(&h->dev) != hipSuccess) return bail(fail(GGP_ERR_HIP, "no HIP device"));
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, h->dev) == hipSuccess) {
        h->ncu = std::max(1, prop.multiProcessorCount);
        h->lds_max = std::min<size_t>(prop.sharedMemPerBlock, 65536);
    }
    if (const char* e = std::getenv("GGP_FACTOR_BLOCKS_PER_CU")) h->nblk_factor = (unsigned)(h->ncu * std::max(1, atoi(e)));
    else h->nblk_factor = (unsigned)(h->ncu * 4);
    if (const char* e = std::getenv("GGP_PULL_BLOCKS_PER_CU")) h->nblk_pull = (unsigned)(h->ncu * std::max(1, atoi(e)));
    else h->nblk_pull = (unsigned)(h->ncu * 6);  // the table + histogram LDS admits ~5 per CU
    // points per workgroup pass: kBlock (a lane per point) or kWidePts (32 lanes per point)
    const int64_t ppb = register_block_k(k) ? kBlock : kWidePts;
    if (!register_block_k(k)) {
        if (!std::getenv("GGP_FACTOR_BLOCKS_PER_CU")) h->nblk_factor = (unsigned)(h->ncu * 8);
        if (!std::getenv("GGP_PULL_BLOCKS_PER_CU")) h->nblk_pull = (unsigned)(h->ncu * 4);
    }
    h->nblk_factor = (unsigned)std::max<int64_t>(1, std::min<int64_t>(h->nblk_factor, (M + ppb - 1) / ppb));
    h->nblk_pull = (unsigned)std::max<int64_t>(1, std::min<int64_t>(h->nblk_pull, (M + ppb - 1) / ppb));
    h->nw_dense = (int)std::max<int64_t>(1, std::min<int64_t>(h->ncu, (n0 * (n0 + 1) / 2 + kBlock - 1) / kBlock));
    Graph& g = h->g;
    g.N = N; g.n0 = n0; g.M = M; g.K = k; g.D = D; g.scale = scale;
    g.offsets.assign(offs, offs + n_off);
    const size_t es = dtype == GGP_F32 ? 4 : 8;
    PackedGraph pk;
    const bool relabel = !std::getenv("GGP_TREE_ORDER");
    if (int rc = pack_graph(coords, nbrs, offs, n_off, indices, n0, k, N, D, relabel, &pk, &err))
        return bail(fail(rc, err));
    g.n_fwd_chunks = (int)pk.fwd.size();
    g.n_rev_chunks = (int)pk.revc.size();
    g.sweep_wgs = h->ncu;
    if (const char* e = std::getenv("GGP_SWEEP_WGS_PER_CU")) g.sweep_wgs = h->ncu * std::max(1, atoi(e));
    int rc = 0;
    rc |= dmalloc(h, (void**)&g.coords, (size_t)(N * D) * 4);
    rc |= dmalloc(h, (void**)&g.nbr, pk.nsoa.size() * 4);
    rc |= dmalloc(h, (void**)&g.rcnt, pk.rcnt.size() * 4);
    rc |= dmalloc(h, (void**)&g.rev, pk.rev.size() * 4);
    if (!pk.idx32.empty()) rc |= dmalloc(h, (void**)&g.idx, (size_t)N * 4);
    if (pk.relabel) {
        rc |= dmalloc(h, (void**)&g.i2t, (size_t)N * 4);
        rc |= dmalloc(h, (void**)&g.i2tm, pk.i2tm.size() * 4);
    }
    rc |= dmalloc(h, &h->mv, (size_t)(M * k) * es);
    rc |= dmalloc(h, &h->sd, (size_t)M * es);
    rc |= dmalloc(h, &h->v, (size_t)N * es);
    rc |= dmalloc(h, &h->xt, (size_t)N * es);
    rc |= dmalloc(h, &h->vb, (size_t)N * es);
    rc |= dmalloc(h, &h->vbt, (size_t)N * es);
    rc |= dmalloc(h, &h->xg, (size_t)N * es);
    rc |= dmalloc(h, &h->tmp, (size_t)n0 * es);
    rc |= dmalloc(h, &h->A, (size_t)(n0 * n0) * es);
    rc |= dmalloc(h, (void**)&h->scal_partial, std::max(h->nblk_factor, h->nblk_pull) * 8);
    rc |= dmalloc(h, &h->dstat, kStatBytes);
    rc |= dmalloc(h, (void**)&h->dsync, (size_t)dense_sync_ints((int)n0) * sizeof(int));
    rc |= dmalloc(h, (void**)&g.fwd_chunks, std::max<size_t>(pk.fwd.size(), 1) * sizeof(int4));
    rc |= dmalloc(h, (void**)&g.rev_chunks, std::max<size_t>(pk.revc.size(), 1) * sizeof(int4));
    rc |= dmalloc(h, (void**)&g.sweep_ticket, 16);
    if (rc) return bail(GGP_ERR_HIP);
    if (hipHostMalloc(&h->hstat, kStatBytes) != hipSuccess)
        return bail(fail(GGP_ERR_HIP, "hipHostMalloc failed"));
    h->dscal = static_cast<double*>(h->dstat);
    h->info = reinterpret_cast<int*>(static_cast<char*>(h->dstat) + 64);
    g.sweep_err = reinterpret_cast<int*>(static_cast<char*>(h->dstat) + 80);
    h->hscal = static_cast<double*>(h->hstat);
    h->hinfo = reinterpret_cast<int*>(static_cast<char*>(h->hstat) + 64);
    h->herr = reinterpret_cast<int*>(static_cast<char*>(h->hstat) + 80);
    static_assert(sizeof(Chunk) == sizeof(int4), "a sweep chunk is uploaded as an int4");
    static_assert(kPackBlock == kBlock && kPackRevSlots == kRevSlots && kPackRevNone == kRevNone,
                  "the packed layout is the sweep kernels' layout");
    if (hipMemcpy(g.coords, pk.coords.data(), (size_t)(N * D) * 4, hipMemcpyHostToDevice) != hipSuccess ||
        (pk.relabel && hipMemcpy(g.i2t, pk.i2t.data(), (size_t)N * 4, hipMemcpyHostToDevice) != hipSuccess) ||
        (pk.relabel && hipMemcpy(g.i2tm, pk.i2tm.data(), pk.i2tm.size() * 4, hipMemcpyHostToDevice) != hipSuccess) ||
        hipMemcpy(g.nbr, pk.nsoa.data(), pk.nsoa.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(g.rcnt, pk.rcnt.data(), pk.rcnt.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(g.rev, pk.rev.data(), pk.rev.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
        (!pk.idx32.empty() && hipMemcpy(g.idx, pk.idx32.data(), (size_t)N * 4, hipMemcpyHostToDevice) != hipSuccess) ||
        (!pk.fwd.empty() && hipMemcpy(g.fwd_chunks, pk.fwd.data(), pk.fwd.size() * sizeof(int4), hipMemcpyHostToDevice) != hipSuccess) ||
        (!pk.revc.empty() && hipMemcpy(g.rev_chunks, pk.revc.data(), pk.revc.size() * sizeof(int4), hipMemcpyHostToDevice) != hipSuccess) ||
        hipMemset(g.sweep_err, 0, 16) != hipSuccess)
        return bail(fail(GGP_ERR_HIP, "hipMemcpy of the graph failed"));
    if (hipStreamCreateWithFlags(&h->s_main, hipStreamNonBlocking) != hipSuccess ||
        hipStreamCreateWithFlags(&h->s_side, hipStreamNonBlocking) != hipSuccess ||
        hipStreamCreateWithFlags(&h->s_rev, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&h->ev_fac, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&h->ev_rev, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&h->ev_fork, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&h->ev_join, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&h->ev_user, hipEventDisableTiming) != hipSuccess)
        return bail(fail(GGP_ERR_HIP, "stream/event creation failed"));
    *out = h;
    return 0;
}

}  // namespace

// ================================== C ABI ======================================================
#define DISPATCH(h, CALL_F, CALL_D) ((h)->dtype == GGP_F32 ? (CALL_F) : (CALL_D))

extern "C" {

const char* ggp_last_error(void) { return g_last_error.c_str(); }

int ggp_supported(int64_t k, int32_t D) {
    if (!supported_k(k)) return fail(GGP_ERR_K, "unsupported k");
    if (!supported_d(D)) return fail(GGP_ERR_D, "unsupported D");
    return 0;
}

int ggp_graph_create(ggp_graph** out, const uint32_t* coords_host, const int64_t* neighbors_host,
                     const int64_t* offsets_host, int64_t n_offsets, const int64_t* indices_host,
                     int64_t n0, int64_t k, int64_t N, int32_t D, double scale, int32_t dtype) {
    return create(out, coords_host, neighbors_host, offsets_host, n_offsets, indices_host, n0, k,
                  N, D, scale, dtype);
}

int ggp_graph_destroy(ggp_graph* h) {
    if (!h) return 0;
    (void)hipSetDevice(h->dev);
    if (h->s_main) (void)hipStreamSynchronize(h->s_main);
    if (h->s_side) (void)hipStreamSynchronize(h->s_side);
    free_all(h);
    delete h;
    return 0;
}

int ggp_graph_shape(const ggp_graph* h, int64_t* N, int64_t* n0, int64_t* k, int32_t* D,
                    int64_t* n_levels, int32_t* dtype) {
    if (!h) return fail(GGP_ERR_ARG, "null handle");
    if (N) *N = h->g.N;
    if (n0) *n0 = h->g.n0;
    if (k) *k = h->g.K;
    if (D) *D = h->g.D;
    if (n_levels) *n_levels = (int64_t)h->g.offsets.size() - 1;
    if (dtype) *dtype = h->dtype;
    return 0;
}

int ggp_kernel_timers(ggp_graph* h, int32_t enable) {
    if (!h) return fail(GGP_ERR_ARG, "null handle");
    (void)hipSetDevice(h->dev);
    if (enable && !h->tev[0])
        for (int i = 0; i < 2 * TM_COUNT; ++i)
            if (hipEventCreate(&h->tev[i]) != hipSuccess) return fail(GGP_ERR_HIP, "hipEventCreate failed");
    h->timing = enable & ((1 << TM_COUNT) - 1);
    for (int t = 0; t < TM_COUNT; ++t) { h->tms[t] = 0; h->tcnt[t] = 0; h->tpending[t] = false; }
    return 0;
}

int ggp_selftest_sqrt_f32(uint32_t first_bits, uint32_t count, uint64_t* mismatches) {
    if (!mismatches) return fail(GGP_ERR_ARG, "null argument");
    unsigned long long* d = nullptr;
    HC(hipMalloc((void**)&d, sizeof(*d)));
    hipError_t e = hipMemset(d, 0, sizeof(*d));
    if (e == hipSuccess && count) {
        ggp::launch_sqrt_check(first_bits, count, d, nullptr);
        e = hipGetLastError();
    }
    unsigned long long hbad = 0;
    if (e == hipSuccess) e = hipMemcpy(&hbad, d, sizeof(hbad), hipMemcpyDeviceToHost);
    (void)hipFree(d);
    if (e != hipSuccess) return fail(GGP_ERR_HIP, std::string("sqrt self-test: ") + hipGetErrorString(e));
    *mismatches = hbad;
    return 0;
}

int ggp_selftest_div(int32_t dtype, uint64_t first, uint64_t count, uint32_t per_divisor,
                     uint64_t seed, uint64_t* mismatches) {
    if (!mismatches) return fail(GGP_ERR_ARG, "null argument");
    if (dtype != GGP_F32 && dtype != GGP_F64) return fail(GGP_ERR_ARG, "dtype must be GGP_F32 or GGP_F64");
    if (dtype == GGP_F32 && (first > 0xffffffffull || count > 0x100000000ull - first))
        return fail(GGP_ERR_ARG, "f32 divisor range past the 32-bit patterns");
    unsigned long long* d = nullptr;
    HC(hipMalloc((void**)&d, sizeof(*d)));
    hipError_t e = hipMemset(d, 0, sizeof(*d));
    if (e == hipSuccess && count && (per_divisor || dtype == GGP_F32)) {  // f32: the reciprocal too
        ggp::launch_div_check(dtype == GGP_F64, first, count, per_divisor, seed, d, nullptr);
        e = hipGetLastError();
    }
    unsigned long long hbad = 0;
    if (e == hipSuccess) e = hipMemcpy(&hbad, d, sizeof(hbad), hipMemcpyDeviceToHost);
    (void)hipFree(d);
    if (e != hipSuccess) return fail(GGP_ERR_HIP, std::string("division self-test: ") + hipGetErrorString(e));
    *mismatches = hbad;
    return 0;
}

int ggp_kernel_timer_read(const ggp_graph* h, const char* name, double* total_ms, int64_t* count) {
    if (!h || !name) return fail(GGP_ERR_ARG, "null argument");
    for (int t = 0; t < TM_COUNT; ++t)
        if (std::strcmp(name, kTimerNames[t]) == 0) {
            if (total_ms) *total_ms = h->tms[t];
            if (count) *count = h->tcnt[t];
            return 0;
        }
    return fail(GGP_ERR_ARG, std::string("unknown timer ") + name);
}

int ggp_set_cov_aniso(ggp_graph* h, const void* spatial_bins_host, int64_t n_s,
                      const void* z_bins_host, int64_t n_z, const void* grid_host, double alpha) {
    if (!h || !spatial_bins_host || !z_bins_host || !grid_host) return fail(GGP_ERR_ARG, "null argument");
    if (hipSetDevice(h->dev) != hipSuccess) return fail(GGP_ERR_HIP, "hipSetDevice failed");
    return DISPATCH(h, set_cov_aniso<float>(h, (const float*)spatial_bins_host, n_s, (const float*)z_bins_host, n_z, (const float*)grid_host, alpha),
                    set_cov_aniso<double>(h, (const double*)spatial_bins_host, n_s, (const double*)z_bins_host, n_z, (const double*)grid_host, alpha));
}

int ggp_set_cov_iso(ggp_graph* h, const void* bins_host, const void* vals_host, int64_t nbins) {
    if (!h || !bins_host || !vals_host) return fail(GGP_ERR_ARG, "null argument");
    if (hipSetDevice(h->dev) != hipSuccess) return fail(GGP_ERR_HIP, "hipSetDevice failed");
    return DISPATCH(h, set_cov<float>(h, (const float*)bins_host, (const float*)vals_host, nbins),
                    set_cov<double>(h, (const double*)bins_host, (const double*)vals_host, nbins));
}

#define ST(s) ((hipStream_t)(s))

int ggp_generate(ggp_graph* h, const void* xi, void* out, void* stream) {
    if (!h) return fail(GGP_ERR_ARG, "null handle");
    return DISPATCH(h, op_generate<float>(h, (const float*)xi, (float*)out, ST(stream)),
                    op_generate<double>(h, (const double*)xi, (double*)out, ST(stream)));
}
int ggp_generate_inv(ggp_graph* h, const void* values, void* xi, void* stream) {
    if (!h) return fail(GGP_ERR_ARG, "null handle");
    return DISPATCH(h, op_generate_inv<float>(h, (const float*)values, (float*)xi, ST(stream)),
                    op_generate_inv<double>(h, (const double*)values, (double*)xi, ST(stream)));
}
int ggp_generate_logdet(ggp_graph* h, double* out, void* stream) {
    if (!h || !out) return fail(GGP_ERR_ARG, "null argument");
    return DISPATCH(h, op_logdet<float>(h, true, out, ST(stream)),
                    op_logdet<double>(h, true, out, ST(stream)));
}
int ggp_refine_logdet(ggp_graph* h, double* out, void* stream) {
    if (!h || !out) return fail(GGP_ERR_ARG, "null argument");
    return DISPATCH(h, op_logdet<float>(h, false, out, ST(stream)),
                    op_logdet<double>(h, false, out, ST(stream)));
}
int ggp_refine_logdet_terms(ggp_graph* h, void* terms, void* stream) {
    if (!h) return fail(GGP_ERR_ARG, "null handle");
    return DISPATCH(h, op_refine_logdet_terms<float>(h, (float*)terms, ST(stream)),
                    op_refine_logdet_terms<double>(h, (double*)terms, ST(stream)));
}
int ggp_refine_inv(ggp_graph* h, const void* values_tree, void* xi_ref, void* stream) {
    if (!h) return fail(GGP_ERR_ARG, "null handle");
    return DISPATCH(h, op_refine_inv<float>(h, (const float*)values_tree, (float*)xi_ref, ST(stream)),
                    op_refine_inv<double>(h, (const double*)values_tree, (double*)xi_ref, ST(stream)));
}
int ggp_refine(ggp_graph* h, void* values_tree, const void* xi_ref, void* stream) {
    if (!h) return fail(GGP_ERR_ARG, "null handle");
    return DISPATCH(h, op_refine<float>(h, (float*)values_tree, (const float*)xi_ref, ST(stream)),
                    op_refine<double>(h, (double*)values_tree, (const double*)xi_ref, ST(stream)));
}
int ggp_generate_grad_xi(ggp_graph* h, const void* vbar, void* xbar, void* stream) {
    if (!h) return fail(GGP_ERR_ARG, "null handle");
    return DISPATCH(h, op_grad_xi<float>(h, (const float*)vbar, (float*)xbar, ST(stream)),
                    op_grad_xi<double>(h, (const double*)vbar, (double*)xbar, ST(stream)));
}
int ggp_generate_grad_vals(ggp_graph* h, const void* xi, const void* vbar, void* d_vals,
                           void* stream) {
    if (!h) return fail(GGP_ERR_ARG, "null handle");
    return DISPATCH(h, op_grad_vals<float>(h, P_GENVALS, DG_GENERATE, (const float*)xi, (const float*)vbar, (float*)d_vals, nullptr, ST(stream)),
                    op_grad_vals<double>(h, P_GENVALS, DG_GENERATE, (const double*)xi, (const double*)vbar, (double*)d_vals, nullptr, ST(stream)));
}
int ggp_refine_logdet_grad_vals(ggp_graph* h, void* d_vals, double* logdet, void* stream) {
    if (!h) return fail(GGP_ERR_ARG, "null handle");
    return DISPATCH(h, op_grad_vals<float>(h, P_LOGDET, DG_NONE, nullptr, nullptr, (float*)d_vals, logdet, ST(stream)),
                    op_grad_vals<double>(h, P_LOGDET, DG_NONE, nullptr, nullptr, (double*)d_vals, logdet, ST(stream)));
}
int ggp_generate_logdet_grad_vals(ggp_graph* h, void* d_vals, double* logdet, void* stream) {
    if (!h) return fail(GGP_ERR_ARG, "null handle");
    return DISPATCH(h, op_grad_vals<float>(h, P_LOGDET, DG_LOGDET, nullptr, nullptr, (float*)d_vals, logdet, ST(stream)),
                    op_grad_vals<double>(h, P_LOGDET, DG_LOGDET, nullptr, nullptr, (double*)d_vals, logdet, ST(stream)));
}
int ggp_refine_inv_loss_grad_vals(ggp_graph* h, const void* values_tree, void* d_vals,
                                  double* loss, void* stream) {
    if (!h) return fail(GGP_ERR_ARG, "null handle");
    return DISPATCH(h, op_grad_vals<float>(h, P_INVLOSS, DG_NONE, (const float*)values_tree, nullptr, (float*)d_vals, loss, ST(stream)),
                    op_grad_vals<double>(h, P_INVLOSS, DG_NONE, (const double*)values_tree, nullptr, (double*)d_vals, loss, ST(stream)));
}
int ggp_generate_inv_loss_grad_vals(ggp_graph* h, const void* data, void* d_vals, double* loss,
                                    void* stream) {
    if (!h) return fail(GGP_ERR_ARG, "null handle");
    return DISPATCH(h, op_grad_vals<float>(h, P_INVLOSS, DG_INVLOSS, (const float*)data, nullptr, (float*)d_vals, loss, ST(stream)),
                    op_grad_vals<double>(h, P_INVLOSS, DG_INVLOSS, (const double*)data, nullptr, (double*)d_vals, loss, ST(stream)));
}

int ggp_refine_logdet_grad_points(ggp_graph* h, void* d_points, double* logdet, void* stream) {
    if (!h) return fail(GGP_ERR_ARG, "null handle");
    return DISPATCH(h, op_grad_points<float>(h, P_LOGDET, false, nullptr, (float*)d_points, logdet, ST(stream)),
                    op_grad_points<double>(h, P_LOGDET, false, nullptr, (double*)d_points, logdet, ST(stream)));
}
int ggp_generate_logdet_grad_points(ggp_graph* h, void* d_points, double* logdet, void* stream) {
    if (!h) return fail(GGP_ERR_ARG, "null handle");
    return DISPATCH(h, op_grad_points<float>(h, P_LOGDET, true, nullptr, (float*)d_points, logdet, ST(stream)),
                    op_grad_points<double>(h, P_LOGDET, true, nullptr, (double*)d_points, logdet, ST(stream)));
}
int ggp_refine_inv_loss_grad_points(ggp_graph* h, const void* values_tree, void* d_points,
                                    double* loss, void* stream) {
    if (!h) return fail(GGP_ERR_ARG, "null handle");
    return DISPATCH(h, op_grad_points<float>(h, P_INVLOSS, false, (const float*)values_tree, (float*)d_points, loss, ST(stream)),
                    op_grad_points<double>(h, P_INVLOSS, false, (const double*)values_tree, (double*)d_points, loss, ST(stream)));
}
int ggp_generate_inv_loss_grad_points(ggp_graph* h, const void* data, void* d_points,
                                      double* loss, void* stream) {
    if (!h) return fail(GGP_ERR_ARG, "null handle");
    return DISPATCH(h, op_grad_points<float>(h, P_INVLOSS, true, (const float*)data, (float*)d_points, loss, ST(stream)),
                    op_grad_points<double>(h, P_INVLOSS, true, (const double*)data, (double*)d_points, loss, ST(stream)));
}

}  // extern "C"
