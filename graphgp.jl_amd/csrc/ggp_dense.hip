// ggp_dense.hip — the dense first layer (n0 x n0) on the GPU: src/dense.jl and the dense parts
// of src/grad.jl / src/grad_generate_vals.jl, which the reference runs on the host every call.
//
// Factor and solves (precision T) accumulate every entry as the same fma chain, in the same
// order, as the unblocked column-by-column Cholesky / substitution: a right-looking blocked
// update that folds each 32-wide panel into the trailing entries in column order produces
// exactly the left-looking sums. Gradients (f64 internally) use the matrix form of the
// Cholesky adjoint, Abar = L^-T Phi(L^T Lbar) L^-1 (Phi = lower triangle, halved diagonal),
// instead of the reference's scalar reverse sweep (src/grad_generate_vals.jl:18-39), which is
// the same derivative evaluated in a parallel order.
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "ggp_internal.h"

namespace ggp {


static inline unsigned cdiv(int64_t a, int64_t b) { return (unsigned)((a + b - 1) / b); }

// ---- assembly (src/dense.jl:15-40) ----------------------------------------------------------
template <typename T, int D, bool ANISO>
__global__ void k_dense_assemble(T* __restrict__ A, const uint32_t* __restrict__ coords, int n,
                                 T scale, const TabEnt<T>* __restrict__ tab,
                                 const uint16_t* __restrict__ acc, const TabParams<T>* __restrict__ Pp, T diag_add,
                                 AnisoArgs<T> an, int* __restrict__ z0, int n_z0,
                                 int* __restrict__ z1, int n_z1, T* __restrict__ mb,
                                 int64_t n_mb, T mbv) {
    // Side jobs, so the Cholesky launch follows this one directly: the first workgroup zeroes
    // the factor's status and task flags (z0, z1); all of them set its mailboxes (mb) to the
    // pending marker mbv.
    if (blockIdx.x == 0 && blockIdx.y == 0) {
        const int t = threadIdx.y * 16 + threadIdx.x;
        for (int q = t; q < n_z0; q += 256) z0[q] = 0;
        for (int q = t; q < n_z1; q += 256) z1[q] = 0;
    }
    if (n_mb) {
        const int64_t nb = (int64_t)gridDim.x * gridDim.y;
        const int64_t b = (int64_t)blockIdx.y * gridDim.x + blockIdx.x;
        for (int64_t q = b * 256 + threadIdx.y * 16 + threadIdx.x; q < n_mb; q += nb * 256) mb[q] = mbv;
    }
    if (blockIdx.x > blockIdx.y) return;  // the whole block lies above the diagonal
    extern __shared__ __align__(16) unsigned char smem[];
    const int j = blockIdx.x * 16 + threadIdx.x;
    const int i = blockIdx.y * 16 + threadIdx.y;
    TabParams<T> P{};
    if (!ANISO) P = *Pp;
    auto entry = [&](const AnisoArgs<T>& av) {
        if (i >= n || j > i) return;
        if (i == j) {
            const T d0 = ANISO ? aniso_lookup(T(0), T(0), av) : P.v0;
            A[(int64_t)i * n + i] = diag_add == T(0) ? d0 : d0 + diag_add;
            return;
        }
        uint32_t ci[D], cj[D];
#pragma unroll
        for (int d = 0; d < D; ++d) {
            ci[d] = coords[(int64_t)i * D + d];
            cj[d] = coords[(int64_t)j * D + d];
        }
        const T v = ANISO ? aniso_pair<T, D>(ci, cj, scale, av)
                          : cov_lookup(radius<T>(sqdist<D>(ci, cj), scale), tab, acc, P);
        A[(int64_t)i * n + j] = v;
        A[(int64_t)j * n + i] = v;
    };
    // staged axes (the whole workgroup stages them) are read from LDS on that side only
    if (ANISO && an.lds != 0) entry(aniso_stage_lds(an, smem));
    else entry(an);
}

// ---- tiled Cholesky: one persistent launch ----------------------------------------------------
// The lower triangle is cut into 32x32 tiles (i, j), i >= j. Every tile is one task:
//   1. its entries receive fma(-L[r][p], L[c][p], .) for p = 0, 1, ... over the finished tiles
//      (i, k) and (j, k), k < j, in increasing k (streamed: each k-tile is applied as soon as its
//      two inputs are published);
//   2. a diagonal tile is then factored right-looking by one wavefront (lane r owns row r; the
//      pivot and the column come from their lanes by readlane), an off-diagonal tile solved row
//      by row against the published L[j][j].
// Entry (r, c) thus receives exactly the fma chain of the unblocked left-looking recurrence, in
// the same order, and the factor is bit-identical to it. LAPACK potrf's failure condition (a
// non-positive pivot, src/dense.jl:47-48) sets bit 0 of *info.
//
// Scheduling: workgroups take tasks from an atomic ticket counter in column-major tile order,
// which is a topological order of the task graph, so a task only ever waits for tasks already
// taken by running workgroups and the launch cannot deadlock, whatever the residency. A finished
// tile is published with a release store of its flag after its stores; consumers acquire the
// flag. Every wait is bounded: past kDfSpinLimit polls the waiter sets bit 1 of *info and goes
// on, so every workgroup exits; the host reports that as an error.
constexpr int kDfThreads = 256;
constexpr int kDfSpinLimit = 1 << 20;  // polls: about a second at most

// Poll with relaxed loads (no cache invalidation per poll), then one acquire fence.
__device__ inline void df_wait(const int* flag, int* info) {
    int spins = 0;
    while (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0) {
        __builtin_amdgcn_s_sleep(1);
        if (++spins > kDfSpinLimit) {
            atomicOr(info, 2);
            break;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}

// df_wait for a whole wavefront in uniform control flow: every lane polls the same flag, and the
// value is made wave-uniform so the loop's exit is too.
__device__ inline void df_wait_uniform(const int* flag, int* info) {
    int spins = 0;
    while (__builtin_amdgcn_readfirstlane(
               __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) == 0) {
        __builtin_amdgcn_s_sleep(1);
        if (++spins > kDfSpinLimit) {
            atomicOr(info, 2);
            break;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}

// sync = [ticket, flags[nt * nt]] (zeroed before the launch).
template <typename T>
__global__ void __launch_bounds__(kDfThreads) k_potrf_tiles(T* __restrict__ A, int n, int nt,
                                                            int* __restrict__ sync,
                                                            int* __restrict__ info) {
    __shared__ T sA[kTile][kTile + 1];
    __shared__ T sB[kTile][kTile + 1];
    __shared__ int s_task;
    int* ticket = sync;
    int* flags = sync + 1;
    const int tid = threadIdx.x;
    const int c = tid & (kTile - 1), r0 = tid >> 5;  // entries (r0 + 8q, c), q = 0..3
    const int ntiles = nt * (nt + 1) / 2;
    // The loop test is on a workgroup-uniform value the compiler can see as uniform
    // (readfirstlane), and the single-thread work (publish, next ticket) sits mid-body between
    // barriers: a lane-divergent branch at the loop head or latch lets the compiler split the
    // loop, which separates the flag store from the task it publishes.
    if (tid == 0) s_task = atomicAdd(ticket, 1);
    __syncthreads();
    int t = __builtin_amdgcn_readfirstlane(s_task);
    while (t < ntiles) {
        __syncthreads();
        int j = 0, rem = t;
        while (rem >= nt - j) { rem -= nt - j; ++j; }
        const int i = j + rem;
        const int i0 = i * kTile, j0 = j * kTile;
        const bool diag = i == j;
        // Rows and columns past n are padding: zero, with a unit diagonal, so they stay finite
        // and never feed a real entry (L is lower triangular).
        T acc[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int r = r0 + 8 * q;
            acc[q] = (i0 + r < n && j0 + c < n) ? A[(int64_t)(i0 + r) * n + j0 + c]
                                                : (diag && r == c ? T(1) : T(0));
        }
        for (int k = 0; k < j; ++k) {
            if (tid == 0) {
                df_wait(&flags[i * nt + k], info);
                if (!diag) df_wait(&flags[j * nt + k], info);
            }
            __syncthreads();
            const int k0 = k * kTile;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int r = r0 + 8 * q;
                sA[r][c] = i0 + r < n ? A[(int64_t)(i0 + r) * n + k0 + c] : T(0);
                sB[r][c] = j0 + r < n ? A[(int64_t)(j0 + r) * n + k0 + c] : T(0);
            }
            __syncthreads();
#pragma unroll 8
            for (int p = 0; p < kTile; ++p) {
                const T lc = sB[c][p];
#pragma unroll
                for (int q = 0; q < 4; ++q) acc[q] = num<T>::fma(-sA[r0 + 8 * q][p], lc, acc[q]);
            }
            __syncthreads();
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) sA[r0 + 8 * q][c] = acc[q];
        if (!diag) {
            if (tid == 0) df_wait(&flags[j * nt + j], info);
            __syncthreads();
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int r = r0 + 8 * q;
                sB[r][c] = (j0 + r < n && c <= r) ? A[(int64_t)(j0 + r) * n + j0 + c] : T(0);
            }
        }
        __syncthreads();
        if (tid < 64) {
            const int r = tid & (kTile - 1);
            const bool live = tid < kTile && i0 + r < n;
            T a[kTile];
#pragma unroll
            for (int cc = 0; cc < kTile; ++cc) a[cc] = sA[r][cc];
            if (diag) {
                // Entries above the diagonal are scratch: they take harmless updates and are
                // never stored, which keeps every update unconditional.
                bool bad = false;
#pragma unroll
                for (int p = 0; p < kTile; ++p) {
                    const T piv = bcast(a[p], p);
                    bad = bad || !(piv > T(0));
                    const T d = num<T>::sqrt(piv);
                    const T l = a[p] / d;
                    a[p] = r == p ? d : l;
#pragma unroll
                    for (int cc = p + 1; cc < kTile; ++cc)
                        a[cc] = num<T>::fma(-a[p], bcast(a[p], cc), a[cc]);
                }
                if (live) {
                    T* wp = A + (int64_t)(i0 + r) * n + j0;
#pragma unroll
                    for (int cc = 0; cc < kTile; ++cc)
                        if (cc <= r) wp[cc] = a[cc];
                }
                if (tid == 0 && bad) atomicOr(info, 1);
            } else {
#pragma unroll
                for (int jj = 0; jj < kTile; ++jj) {
                    T tt = a[jj];
#pragma unroll
                    for (int p = 0; p < jj; ++p) tt = num<T>::fma(-a[p], sB[jj][p], tt);
                    a[jj] = tt / sB[jj][jj];
                }
                if (live) {
                    T* wp = A + (int64_t)(i0 + r) * n + j0;
#pragma unroll
                    for (int cc = 0; cc < kTile; ++cc) wp[cc] = a[cc];
                }
            }
        }
        __syncthreads();
        if (tid == 0) {
            __hip_atomic_store(&flags[i * nt + j], 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
            s_task = atomicAdd(ticket, 1);
        }
        __syncthreads();
        t = __builtin_amdgcn_readfirstlane(s_task);
    }
}

// ---- the same factor with the diagonal chain kept in one workgroup -----------------------
// The critical path of the tiled factor is the chain diagonal (j, j) -> sub-diagonal (j+1, j)
// -> diagonal (j+1, j+1). Above, each link is a different task, so every step pays two
// cross-workgroup hand-offs (publish, poll, reload). Here the first workgroup to start (ticket
// 0) is the walker: for every j it factors (j, j) and then solves (j+1, j) itself, keeping
// L[j][j] and L[j+1][j] in LDS. It starts each tile from a partial sum over k < j-1 that a
// helper task accumulated one step earlier (in place, flagged), and adds the k = j-1 term
// itself, so each entry still receives its fma chain in increasing k. The helpers take, by
// ticket, in column-group order g = 0, 1, ...: the tiles (i, g), i >= g+2 (as above), then the
// partial sums of (g+2, g+2) and (g+3, g+2) over k < g+1. Every helper task waits only for
// tasks of earlier groups (or earlier in its own group) and for walker steps <= g, and walker
// step j waits only for groups <= j-1, so the launch cannot deadlock whatever the residency.
template <typename T>
__device__ __forceinline__ void walk_load(T (&acc)[4], const T* A, int n, int i, int j, int r0, int c) {
    const int i0 = i * kTile, j0 = j * kTile;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int r = r0 + 8 * q;
        acc[q] = (i0 + r < n && j0 + c < n) ? A[(int64_t)(i0 + r) * n + j0 + c]
                                            : (i == j && r == c ? T(1) : T(0));
    }
}

// acc[q] -= X[r0+8q][:] . Y[c][:] over the 32 columns, in column order.
template <typename T>
__device__ __forceinline__ void walk_term(T (&acc)[4], const T (*X)[kTile + 1], const T (*Y)[kTile + 1],
                                 int r0, int c) {
#pragma unroll 8
    for (int p = 0; p < kTile; ++p) {
        const T lc = Y[c][p];
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[q] = num<T>::fma(-X[r0 + 8 * q][p], lc, acc[q]);
    }
}

// Terms k in [k0, k1) of tile (i, j) from the published tiles (i, k) and (j, k).
template <typename T>
__device__ __forceinline__ void walk_accumulate(T (&acc)[4], const T* A, int n, int nt, int i, int j,
                                       int k0, int k1, const int* flags, int* info,
                                       T (*sA)[kTile + 1], T (*sB)[kTile + 1], int tid, int r0,
                                       int c) {
    const int i0 = i * kTile, j0 = j * kTile;
    for (int k = k0; k < k1; ++k) {
        if (tid == 0) {
            df_wait(&flags[i * nt + k], info);
            if (i != j) df_wait(&flags[j * nt + k], info);
        }
        __syncthreads();
        const int kk = k * kTile;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int r = r0 + 8 * q;
            sA[r][c] = i0 + r < n ? A[(int64_t)(i0 + r) * n + kk + c] : T(0);
            sB[r][c] = j0 + r < n ? A[(int64_t)(j0 + r) * n + kk + c] : T(0);
        }
        __syncthreads();
        walk_term(acc, sA, sB, r0, c);
        __syncthreads();
    }
}

// Whether the walker factor of the element type takes one reciprocal square root per column
// (pivot * rsq, within 1 ulp) instead of sqrt and a division. Off for both types: with sqrt and
// the IEEE division every entry of the factor carries the unblocked recurrence's bits, so the
// factor equals the oracle's (and the Float32 dense-layer cotangents, which amplify the
// factor's rounding through L^-1, agree with the oracle's to the rounding of their own sums).
template <typename T> constexpr bool kRsqFactor = false;

__host__ __device__ inline int walk_group_tasks(int g, int nt) {
    return std::max(0, nt - g - 2) + (g + 2 < nt ? 1 : 0) + (g + 3 < nt ? 1 : 0);
}

constexpr int kLtPitch = kTile + 4;  // transposed L rows, 16-byte aligned

// Position of row c of L in a row of the tile solves' transposed L (G lanes per row, lane g
// holding columns g, g + G, ...): the columns of lane g are contiguous.
template <int G>
__host__ __device__ constexpr int walk_perm(int c) {
    return (c % G) * (kTile / G) + c / G;
}

// sync = [ticket, tile flags[nt*nt], diagonal-partial flags[nt], sub-diagonal-partial flags[nt],
// (padding to 8 bytes), reciprocal diagonal[nt*kTile] (f32 walker)]: ints before the last part.
__host__ __device__ inline int dense_sync_flag_ints(int nt) { return (nt * nt + 2 * nt + 2) & ~1; }
// After the reciprocal diagonal (2 nt kTile ints): the walker's two mailboxes, each nt tiles of
// kTile x kTile values of the element type, published value by value (sweep_publish): L[g][g]
// for the helpers' solves, and the helpers' L[g+2][g] for the walker's sub-diagonal term. They
// hold the pending marker before a launch.
template <typename T>
__host__ __device__ inline T* dense_mbox(int* sync, int nt) {
    return reinterpret_cast<T*>(sync + dense_sync_flag_ints(nt) + 2 * nt * kTile);
}
__host__ __device__ inline int64_t dense_mbox_values(int nt) { return (int64_t)2 * nt * kTile * kTile; }

// Walker factor of the tile in sA into global tile (j, j) and, transposed, into Lt (LDS; zero
// above the diagonal). Right-looking by columns on one wavefront: lane 32h + r holds row r,
// columns 16h .. 16h+15. At step p the pivot comes from its lane by readlane; the lanes holding
// column p scale it and publish it to LDS (col, rows <= p as zero), and every lane reads its 16
// column values back with broadcast reads and updates its entries: entry (r, c) takes
// fma(-L[r][p], L[c][p], .) when p < c, so each entry keeps the unblocked left-looking chain in
// its order; a finished entry (c <= p) takes fma(-L[r][p], 0, .), no change but for the sign of
// a zero, until p = 15 and nothing after (both halves skip columns that are finished in both).
// Entries above the diagonal are scratch (updated, never stored).
// L[p][p] = sqrt(pivot) (f32: sqrt_rn_any_f32, the same bits) and the column divided by it (the
// oracle's bits). With kRsqFactor (off):
// one reciprocal square root per column (v_rsq_f32, within 1 ulp), L[p][p] = pivot * rsq and
// the column multiplied by rsq, which takes the square root and the division off the
// column-to-column chain; rsq then goes to inv (LDS) and dinv (global, for the helpers' solves).
// Called by wave 0. STREAM: column p of L goes to row p of Lt in the order of walk_perm<4> as
// it is finished, and after every fourth column *prog = pbase + p + 1 (LDS, release), so the
// solve walk_solve_grp<T, 4, true> on other wavefronts can follow four columns at a time.
template <typename T, bool STREAM = false>
__device__ __forceinline__ void walk_factor_t(T* A, int n, int j, const T (*sA)[kTile + 1],
                                     T (*Lt)[kLtPitch], T* inv, T* dinv, T (*col)[kTile],
                                     int tid, int* info, int* prog = nullptr, int pbase = 0,
                                     T* mbox = nullptr) {
    constexpr bool kRsq = kRsqFactor<T>;
    const int r = tid & (kTile - 1), h = tid >> 5;
    const bool live = j * kTile + r < n;
    T a[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) a[u] = sA[r][16 * h + u];
    bool bad = false;
    T myinv = T(0);
#pragma unroll
    for (int p = 0; p < kTile; ++p) {
        const int hp = p >> 4, up = p & 15;
        const bool mine = h == hp;  // this lane holds column p
        const T piv = bcast(a[up], 32 * hp + p);
        bad = bad || !(piv > T(0));
        T d, l;
        if (kRsq) {
            const T rs = (T)__builtin_amdgcn_rsqf((float)piv);
            d = piv * rs;
            l = a[up] * rs;
            myinv = (mine && r == p) ? rs : myinv;
        } else {
            if constexpr (std::is_same<T, float>::value) d = sqrt_rn_any_f32(piv);
            else d = num<T>::sqrt(piv);
            l = a[up] / d;
        }
        a[up] = mine ? (r == p ? d : l) : a[up];
        T* cp = col[p & 1];
        if (mine) cp[r] = r > p ? l : T(0);
        if (STREAM && mine) Lt[p][walk_perm<4>(r)] = r > p ? l : (r == p ? d : T(0));
        wave_sync_lds();
        if (STREAM && (p & 3) == 3) {  // columns released four at a time
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            if (tid == 0) __hip_atomic_store(prog, pbase + p + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        const T own = cp[r];
        T cv[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) cv[u] = cp[16 * h + u];
        // columns <= p are finished: past p = 15 both halves skip them (below, every lane's
        // column u of half 0 is finished, and cv is zero there)
#pragma unroll
        for (int u = 0; u < 16; ++u)
            if (p < 16 || u > p - 16) a[u] = num<T>::fma(-own, cv[u], a[u]);
    }
    const bool diag_lane = h == (r >> 4);  // holds L[r][r] (and its reciprocal)
    if (live) {
        T* wp = A + (int64_t)(j * kTile + r) * n + j * kTile + 16 * h;
        if (sizeof(T) == 4 && (n & 1) == 0) {
            // f32 rows of even length: pairs of columns in one 64-bit store where both are in
            // the lower triangle
#pragma unroll
            for (int u = 0; u < 16; u += 2) {
                if (16 * h + u + 1 <= r) {
                    const uint64_t b2 = (uint64_t)num<T>::bits(a[u]) |
                                        ((uint64_t)num<T>::bits(a[u + 1]) << 32);
                    *reinterpret_cast<uint64_t*>(wp + u) = b2;
                } else if (16 * h + u == r) {
                    wp[u] = a[u];
                }
            }
        } else {
#pragma unroll
            for (int u = 0; u < 16; ++u)
                if (16 * h + u <= r) wp[u] = a[u];
        }
        if (kRsq && diag_lane) dinv[j * kTile + r] = myinv;
    }
    if (mbox) {  // the whole tile, row-major, value by value (f32: two per 64-bit store)
        if constexpr (sizeof(T) == 4) {
#pragma unroll
            for (int u = 0; u < 16; u += 2) {
                const uint64_t b2 = (uint64_t)__float_as_uint(a[u]) |
                                    ((uint64_t)__float_as_uint(a[u + 1]) << 32);
                __hip_atomic_store(reinterpret_cast<uint64_t*>(&mbox[r * kTile + 16 * h + u]), b2,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        } else {
#pragma unroll
            for (int u = 0; u < 16; ++u) sweep_publish(&mbox[r * kTile + 16 * h + u], a[u]);
        }
    }
    if (kRsq && diag_lane) inv[r] = myinv;
    if (!STREAM) {
#pragma unroll
        for (int u = 0; u < 16; ++u) Lt[16 * h + u][r] = 16 * h + u <= r ? a[u] : T(0);
    }
    if (tid == 0 && bad) atomicOr(info, 1);
}

// Waits, wave-uniformly, until the LDS counter *v reaches target (bounded: past kDfSpinLimit
// polls bit 1 of *info is set and the wait ends), then orders the later LDS reads after it;
// returns the value seen (target after a timeout).
__device__ __forceinline__ int lds_wait_ge(const int* v, int target, int* info) {
    int spins = 0, seen;
    while ((seen = __builtin_amdgcn_readfirstlane(
                __hip_atomic_load(v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP))) < target) {
        __builtin_amdgcn_s_sleep(1);
        if (++spins > kDfSpinLimit) {
            atomicOr(info, 2);
            seen = target;
            break;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    return seen;
}


// ---- tile solves X L^T = B with G lanes per row ----
// Lane g of a row's group holds the row's columns c = G k + g (k < kTile / G). Column p is
// divided on its lane (g = p mod G) by L[p][p], and the quotient goes to the other lanes of the
// group by a DPP broadcast (quad_perm for G <= 4; for G = 8, row_newbcast into each half of a
// 16-lane row), after which every later column of the row takes fma(-x, L[c][p], .): each
// entry receives the row-by-row substitution's terms in its order, then its division, which is
// div_rcp with RN(1 / L[c][c]) from rcp_rn (together the IEEE quotient). L comes transposed and
// permuted: Lp[p][walk_perm<G>(c)] = L[c][p], zero for c < p, so a lane's values of column p
// are 16-byte aligned and contiguous.
template <int G, int O>
constexpr int walk_qsel() {
    int s = 0;
    for (int q = 0; q < 4; ++q) s |= ((q & ~(G - 1)) | O) << (2 * q);
    return s;
}

// The value of lane O of each G-lane group, for every lane of the group.
template <int G, int O>
__device__ __forceinline__ int walk_gbcast(int x) {
    static_assert(G == 2 || G == 4 || G == 8, "groups of 2, 4 or 8 lanes");
    if constexpr (G <= 4) {
        return __builtin_amdgcn_update_dpp(0, x, walk_qsel<G, O>(), 0xf, 0xf, false);
    } else {
        // row_newbcast:n (DPP control 0x150 + n): lane n of the 16-lane row; bank mask 0x3
        // writes lanes 0-7 of the row, 0xc lanes 8-15
        const int lo = __builtin_amdgcn_update_dpp(0, x, 0x150 + O, 0xf, 0x3, false);
        return __builtin_amdgcn_update_dpp(lo, x, 0x158 + O, 0xf, 0xc, false);
    }
}
template <int G, int O>
__device__ __forceinline__ float walk_gbcast(float x) {
    return __int_as_float(walk_gbcast<G, O>(__float_as_int(x)));
}
template <int G, int O>
__device__ __forceinline__ double walk_gbcast(double x) {
    const long long v = __double_as_longlong(x);
    const int lo = walk_gbcast<G, O>((int)(v & 0xffffffffLL));
    const int hi = walk_gbcast<G, O>((int)(v >> 32));
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

// Solves X L^T = B for the 32 x 32 tile B in sX into global tile (i, j) (rows below n), if P is
// given into P, and if mbox is given into that mailbox tile (sweep_publish). Threads
// gt = 0 .. 32 G - 1 take part: lane (gt & 63) of wavefront gt >> 6 holds row
// (gt >> 6) * (64 / G) + (gt & 63) / G. STREAM (G = 4): the columns of L arrive four at a time
// from walk_factor_t<T, true> on another wavefront; before column p = 4b a wavefront that has
// not yet seen *prog >= pbase + 4b + 4 waits for it.
template <typename T, int G, bool STREAM>
__device__ __forceinline__ void walk_solve_grp(T* A, int n, int i, int j, const T (*sX)[kTile + 1],
                                               const T (*Lp)[kLtPitch], T (*P)[kLtPitch], int gt,
                                               const int* prog, int pbase, int* info,
                                               T* mbox = nullptr) {
    static_assert(!kRsqFactor<T>, "the division by L[p][p] is the IEEE quotient");
    static_assert(!STREAM || G == 4, "a streamed batch of four columns is one k");
    constexpr int K = kTile / G;
    constexpr int V = 16 / (int)sizeof(T);
    struct alignas(16) Q { T e[V]; };
    const int lane = gt & 63, g = lane & (G - 1);
    const int r = (gt >> 6) * (64 / G) + lane / G;
    T a[K], dv[K], yv[K];
#pragma unroll
    for (int k = 0; k < K; ++k) a[k] = sX[r][G * k + g];
    if constexpr (!STREAM) {
#pragma unroll
        for (int k = 0; k < K; ++k) dv[k] = Lp[G * k + g][g * K + k];
#pragma unroll
        for (int k = 0; k < K; ++k) yv[k] = rcp_rn(dv[k]);
    }
    T piv = a[0];  // on lane p mod G: column p, all earlier terms in
    int avail = 0;  // STREAM: columns of L seen to be out (a wait only when past them)
    static_for<0, kTile>([&](auto PI) __attribute__((always_inline)) {
        constexpr int p = decltype(PI)::value;
        constexpr int go = p % G, ko = p / G;
        if constexpr (STREAM && p % 4 == 0) {
            if (avail < p + 4) avail = lds_wait_ge(prog, pbase + p + 4, info) - pbase;
            dv[ko] = Lp[p + g][g * K + ko];
            yv[ko] = rcp_rn(dv[ko]);
        }
        const T x = div_rcp(piv, dv[ko], yv[ko]);
        const T xb = walk_gbcast<G, go>(x);
        T lc[K];
#pragma unroll
        for (int k0 = 0; k0 < K; k0 += V) {
            if (k0 + V > ko) {
                const Q q = *reinterpret_cast<const Q*>(&Lp[p][g * K + k0]);
#pragma unroll
                for (int e = 0; e < V; ++e) lc[k0 + e] = q.e[e];
            }
        }
        const T upd = num<T>::fma(-xb, lc[ko], a[ko]);
        a[ko] = g == go ? x : (g > go ? upd : a[ko]);
#pragma unroll
        for (int k = ko + 1; k < K; ++k) a[k] = num<T>::fma(-xb, lc[k], a[k]);
        if constexpr (go + 1 < G) piv = upd;
        else if constexpr (ko + 1 < K) piv = a[ko + 1];
    });
    if (i * kTile + r < n) {
        T* wp = A + (int64_t)(i * kTile + r) * n + j * kTile;
#pragma unroll
        for (int k = 0; k < K; ++k) wp[G * k + g] = a[k];
    }
    if (P) {
#pragma unroll
        for (int k = 0; k < K; ++k) P[r][G * k + g] = a[k];
    }
    if (mbox) {  // the tile, row-major, value by value
#pragma unroll
        for (int k = 0; k < K; ++k) sweep_publish(&mbox[r * kTile + G * k + g], a[k]);
    }
}

// Rows [R, R+16) of tile (i, j) for a 64-lane wavefront: lane l holds (R + (l >> 5) + 2q, l & 31).
template <typename T>
__device__ __forceinline__ void walk_load16(T (&v)[8], const T* A, int n, int i, int j, int R, int lane) {
    const int c = lane & (kTile - 1), rr = lane >> 5;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const int r = R + rr + 2 * q;
        v[q] = (i * kTile + r < n && j * kTile + c < n) ? A[(int64_t)(i * kTile + r) * n + j * kTile + c]
                                                          : (i == j && r == c ? T(1) : T(0));
    }
}

// sync: the layout above (dense_sync_flag_ints).
template <typename T>
__global__ void __launch_bounds__(kDfThreads) __attribute__((amdgpu_waves_per_eu(sizeof(T) == 4 ? 2 : 1))) k_potrf_walk(T* __restrict__ A, int n, int nt,
                                                           int ntasks, int* __restrict__ sync,
                                                           int* __restrict__ info) {
    __shared__ T sA[kTile][kTile + 1];
    __shared__ T sB[kTile][kTile + 1];
    __shared__ T sC[kTile][kTile + 1];
    __shared__ __align__(16) T sP[kTile][kLtPitch];  // walker: L[j][j-1], then L[j+1][j]
    __shared__ T sA2[kTile][kTile + 1];           // walker: the next diagonal partial sum
    __shared__ __align__(16) T sBw[kTile][kLtPitch];  // walker: tile (j+1, j-1), aligned rows
    __shared__ __align__(16) T sLt[kTile][kLtPitch];  // walker: L[j][j] transposed
    __shared__ T sInv[kTile];                         // f32: 1 / L[p][p] of the current tile
    __shared__ __align__(16) T sCol[2][kTile];        // walker factor: the published column
    __shared__ int s_task;
    __shared__ int s_prog, s_subready;  // walker: columns of L[j][j] out; sub-diagonal tiles in
    int* ticket = sync;
    int* flags = sync + 1;
    int* pdf = flags + nt * nt;
    int* psf = pdf + nt;
    T* dinv = reinterpret_cast<T*>(sync + dense_sync_flag_ints(nt));
    T* mb_diag = dense_mbox<T>(sync, nt);                       // L[g][g]
    T* mb_sub = mb_diag + (int64_t)nt * kTile * kTile;         // L[g+2][g]
    const int tid = threadIdx.x;
    const int c = tid & (kTile - 1), r0 = tid >> 5;
    if (tid == 0) {
        s_task = atomicAdd(ticket, 1);
        s_prog = 0;
        s_subready = 0;
    }
    __syncthreads();
    int t = __builtin_amdgcn_readfirstlane(s_task);
    if (t == 0) {
        // ---- the walker ----
        // Per step j: all waves add the k = j-1 term to the diagonal tile; wave 0 factors it
        // and publishes its columns four at a time as they are finished; waves 1 and 2 (rows
        // 0-15 and 16-31) prepare the sub-diagonal tile (j+1, j); then waves 2 and 3 solve it
        // against the published columns, four lanes per row, behind the factor, while wave 1
        // forms the next diagonal tile up to its k = j term (in the other buffer); wave 3
        // publishes the previous step's sub-diagonal tile meanwhile. The walker is the critical
        // path and shares its CU with the concurrent per-point kernels: its waves take issue
        // priority on their SIMDs.
        __builtin_amdgcn_s_setprio(3);
        const int w = tid >> 6, lane = tid & 63;
        T (*cur)[kTile + 1] = sA;
        T (*nxt)[kTile + 1] = sA2;
        {
            T v[4];
            walk_load(v, A, n, 0, 0, r0, c);
#pragma unroll
            for (int q = 0; q < 4; ++q) cur[r0 + 8 * q][c] = v[q];
        }
        __syncthreads();
        for (int j = 0; j < nt; ++j) {
            const bool sub = j + 1 < nt;
            // diagonal tile: partial sum (in cur) plus the k = j-1 term; thread (ra, cb) holds
            // rows 2ra, 2ra+1 and columns 2cb, 2cb+1, the rows of L[j][j-1] read four terms at a
            // time, every entry's chain in increasing p
            if (j >= 1) {
                constexpr int V = 16 / (int)sizeof(T);
                struct alignas(16) Q { T e[V]; };
                const int ra = tid >> 4, cb = tid & 15;
                T acc[2][2];
#pragma unroll
                for (int a = 0; a < 2; ++a)
#pragma unroll
                    for (int b = 0; b < 2; ++b) acc[a][b] = cur[2 * ra + a][2 * cb + b];
#pragma unroll
                for (int p0 = 0; p0 < kTile; p0 += V) {
                    Q x[2], y[2];
#pragma unroll
                    for (int a = 0; a < 2; ++a) x[a] = *reinterpret_cast<const Q*>(&sP[2 * ra + a][p0]);
#pragma unroll
                    for (int b = 0; b < 2; ++b) y[b] = *reinterpret_cast<const Q*>(&sP[2 * cb + b][p0]);
#pragma unroll
                    for (int u = 0; u < V; ++u)
#pragma unroll
                        for (int a = 0; a < 2; ++a)
#pragma unroll
                            for (int b = 0; b < 2; ++b)
                                acc[a][b] = num<T>::fma(-x[a].e[u], y[b].e[u], acc[a][b]);
                }
#pragma unroll
                for (int a = 0; a < 2; ++a)
#pragma unroll
                    for (int b = 0; b < 2; ++b) cur[2 * ra + a][2 * cb + b] = acc[a][b];
                __syncthreads();
            }
            if (w == 3 && j >= 1) {
                // the previous step's sub-diagonal tile (j, j-1), stored by waves 2 and 3 before
                // the step's barrier: published here, off the step's critical path
                __hip_atomic_store(&flags[j * nt + j - 1], 1, __ATOMIC_RELEASE,
                                   __HIP_MEMORY_SCOPE_AGENT);
            }
            if (w == 0) {
                // L[j][j] goes to the helpers through its mailbox tile (no flag, no release)
                walk_factor_t<T, true>(A, n, j, cur, sLt, sInv, dinv, sCol, tid, info, &s_prog,
                                       j * kTile, mb_diag + (int64_t)j * kTile * kTile);
            } else if (sub && w <= 2) {
                // sub-diagonal tile: partial sum over k < j-1 plus the k = j-1 term, into sC.
                // Lane (rb, cb) of wave w holds rows R + 4rb .. R + 4rb + 3, columns 2cb, 2cb + 1;
                // the rows of (j+1, j-1) come from a 16-byte-aligned copy, four terms per read,
                // every entry's chain in increasing p.
                const int R = 16 * (w - 1);
                // the partial sum is ready long before the tile (j+1, j-1): load it first
                if (lane == 0 && j >= 2) df_wait(&psf[j], info);
                constexpr int V = 16 / (int)sizeof(T);
                struct alignas(16) Q { T e[V]; };
                const int rb = lane >> 4, cb = lane & 15;
                const int row0 = R + 4 * rb, col0 = 2 * cb;
                T nx[4][2];
#pragma unroll
                for (int a = 0; a < 4; ++a)
#pragma unroll
                    for (int b = 0; b < 2; ++b) {
                        const int gr = (j + 1) * kTile + row0 + a;
                        nx[a][b] = gr < n ? A[(int64_t)gr * n + j * kTile + col0 + b] : T(0);
                    }
                if (j >= 1) {
                    // the helpers' L[j+1][j-1], read value by value from its mailbox tile
                    T lo[8];
                    {
                        const T* mt = mb_sub + (int64_t)(j - 1) * kTile * kTile;
                        int64_t idx[8];
                        bool live[8];
#pragma unroll
                        for (int q = 0; q < 8; ++q) {
                            const int r = R + (lane >> 5) + 2 * q;
                            idx[q] = r * kTile + (lane & 31);
                            live[q] = (j + 1) * kTile + r < n;
                        }
                        sweep_read_all<T, 8>(lo, mt, idx, live, info, 2);
                    }
#pragma unroll
                    for (int q = 0; q < 8; ++q) sBw[R + (lane >> 5) + 2 * q][lane & 31] = lo[q];
                    wave_sync_lds();
#pragma unroll
                    for (int p0 = 0; p0 < kTile; p0 += V) {
                        Q rv[4];
#pragma unroll
                        for (int a = 0; a < 4; ++a) rv[a] = *reinterpret_cast<const Q*>(&sBw[row0 + a][p0]);
                        T cv[2][V];
#pragma unroll
                        for (int b = 0; b < 2; ++b)
#pragma unroll
                            for (int u = 0; u < V; ++u) cv[b][u] = sP[col0 + b][p0 + u];
#pragma unroll
                        for (int u = 0; u < V; ++u)
#pragma unroll
                            for (int a = 0; a < 4; ++a)
#pragma unroll
                                for (int b = 0; b < 2; ++b)
                                    nx[a][b] = num<T>::fma(-rv[a].e[u], cv[b][u], nx[a][b]);
                    }
                }
#pragma unroll
                for (int a = 0; a < 4; ++a)
#pragma unroll
                    for (int b = 0; b < 2; ++b) sC[row0 + a][col0 + b] = nx[a][b];
                // sC (and the reads of sP above) before the solve starts: it overwrites sP
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
                if (lane == 0) atomicAdd(&s_subready, 1);
                if (w == 1) {
                    // next diagonal tile (j+1, j+1) into nxt: the helpers' partial sum over
                    // k < j-1, then the k = j-1 term from (j+1, j-1) (in sBw); lane (rb, cb)
                    // holds rows 4rb .. 4rb+3, columns 4cb .. 4cb+3, every entry's chain in
                    // increasing p
                    if (lane == 0 && j + 1 >= 2) df_wait(&pdf[j + 1], info);
                    const int rb4 = 4 * (lane >> 3), cb4 = 4 * (lane & 7);
                    const int t0 = (j + 1) * kTile;
                    T dg[4][4];
#pragma unroll
                    for (int a = 0; a < 4; ++a)
#pragma unroll
                        for (int b = 0; b < 4; ++b) {
                            const int gr = t0 + rb4 + a, gc = t0 + cb4 + b;
                            dg[a][b] = (gr < n && gc < n) ? A[(int64_t)gr * n + gc]
                                                          : (gr == gc ? T(1) : T(0));
                        }
                    if (j >= 1) {
                        lds_wait_ge(&s_subready, 2 * (j + 1), info);  // rows 16-31 from wave 2
#pragma unroll 1
                        for (int p0 = 0; p0 < kTile; p0 += V) {
                            Q rv[4], cq[4];
#pragma unroll
                            for (int a = 0; a < 4; ++a) rv[a] = *reinterpret_cast<const Q*>(&sBw[rb4 + a][p0]);
#pragma unroll
                            for (int b = 0; b < 4; ++b) cq[b] = *reinterpret_cast<const Q*>(&sBw[cb4 + b][p0]);
#pragma unroll
                            for (int u = 0; u < V; ++u)
#pragma unroll
                                for (int a = 0; a < 4; ++a)
#pragma unroll
                                    for (int b = 0; b < 4; ++b)
                                        dg[a][b] = num<T>::fma(-rv[a].e[u], cq[b].e[u], dg[a][b]);
                        }
                    }
#pragma unroll
                    for (int a = 0; a < 4; ++a)
#pragma unroll
                        for (int b = 0; b < 4; ++b) nxt[rb4 + a][cb4 + b] = dg[a][b];
                } else {
                    // rows 0-15 of the solve
                    lds_wait_ge(&s_subready, 2 * (j + 1), info);
                    walk_solve_grp<T, 4, true>(A, n, j + 1, j, sC, sLt, sP, tid - 128, &s_prog,
                                               j * kTile, info);
                }
            } else if (sub && w == 3) {
                // rows 16-31 of the solve (wave 3 publishes the tile in the next step)
                lds_wait_ge(&s_subready, 2 * (j + 1), info);
                walk_solve_grp<T, 4, true>(A, n, j + 1, j, sC, sLt, sP, tid - 128, &s_prog,
                                           j * kTile, info);
            }
            __syncthreads();
            T (*tmp)[kTile + 1] = cur;
            cur = nxt;
            nxt = tmp;
        }
        return;
    }
    // ---- helpers ----
    t -= 1;
    while (t < ntasks) {
        __syncthreads();
        int g = 0, rem = t;
        while (rem >= walk_group_tasks(g, nt)) { rem -= walk_group_tasks(g, nt); ++g; }
        const int nreg = std::max(0, nt - g - 2);
        T acc[4];
        if (rem < nreg) {
            // tile (i, g), i >= g+2: all terms, then the solve against L[g][g]
            const int i = g + 2 + rem;
            walk_load(acc, A, n, i, g, r0, c);
            walk_accumulate(acc, A, n, nt, i, g, 0, g, flags, info, sA, sB, tid, r0, c);
            // L[g][g] (a full tile: g < nt-2) from its mailbox, transposed into sLt in the order
            // of walk_perm<8>
            {
                T lv[4];
                int64_t idx[4];
                bool live[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int r = r0 + 8 * q;
                    idx[q] = r * kTile + c;
                    live[q] = c <= r;
                }
                sweep_read_all<T, 4>(lv, mb_diag + (int64_t)g * kTile * kTile, idx, live, info, 2);
                __syncthreads();  // the previous task's reads of sA and sLt are done
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int r = r0 + 8 * q;
                    sA[r][c] = acc[q];
                    sLt[c][walk_perm<8>(r)] = lv[q];
                }
            }
            __syncthreads();
            // the walker reads (g+2, g) for its sub-diagonal term from the mailbox
            walk_solve_grp<T, 8, false>(A, n, i, g, sA, sLt, (T(*)[kLtPitch])nullptr, tid, nullptr, 0,
                                        info, i == g + 2 ? mb_sub + (int64_t)g * kTile * kTile : nullptr);
            __syncthreads();
            if (tid == 0) {
                __hip_atomic_store(&flags[i * nt + g], 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
                s_task = atomicAdd(ticket, 1);
            }
        } else {
            // partial sums for the walker, d = g+2: of its tile (d, d) over k < g (the walker
            // adds k = g from the tile (d, g) it holds for its sub-diagonal tile), of (d+1, d)
            // over k < g+1
            const int d = g + 2;
            const bool diag = rem == nreg;
            const int i = diag ? d : d + 1;
            walk_load(acc, A, n, i, d, r0, c);
            walk_accumulate(acc, A, n, nt, i, d, 0, diag ? g : g + 1, flags, info, sA, sB, tid, r0,
                            c);
            // (the diagonal tile keeps its upper triangle, which no one reads)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int r = r0 + 8 * q;
                if (i * kTile + r < n && d * kTile + c < n && (!diag || c <= r))
                    A[(int64_t)(i * kTile + r) * n + d * kTile + c] = acc[q];
            }
            __syncthreads();
            if (tid == 0) {
                __hip_atomic_store(diag ? &pdf[d] : &psf[d], 1, __ATOMIC_RELEASE,
                                   __HIP_MEMORY_SCOPE_AGENT);
                s_task = atomicAdd(ticket, 1);
            }
        }
        __syncthreads();
        t = __builtin_amdgcn_readfirstlane(s_task) - 1;
    }
}

// ---- the same factor for large blocks: a few launches per tile column --------------------------
// In the persistent launches above every 32 x 32 tile re-reads two input tiles per 32 terms, so
// at a few thousand points the helpers' tile traffic and hand-offs, not arithmetic, set the
// time. For large blocks the matrix is instead swept in super-panels of 4 or 8 tile columns:
//   k_panel_step (one launch per tile column s of the super-panel): workgroup i - s takes tile
//     (i, s), adds the terms of the super-panel's earlier columns k in [32*s0, 32*s) from the
//     finished tiles (i, k) and (s, k); workgroup 0 then factors the diagonal tile (the walker
//     factor) and publishes it, and every other workgroup solves its tile against it (the walker
//     solve). Workgroup 0 is dispatched first and waits for nothing, so the others' waits end.
//   k_syrk_blk (one launch per super-panel): every 128 x 128 block of the trailing lower
//     triangle receives the super-panel's 128 or 256 terms, k increasing, in register
//     accumulators; the panel rows are staged in LDS a few columns at a time. A block takes one
//     workgroup about 60 us whatever the grid, so a trailing matrix of too few 128-blocks to
//     give every CU two is cut into 64 x 64 blocks instead (four times the workgroups, a
//     quarter of the work each; the terms and their order are the same).
// Entry (r, c) thus receives the terms of earlier super-panels through k_syrk_blk, then those of
// its own super-panel through k_panel_step, every one in increasing k: the unblocked chain, so
// the factor is bit-identical to the persistent launches' and to the oracle's.
// Tile columns per super-panel: 4 below kSuperWideMin points, 8 from there and 16 from twice
// that. Wider panels halve the trailing-update launches and double the terms per accumulator
// load (16384 points: 103 ms with 4, 94 with 8, 90 with 16), but lengthen the panel steps,
// which costs more at a few thousand points (4096: 4.3 ms with 4, 4.7 with 8).
constexpr int kSuper = 16;            // the widest super-panel
constexpr int kSuperWideMin = 8192;
constexpr int kBlockedMin = 2049;  // blocks of at least this many points take this path

template <typename T>
__global__ void __launch_bounds__(kDfThreads) k_panel_step(T* __restrict__ A, int n, int s,
                                                           int s0, int* __restrict__ flag,
                                                           int* __restrict__ info) {
    __shared__ T sA[kTile][kTile + 1];
    __shared__ T sB[kTile][kTile + 1];
    __shared__ __align__(16) T sLt[kTile][kLtPitch];
    __shared__ T sInv[kTile];
    __shared__ __align__(16) T sCol[2][kTile];
    const int tid = threadIdx.x;
    const int c = tid & (kTile - 1), r0 = tid >> 5;
    const int i = s + (int)blockIdx.x;
    const int i0 = i * kTile, s0r = s * kTile;
    T acc[4];
    walk_load(acc, A, n, i, s, r0, c);
    // the super-panel's finished columns (tiles k < s, all full: only the last tile column can
    // be partial), rows past n read as zero; all their loads are issued first, so the tiles
    // cost one round trip together, and the terms are then added tile by tile, k increasing
    T xa[kSuper - 1][4], xb[kSuper - 1][4];
#pragma unroll
    for (int u = 0; u < kSuper - 1; ++u) {
        if (s0 + u < s) {
            const int kk = (s0 + u) * kTile;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int r = r0 + 8 * q;
                xa[u][q] = i0 + r < n ? A[(int64_t)(i0 + r) * n + kk + c] : T(0);
                xb[u][q] = s0r + r < n ? A[(int64_t)(s0r + r) * n + kk + c] : T(0);
            }
        }
    }
#pragma unroll
    for (int u = 0; u < kSuper - 1; ++u) {
        if (s0 + u < s) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                sA[r0 + 8 * q][c] = xa[u][q];
                sB[r0 + 8 * q][c] = xb[u][q];
            }
            __syncthreads();
            walk_term(acc, sA, sB, r0, c);
            __syncthreads();
        }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) sA[r0 + 8 * q][c] = acc[q];
    __syncthreads();
    if (blockIdx.x == 0) {
        if (tid < 64) walk_factor_t(A, n, s, sA, sLt, sInv, (T*)nullptr, sCol, tid, info);
        __syncthreads();
        if (tid == 0) __hip_atomic_store(flag, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    if (tid == 0) df_wait(flag, info);
    __syncthreads();
    // L[s][s] transposed in the order of walk_perm<8>, zero above the diagonal (rows past n: the
    // identity's)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int r = r0 + 8 * q;
        T v = c <= r ? (s0r + r < n ? A[(int64_t)(s0r + r) * n + s0r + c] : T(r == c ? 1 : 0)) : T(0);
        sLt[c][walk_perm<8>(r)] = v;
    }
    __syncthreads();
    walk_solve_grp<T, 8, false>(A, n, i, s, sA, sLt, (T(*)[kLtPitch])nullptr, tid, nullptr, 0, info);
}

// A[r][c] = fma(-A[r][k], A[c][k], A[r][c]) for k = k0, ..., k0 + kd - 1 over the lower blocks of
// the trailing matrix (r, c >= t0), one BS x BS block per workgroup: thread (ty, tx) holds rows
// ty*TM .. ty*TM+TM-1 and columns tx*TM .. tx*TM+TM-1 of it (TM = BS/16). Diagonal blocks are
// computed whole; their upper part lies in the unused upper triangle of A.
template <typename T, int BS>
__global__ void __launch_bounds__(256) k_syrk_blk(T* __restrict__ A, int n, int t0, int k0,
                                                  int kd) {
    constexpr int TM = BS / 16;
    constexpr int Kc = sizeof(T) == 4 ? 32 : 16;  // panel columns per LDS round
    constexpr int P = BS + 4;                     // row pitch: 16-byte aligned rows
    __shared__ __align__(16) T sa[Kc][P];         // sa[k][r] = A[R0 + r][k0 + kc + k]
    __shared__ __align__(16) T sb[Kc][P];         // sb[k][c] = A[C0 + c][k0 + kc + k]
    const int L = (int)blockIdx.x;
    int I = (int)((__builtin_sqrt(8.0 * (double)L + 1.0) - 1.0) * 0.5);
    while ((I + 1) * (I + 2) / 2 <= L) ++I;
    while (I * (I + 1) / 2 > L) --I;
    const int J = L - I * (I + 1) / 2;
    const int R0 = t0 + I * BS, C0 = t0 + J * BS;
    const int tid = threadIdx.x, ty = tid >> 4, tx = tid & 15;
    T acc[TM][TM];
#pragma unroll
    for (int a = 0; a < TM; ++a) {
        const int r = R0 + ty * TM + a;
#pragma unroll
        for (int b = 0; b < TM; ++b) {
            const int cc = C0 + tx * TM + b;
            acc[a][b] = (r < n && cc < n) ? A[(int64_t)r * n + cc] : T(0);
        }
    }
    for (int kc = 0; kc < kd; kc += Kc) {
        __syncthreads();
        // rows of the two panels, Kc consecutive columns each (k fastest: coalesced)
        for (int e = tid; e < BS * Kc; e += 256) {
            const int r = e / Kc, k = e - r * Kc;
            const int64_t col = (int64_t)k0 + kc + k;
            sa[k][r] = R0 + r < n ? A[(int64_t)(R0 + r) * n + col] : T(0);
            sb[k][r] = C0 + r < n ? A[(int64_t)(C0 + r) * n + col] : T(0);
        }
        __syncthreads();
#pragma unroll 4
        for (int k = 0; k < Kc; ++k) {
            T x[TM], y[TM];
#pragma unroll
            for (int a = 0; a < TM; ++a) x[a] = sa[k][ty * TM + a];
#pragma unroll
            for (int b = 0; b < TM; ++b) y[b] = sb[k][tx * TM + b];
#pragma unroll
            for (int a = 0; a < TM; ++a)
#pragma unroll
                for (int b = 0; b < TM; ++b) acc[a][b] = num<T>::fma(-x[a], y[b], acc[a][b]);
        }
    }
#pragma unroll
    for (int a = 0; a < TM; ++a) {
        const int r = R0 + ty * TM + a;
#pragma unroll
        for (int b = 0; b < TM; ++b) {
            const int cc = C0 + tx * TM + b;
            if (r < n && cc < n) A[(int64_t)r * n + cc] = acc[a][b];
        }
    }
}

// Whether a block of n points takes the blocked path (GGP_POTRF_BLOCKED=1 / 0 forces it).
bool dense_blocked(int n) {
    if (const char* e = std::getenv("GGP_POTRF_BLOCKED")) return e[0] == '1';
    return n >= kBlockedMin;
}

template <typename T>
void dense_potrf_blocked(T* A, int n, int* info, int* flags, hipStream_t st) {
    const int nt = (n + kTile - 1) / kTile;
    const char* fs = std::getenv("GGP_POTRF_SUPER");  // "4" / "8" / "16" forces the width
    const int fw = fs ? std::atoi(fs) : 0;
    const int ks = (fw == 4 || fw == 8 || fw == 16)
                       ? fw
                       : (n >= 2 * kSuperWideMin ? 16 : n >= kSuperWideMin ? 8 : 4);
    int dev = 0, ncu = 256;
    if (hipGetDevice(&dev) == hipSuccess)
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
    for (int s0 = 0; s0 < nt; s0 += ks) {
        const int s1 = std::min(nt, s0 + ks);
        for (int s = s0; s < s1; ++s)
            hipLaunchKernelGGL((k_panel_step<T>), dim3(nt - s), dim3(kDfThreads), 0, st, A, n, s,
                               s0, flags + s, info);
        const int t0 = s1 * kTile;
        if (t0 < n) {
            const int mb = (n - t0 + 127) / 128;
            const char* force = std::getenv("GGP_SYRK_BLOCK");  // "64" / "128" forces the edge
            const bool big = force ? std::atoi(force) == 128 : mb * (mb + 1) / 2 >= 2 * ncu;
            if (big) {
                hipLaunchKernelGGL((k_syrk_blk<T, 128>), dim3(mb * (mb + 1) / 2), dim3(256), 0,
                                   st, A, n, t0, s0 * kTile, (s1 - s0) * kTile);
            } else {
                const int m64 = (n - t0 + 63) / 64;
                hipLaunchKernelGGL((k_syrk_blk<T, 64>), dim3(m64 * (m64 + 1) / 2), dim3(256), 0,
                                   st, A, n, t0, s0 * kTile, (s1 - s0) * kTile);
            }
        }
    }
}

int dense_sync_ints(int n) {
    const int nt = (n + kTile - 1) / kTile;
    // + the reciprocal diagonal and the walker's two mailboxes (<= f64)
    return dense_sync_flag_ints(nt) + 2 * nt * kTile + (int)(2 * dense_mbox_values(nt));
}

template <typename T>
static T pending_value() {
    T v;
    const auto b = Pending<T>::bits;
    static_assert(sizeof(b) == sizeof(T), "marker width");
    std::memcpy(&v, &b, sizeof(T));
    return v;
}

template <typename T>
void dense_potrf(T* A, int n, int* info, int* sync, int max_wg, hipStream_t st, bool zeroed) {
    if (n <= 0) return;
    const int nt = (n + kTile - 1) / kTile;
    if (!zeroed) {
        launch_fill<int>(sync, 0, dense_sync_flag_ints(nt), st);
        if (!dense_blocked(n))
            launch_fill<T>(dense_mbox<T>(sync, nt), pending_value<T>(), dense_mbox_values(nt), st);
    }
    if (dense_blocked(n)) {
        dense_potrf_blocked(A, n, info, sync + 1, st);  // flags: one per tile column
        return;
    }
    static const bool tiles = std::getenv("GGP_POTRF_TILES") != nullptr;
    if (tiles) {
        const int ntiles = nt * (nt + 1) / 2;
        const int nwg = std::max(1, std::min(ntiles, max_wg));
        hipLaunchKernelGGL((k_potrf_tiles<T>), dim3(nwg), dim3(kDfThreads), 0, st, A, n, nt, sync,
                           info);
        return;
    }
    int ntasks = 0;
    for (int g = 0; g < nt; ++g) ntasks += walk_group_tasks(g, nt);
    const int nwg = std::max(1, std::min(ntasks + 1, max_wg));
    hipLaunchKernelGGL((k_potrf_walk<T>), dim3(nwg), dim3(kDfThreads), 0, st, A, n, nt, ntasks,
                       sync, info);
}

// ---- triangular products and solves ---------------------------------------------------------
// Products with L and L^T. One workgroup per kTvRows outputs: all 256 threads stage the
// entries those outputs use (and x) in LDS with coalesced loads, kTvCols at a time; lane r then
// runs output r's fma chain from LDS in the serial order below. Every output keeps the chain of
// a row-by-row loop, so the result is that loop's, bit for bit. Acc is the accumulation type
// (T, or double for the f64 dense cotangents).
constexpr int kTvRows = 4, kTvCols = 1024, kTvLoads = kTvRows * kTvCols / 256;

template <typename A>
__device__ inline A fma_acc(A a, A b, A c) { return num<A>::fma(a, b, c); }

// acc chained over c in [c0, c1) of row r of the staged tile, 16 entries per batch (the batch's
// LDS reads are issued together; row starts are 16-byte aligned, so aligned batches vectorise).
template <typename T, typename Acc>
__device__ inline Acc tv_chain(const T* __restrict__ row, const T* __restrict__ sx, int c0, int c1,
                               Acc acc) {
    int c = c0;
    for (; c < c1 && (c & 3); ++c) acc = fma_acc<Acc>((Acc)row[c], (Acc)sx[c], acc);
    for (; c + 16 <= c1; c += 16) {
        T a[16], b[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) { a[u] = row[c + u]; b[u] = sx[c + u]; }
#pragma unroll
        for (int u = 0; u < 16; ++u) acc = fma_acc<Acc>((Acc)a[u], (Acc)b[u], acc);
    }
    for (; c < c1; ++c) acc = fma_acc<Acc>((Acc)row[c], (Acc)sx[c], acc);
    return acc;
}

// y = L x (src/dense.jl:118): row i accumulates j = 0..i.
template <typename T, typename Acc, typename Out>
__global__ void __launch_bounds__(256) k_trmv(const T* __restrict__ L, int n,
                                              const T* __restrict__ x, Out* __restrict__ y,
                                              Out* __restrict__ out, const int32_t* __restrict__ oidx) {
    constexpr int pitch = kTvCols + 16 / (int)sizeof(T);
    __shared__ __align__(16) T sL[kTvRows * pitch];
    __shared__ __align__(16) T sx[kTvCols];
    const int i0 = blockIdx.x * kTvRows, tid = threadIdx.x;
    const int nr = min(kTvRows, n - i0), jmax = i0 + nr;
    Acc acc = Acc(0);
    for (int j0 = 0; j0 < jmax; j0 += kTvCols) {
        const int w = min(kTvCols, jmax - j0);
        T t[kTvLoads];
        __syncthreads();
#pragma unroll
        for (int q = 0; q < kTvLoads; ++q) {
            const int e = q * 256 + tid, r = e / kTvCols, c = e % kTvCols;
            t[q] = (r < nr && c < w) ? L[(int64_t)(i0 + r) * n + j0 + c] : T(0);
        }
        for (int c = tid; c < w; c += 256) sx[c] = x[j0 + c];
#pragma unroll
        for (int q = 0; q < kTvLoads; ++q) {
            const int e = q * 256 + tid;
            sL[(e / kTvCols) * pitch + e % kTvCols] = t[q];
        }
        __syncthreads();
        if (tid < nr)
            acc = tv_chain<T, Acc>(sL + tid * pitch, sx, 0, min(i0 + tid + 1, j0 + w) - j0, acc);
    }
    if (tid < nr) {
        y[i0 + tid] = (Out)acc;
        if (out) out[oidx ? oidx[i0 + tid] : i0 + tid] = (Out)acc;  // null map: identity
    }
}
// y = L^T x (src/grad.jl:457, 493): entry i accumulates j = i..n-1.
template <typename T, typename Acc, typename Out>
__global__ void __launch_bounds__(256) k_trmv_t(const T* __restrict__ L, int n,
                                                const T* __restrict__ x, Out* __restrict__ y,
                                                Out* __restrict__ out, const int32_t* __restrict__ oidx) {
    constexpr int pitch = kTvCols + 16 / (int)sizeof(T);
    __shared__ __align__(16) T sL[kTvRows * pitch];
    __shared__ __align__(16) T sx[kTvCols];
    const int i0 = blockIdx.x * kTvRows, tid = threadIdx.x;
    const int nr = min(kTvRows, n - i0);
    Acc acc = Acc(0);
    for (int j0 = i0; j0 < n; j0 += kTvCols) {
        const int w = min(kTvCols, n - j0);
        T t[kTvLoads];
        __syncthreads();
#pragma unroll
        for (int q = 0; q < kTvLoads; ++q) {
            const int e = q * 256 + tid, c = e / kTvRows, r = e % kTvRows;
            t[q] = (r < nr && c < w) ? L[(int64_t)(j0 + c) * n + i0 + r] : T(0);
        }
        for (int c = tid; c < w; c += 256) sx[c] = x[j0 + c];
#pragma unroll
        for (int q = 0; q < kTvLoads; ++q) {
            const int e = q * 256 + tid;
            sL[(e % kTvRows) * pitch + e / kTvRows] = t[q];
        }
        __syncthreads();
        if (tid < nr)
            acc = tv_chain<T, Acc>(sL + tid * pitch, sx, max(i0 + tid - j0, 0), w, acc);
    }
    if (tid < nr) {
        y[i0 + tid] = (Out)acc;
        if (out) out[oidx ? oidx[i0 + tid] : i0 + tid] = (Out)acc;  // null map: identity
    }
}

// x = L \ b (src/dense.jl:134) and x = L^T \ b (src/dense.jl:236): the row-by-row
// substitutions, each row's fma chain in the serial order (the earlier unknowns in increasing
// index for L, decreasing blocks of 32 for L^T), then its division. One wavefront per 32-row
// block; blocks are taken from a ticket counter in the order of the substitution (forward
// for L, backward for L^T), so a block waits only for blocks taken earlier by running
// wavefronts and the launch cannot deadlock. A block folds in each earlier block's unknowns as
// soon as they are published (release / acquire of a per-block flag), so only the last block's
// terms and the block's own 32-step solve stay on the chain from block to block. Every wait is
// bounded (bit 1 of *info when exceeded). sync = [ticket, flags[nt]], zeroed by the caller.
template <typename T, bool TRANS>
__global__ void __launch_bounds__(64) k_trsv_mw(const T* __restrict__ L, int n, int nt,
                                                const T* __restrict__ b, T* __restrict__ x,
                                                int* __restrict__ sync, int* __restrict__ info) {
    int* ticket = sync;
    int* flags = sync + 1;
    const int lane = threadIdx.x;
    // Every lane runs the ticket, wait and publish steps (uniform control flow: with a
    // lane-0-only branch around them the compiler may let the other lanes run ahead into the
    // next block on a stale ticket). Only lane 0 adds to the ticket; every lane polls the flag
    // (one request per wavefront) and stores the same flag value.
    while (true) {
        const int t = __builtin_amdgcn_readfirstlane(atomicAdd(ticket, lane == 0 ? 1 : 0));
        if (t >= nt) break;
        const int blk = TRANS ? nt - 1 - t : t;
        const int i0 = blk * kTile, ni = min(kTile, n - i0);
        const bool live = lane < ni;
        T v = live ? b[i0 + lane] : T(0);
        for (int q = 0; q < t; ++q) {
            const int kb = TRANS ? nt - 1 - q : q;
            const int k0 = kb * kTile, nk = min(kTile, n - k0);
            df_wait_uniform(&flags[kb], info);
            T xk[kTile], lr[kTile];
#pragma unroll
            for (int p = 0; p < kTile; ++p) {
                xk[p] = p < nk ? x[k0 + p] : T(0);
                lr[p] = (live && p < nk) ? (TRANS ? L[(int64_t)(k0 + p) * n + i0 + lane]
                                                  : L[(int64_t)(i0 + lane) * n + k0 + p])
                                         : T(0);
            }
#pragma unroll
            for (int p = 0; p < kTile; ++p)
                if (p < nk) v = num<T>::fma(-lr[p], xk[p], v);
        }
        // the block's own unknowns, by broadcasts (same chains as the serial substitution)
        if (!TRANS) {
            for (int jj = 0; jj < ni; ++jj) {
                const T xj = bcast(v, jj) / L[(int64_t)(i0 + jj) * n + i0 + jj];
                if (lane == jj) v = xj;
                else if (lane > jj && lane < ni)
                    v = num<T>::fma(-L[(int64_t)(i0 + lane) * n + i0 + jj], xj, v);
            }
        } else {
            for (int jj = ni - 1; jj >= 0; --jj) {
                const T xj = bcast(v, jj) / L[(int64_t)(i0 + jj) * n + i0 + jj];
                if (lane == jj) v = xj;
                else if (lane < jj) v = num<T>::fma(-L[(int64_t)(i0 + jj) * n + i0 + lane], xj, v);
            }
        }
        if (live) x[i0 + lane] = v;
        __hip_atomic_store(&flags[blk], 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// out = sum_i log L[i][i] (src/dense.jl:146), accumulated in double.
template <typename T>
__global__ void k_logdiag(const T* __restrict__ L, int n, double* __restrict__ out) {
    __shared__ double s[256];
    double t = 0.0;
    for (int i = threadIdx.x; i < n; i += blockDim.x) t += (double)num<T>::log(L[(int64_t)i * n + i]);
    s[threadIdx.x] = t;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) s[threadIdx.x] += s[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) out[0] = s[0];
}

template <typename T>
void dense_trmv(const T* L, int n, const T* x, T* y, hipStream_t st, T* out, const int32_t* oidx) {
    hipLaunchKernelGGL((k_trmv<T, T, T>), dim3(cdiv(n, kTvRows)), dim3(256), 0, st, L, n, x, y,
                       out, oidx);
}
template <typename T>
void dense_trmv_t(const T* L, int n, const T* x, T* y, hipStream_t st, T* out,
                  const int32_t* oidx) {
    hipLaunchKernelGGL((k_trmv_t<T, T, T>), dim3(cdiv(n, kTvRows)), dim3(256), 0, st, L, n, x, y,
                       out, oidx);
}
template <typename T, bool TRANS>
static void trsv_mw(const T* L, int n, const T* b, T* x, int* sync, int* info, hipStream_t st) {
    if (n <= 0) return;
    const int nt = (n + kTile - 1) / kTile;
    launch_fill<int>(sync, 0, nt + 1, st);
    hipLaunchKernelGGL((k_trsv_mw<T, TRANS>), dim3(std::min(nt, 1024)), dim3(64), 0, st, L, n, nt,
                       b, x, sync, info);
}
template <typename T>
void dense_trsv(const T* L, int n, const T* b, T* x, int* sync, int* info, hipStream_t st) {
    trsv_mw<T, false>(L, n, b, x, sync, info, st);
}
template <typename T>
void dense_trsv_t(const T* L, int n, const T* b, T* x, int* sync, int* info, hipStream_t st) {
    trsv_mw<T, true>(L, n, b, x, sync, info, st);
}
template <typename T>
void dense_logdiag(const T* L, int n, double* out, hipStream_t st) {
    hipLaunchKernelGGL((k_logdiag<T>), dim3(1), dim3(256), 0, st, L, n, out);
}

template <typename T>
void dense_assemble(const Graph& g, const Table<T>& tb, T* A, T diag_add, hipStream_t st,
                    int* zero_info, int* zero_sync) {
    const int nt0 = (int)cdiv((int)g.n0, kTile);
    const int nz1 = zero_sync ? dense_sync_flag_ints(nt0) : 0;
    // the walker's mailboxes (the blocked factor has none)
    T* mb = zero_sync && !dense_blocked((int)g.n0) ? dense_mbox<T>(zero_sync, nt0) : nullptr;
    const int64_t nmb = mb ? dense_mbox_values(nt0) : 0;
    const T mbv = pending_value<T>();
    const int n = (int)g.n0;
    const dim3 grid(cdiv(n, 16), cdiv(n, 16)), blk(16, 16);
    const T scale = (T)g.scale;
    const bool an = tb.aniso.grid != nullptr;
#define GGP_ASM(DD)                                                                             \
    do {                                                                                        \
        if (an) hipLaunchKernelGGL((k_dense_assemble<T, DD, true>), grid, blk, tb.aniso.lds, st, A, g.coords, n, scale, tb.tab, tb.acc, tb.params, diag_add, tb.aniso, zero_info, zero_info ? 1 : 0, zero_sync, nz1, mb, nmb, mbv); \
        else hipLaunchKernelGGL((k_dense_assemble<T, DD, false>), grid, blk, 0, st, A, g.coords, n, scale, tb.tab, tb.acc, tb.params, diag_add, tb.aniso, zero_info, zero_info ? 1 : 0, zero_sync, nz1, mb, nmb, mbv); \
    } while (0)
    switch (g.D) {
        case 2: GGP_ASM(2); break;
        case 3: GGP_ASM(3); break;
        case 4: GGP_ASM(4); break;
        default: break;
    }
#undef GGP_ASM
}

// ---- dense cotangents (f64) -----------------------------------------------------------------
// ---- f64 matrix-core GEMM ---------------------------------------------------------------------
// C = alpha * op(A) * B for a batch of independent jobs, on v_mfma_f64_16x16x4f64. Each
// workgroup owns a TM x TM tile of one job's C (TM = 64, or 32 for batches with too few 64-tiles
// to fill the chip); its four wavefronts own TM/2 x TM/2 quarters (2 x 2 or 1 x 1 MFMA blocks).
// k advances in 32-deep chunks staged in LDS, the next chunk prefetched into registers while the
// current one is multiplied. Operand layout of the instruction: A[i][k] in lane i + 16k, B[k][j]
// in lane j + 16k; D[i][j] in lane j + 16(i mod 4), element i / 4.
//
// Triangular operands: flags restrict k to the part that can be non-zero for the tile
// (GK_FROM_I: k >= i0, GK_FROM_J: k >= j0, GK_TO_I: k < i0 + TM); entries the flags skip are zero
// in the operand, so the product is unchanged. GK_LOWER skips tiles strictly above the diagonal.
typedef double f64x4 __attribute__((ext_vector_type(4)));
constexpr int kGK = 32, kGemmJobs = 24;
enum GemmFlags { GK_FROM_I = 1, GK_FROM_J = 2, GK_TO_I = 4, GK_LOWER = 8 };
struct GemmJob {
    const void* A;
    const double* B;
    double* C;
    int lda, ldb, ldc;
    int M, N, K;
    int atrans;  // op(A)(i, k) = A[k*lda + i] when set, A[i*lda + k] otherwise
    int flags;
    int tiles_n, tile0;
    double alpha;
};
struct GemmBatch {
    GemmJob job[kGemmJobs];
    int njobs;
};

template <typename TA, int TM>
__global__ void __launch_bounds__(256) k_gemm64(GemmBatch batch) {
    constexpr int WQ = TM / 2, NB = WQ / 16, NF = TM * kGK / 256;
    __shared__ double sA[kGK][TM + 2];
    __shared__ double sB[kGK][TM + 2];
    int jb = 0;
    while (jb + 1 < batch.njobs && batch.job[jb + 1].tile0 <= (int)blockIdx.x) ++jb;
    const GemmJob& g = batch.job[jb];
    const int t = (int)blockIdx.x - g.tile0;
    const int i0 = (t / g.tiles_n) * TM, j0 = (t % g.tiles_n) * TM;
    if ((g.flags & GK_LOWER) && j0 > i0) return;
    int ks = 0, ke = g.K;
    if (g.flags & GK_FROM_I) ks = max(ks, i0);
    if (g.flags & GK_FROM_J) ks = max(ks, j0);
    if (g.flags & GK_TO_I) ke = min(ke, i0 + TM);
    ks = (ks / kGK) * kGK;
    const TA* __restrict__ A = static_cast<const TA*>(g.A);
    const double* __restrict__ B = g.B;
    const int tid = threadIdx.x, l = tid & 63, w = tid >> 6;
    const int wr = (w >> 1) * WQ, wc = (w & 1) * WQ;
    f64x4 acc[NB][NB];
#pragma unroll
    for (int a = 0; a < NB; ++a)
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[a][b] = (f64x4){0.0, 0.0, 0.0, 0.0};
    // register staging of one chunk: NF A and NF B entries per thread
    double ra[NF], rb[NF];
    auto fetch = [&](int k0) {
#pragma unroll
        for (int q = 0; q < NF; ++q) {
            const int e = tid + 256 * q;
            int ii, kk;
            if (g.atrans) { kk = e / TM; ii = e % TM; } else { ii = e / kGK; kk = e % kGK; }
            const int gi = i0 + ii, gk = k0 + kk;
            ra[q] = (gi < g.M && gk < ke)
                        ? (double)(g.atrans ? A[(int64_t)gk * g.lda + gi] : A[(int64_t)gi * g.lda + gk])
                        : 0.0;
            const int kb = e / TM, jj = e % TM;
            const int gj = j0 + jj, gkb = k0 + kb;
            rb[q] = (gj < g.N && gkb < ke) ? B[(int64_t)gkb * g.ldb + gj] : 0.0;
        }
    };
    auto stash = [&]() {
#pragma unroll
        for (int q = 0; q < NF; ++q) {
            const int e = tid + 256 * q;
            int ii, kk;
            if (g.atrans) { kk = e / TM; ii = e % TM; } else { ii = e / kGK; kk = e % kGK; }
            sA[kk][ii] = ra[q];
            sB[e / TM][e % TM] = rb[q];
        }
    };
    if (ks < ke) fetch(ks);
    for (int k0 = ks; k0 < ke; k0 += kGK) {
        __syncthreads();
        stash();
        __syncthreads();
        if (k0 + kGK < ke) fetch(k0 + kGK);
#pragma unroll
        for (int s = 0; s < kGK / 4; ++s) {
            const int kr = s * 4 + (l >> 4);
            double av[NB], bv[NB];
#pragma unroll
            for (int a = 0; a < NB; ++a) av[a] = sA[kr][wr + 16 * a + (l & 15)];
#pragma unroll
            for (int b = 0; b < NB; ++b) bv[b] = sB[kr][wc + 16 * b + (l & 15)];
#pragma unroll
            for (int a = 0; a < NB; ++a)
#pragma unroll
                for (int b = 0; b < NB; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f64_16x16x4f64(av[a], bv[b], acc[a][b], 0, 0, 0);
        }
    }
#pragma unroll
    for (int a = 0; a < NB; ++a)
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int i = i0 + wr + 16 * a + (l >> 4) + 4 * v;
                const int j = j0 + wc + 16 * b + (l & 15);
                if (i < g.M && j < g.N) g.C[(int64_t)i * g.ldc + j] = g.alpha * acc[a][b][v];
            }
}

// Launch a list of jobs (split into batches of kGemmJobs). A batch whose 64 x 64 tiles would
// give fewer than kGemmFill workgroups runs on 32 x 32 tiles (4x the workgroups).
constexpr int kGemmFill = 512;
template <typename TA>
static void launch_gemm(std::vector<GemmJob> jobs, hipStream_t st) {
    for (size_t s = 0; s < jobs.size(); s += kGemmJobs) {
        const int nj = (int)std::min<size_t>(kGemmJobs, jobs.size() - s);
        int t64 = 0;
        for (int q = 0; q < nj; ++q)
            t64 += (int)(cdiv(jobs[s + q].M, 64) * cdiv(jobs[s + q].N, 64));
        const int tm = t64 < kGemmFill ? 32 : 64;
        GemmBatch b{};
        int tiles = 0;
        b.njobs = nj;
        for (int q = 0; q < nj; ++q) {
            GemmJob j = jobs[s + q];
            j.tiles_n = (j.N + tm - 1) / tm;
            j.tile0 = tiles;
            tiles += ((j.M + tm - 1) / tm) * j.tiles_n;
            b.job[q] = j;
        }
        if (tiles <= 0) continue;
        if (tm == 32) hipLaunchKernelGGL((k_gemm64<TA, 32>), dim3(tiles), dim3(256), 0, st, b);
        else hipLaunchKernelGGL((k_gemm64<TA, 64>), dim3(tiles), dim3(256), 0, st, b);
    }
}

static GemmJob gemm_job(const void* A, int lda, int atrans, const double* B, int ldb, double* C,
                        int ldc, int M, int N, int K, int flags, double alpha) {
    GemmJob j{};
    j.A = A; j.lda = lda; j.atrans = atrans;
    j.B = B; j.ldb = ldb;
    j.C = C; j.ldc = ldc;
    j.M = M; j.N = N; j.K = K;
    j.flags = flags;
    j.alpha = alpha;
    return j;
}

// ---- W = L^-1 (f64) ---------------------------------------------------------------------------
// Diagonal 32x32 blocks are inverted directly (one column per lane, forward substitution); then
// the off-diagonal blocks follow from the 2x2 block identity
//   [A 0; B C]^-1 = [A^-1 0; -C^-1 B A^-1  C^-1],
// applied recursively (splits on 32-row boundaries): every recursion level is one batched GEMM
// T = B A^-1 followed by one batched GEMM X = -C^-1 T, the nodes of a level being independent.
template <typename T>
__global__ void __launch_bounds__(64) k_trinv_leaf(const T* __restrict__ L, int n,
                                                   double* __restrict__ W) {
    __shared__ double sL[32][33];
    const int o = blockIdx.x * 32, tid = threadIdx.x;
    const int nb = min(32, n - o);
    for (int e = tid; e < 32 * 32; e += 64) {
        const int r = e / 32, c = e % 32;
        sL[r][c] = (r < nb && c <= r) ? (double)L[(int64_t)(o + r) * n + o + c] : (r == c ? 1.0 : 0.0);
    }
    __syncthreads();
    if (tid >= 32) return;
    const int c = tid;
    double w[32];
#pragma unroll
    for (int r = 0; r < 32; ++r) {
        double s = r == c ? 1.0 : 0.0;
#pragma unroll
        for (int k = 0; k < r; ++k) s = __builtin_fma(-sL[r][k], w[k], s);
        w[r] = r >= c ? s / sL[r][r] : 0.0;
    }
    if (c < nb)
#pragma unroll
        for (int r = 0; r < 32; ++r)
            if (r < nb) W[(int64_t)(o + r) * n + o + c] = w[r];
}

// Recursion plan: jobs[depth] = {first GEMMs, second GEMMs} of the nodes at that depth.
template <typename T>
static void trinv_plan(const T* L, double* W, double* S, int n, int o, int sz, int depth,
                       std::vector<std::vector<GemmJob>>& g1, std::vector<std::vector<GemmJob>>& g2) {
    if (sz <= 32) return;
    const int nb = (sz + 31) / 32;
    const int m = 32 * ((nb + 1) / 2), s2 = sz - m;
    trinv_plan(L, W, S, n, o, m, depth + 1, g1, g2);
    trinv_plan(L, W, S, n, o + m, s2, depth + 1, g1, g2);
    if ((int)g1.size() <= depth) { g1.resize(depth + 1); g2.resize(depth + 1); }
    const int64_t off = (int64_t)(o + m) * n + o;
    // T = B A^-1: B = L[o+m.., o..] (s2 x m), A^-1 = W[o.., o..] lower (k >= column)
    g1[depth].push_back(gemm_job(L + off, n, 0, W + (int64_t)o * n + o, n, S + off, n, s2, m, m,
                                 GK_FROM_J, 1.0));
    // X = -C^-1 T: C^-1 = W[o+m.., o+m..] lower (k <= row)
    g2[depth].push_back(gemm_job(W + (int64_t)(o + m) * n + o + m, n, 0, S + off, n, W + off, n,
                                 s2, m, s2, GK_TO_I, -1.0));
}

template <typename T>
static void dense_inverse64(const T* L, int n, double* W, double* S, hipStream_t st) {
    launch_fill<double>(W, 0.0, (int64_t)n * n, st);
    hipLaunchKernelGGL((k_trinv_leaf<T>), dim3(cdiv(n, 32)), dim3(64), 0, st, L, n, W);
    std::vector<std::vector<GemmJob>> g1, g2;
    trinv_plan<T>(L, W, S, n, 0, n, 0, g1, g2);
    for (int d = (int)g1.size() - 1; d >= 0; --d) {
        launch_gemm<T>(g1[d], st);
        launch_gemm<double>(g2[d], st);
    }
}

// Q[a][j] = u[a] (h_j(a) + xi[a] W[a][j] / 2), h_j(a) = sum_{b<a} xi[b] W[b][j] (W is lower
// triangular, so rows above j add zeros). Workgroup = 32 columns x 8 row chunks: chunk sums,
// an exclusive prefix over the chunks in LDS, then the running sum within each chunk.
template <typename T>
__global__ void __launch_bounds__(256) k_qprefix(const double* __restrict__ W, int n,
                                                 const T* __restrict__ xi,
                                                 const double* __restrict__ u,
                                                 double* __restrict__ Q) {
    __shared__ double part[8][33];
    const int jl = threadIdx.x % 32, ck = threadIdx.x / 32;
    const int j = blockIdx.x * 32 + jl;
    const int clen = (n + 7) / 8;
    const int a_lo = ck * clen, a_hi = min(n, a_lo + clen);
    double s = 0.0;
    if (j < n)
#pragma unroll 8
        for (int a = a_lo; a < a_hi; ++a) s += W[(int64_t)a * n + j] * (double)xi[a];
    part[ck][jl] = s;
    __syncthreads();
    double h = 0.0;
    for (int q = 0; q < ck; ++q) h += part[q][jl];
    if (j >= n) return;
#pragma unroll 8
    for (int a = a_lo; a < a_hi; ++a) {
        const double w = W[(int64_t)a * n + j] * (double)xi[a];
        Q[(int64_t)a * n + j] = u[a] * (h + 0.5 * w);
        h += w;
    }
}

enum DenseMode { DM_LOGDET = 0, DM_GENERATE = 1, DM_INVLOSS = 2 };

// Scatter the dense covariance cotangent through the lookup weights (src/dense.jl:166-181,
// 244-252; src/grad_generate_vals.jl:196-211). Pairs (a >= b) of the lower triangle are split
// over the grid; each workgroup accumulates an f64 LDS histogram and writes it to its row of
// hist_partial. HG (a table too large for LDS): the workgroup accumulates with f64 atomics
// directly in its row, which the host zeroes before the launch.
template <typename T, int D, int MODE, bool HG>
__global__ void __launch_bounds__(256) k_dense_scatter(const uint32_t* __restrict__ coords,
                                                       int n, T scale,
                                                       const TabEnt<T>* __restrict__ tab,
                                                       const uint16_t* __restrict__ acc,
                                                       const TabParams<T>* __restrict__ Pp,
                                                       const double* __restrict__ C,
                                                       const T* __restrict__ alpha,
                                                       double* __restrict__ hist_partial) {
    const TabParams<T> P = *Pp;
    extern __shared__ double s_lds_hist[];
    double* s_hist = HG ? hist_partial + (size_t)blockIdx.x * P.nb : s_lds_hist;
    if (!HG) {
        for (int i = threadIdx.x; i < P.nb; i += blockDim.x) s_hist[i] = 0.0;
        __syncthreads();
    }
    const int64_t npairs = (int64_t)n * (n + 1) / 2;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < npairs; t += stride) {
        int64_t a = (int64_t)((sqrt(8.0 * (double)t + 1.0) - 1.0) * 0.5);
        while ((a + 1) * (a + 2) / 2 <= t) ++a;
        while (a * (a + 1) / 2 > t) --a;
        const int64_t b = t - a * (a + 1) / 2;
        double gv;
        if (MODE == DM_LOGDET) {
            const double kinv = C[a * n + b];
            gv = a == b ? 0.5 * kinv : kinv;
        } else if (MODE == DM_GENERATE) {
            gv = a == b ? C[a * n + a] : C[a * n + b] + C[b * n + a];
        } else {
            const double aa = (double)alpha[a], ab = (double)alpha[b];
            gv = a == b ? -0.5 * aa * aa : -aa * ab;
        }
        if (a == b) {
            atomicAdd(&s_hist[0], gv);
            continue;
        }
        uint32_t ca[D], cb[D];
#pragma unroll
        for (int d = 0; d < D; ++d) { ca[d] = coords[a * D + d]; cb[d] = coords[b * D + d]; }
        const T r = radius<T>(sqdist<D>(ca, cb), scale);
        T wlo, whi;
        const int lo = cov_weights(r, tab, acc, P, wlo, whi);
        atomicAdd(&s_hist[lo], gv * (double)wlo);
        atomicAdd(&s_hist[lo + 1], gv * (double)whi);
    }
    if (!HG) {
        __syncthreads();
        double* out = hist_partial + (size_t)blockIdx.x * P.nb;
        for (int i = threadIdx.x; i < P.nb; i += blockDim.x) out[i] = s_hist[i];
    }
}

template <typename T>
size_t dense_scatter_lds(const Table<T>& tb) {
    return tb.global ? 0 : (size_t)tb.P.nb * sizeof(double);
}

template <typename T, int MODE>
static void launch_dense_scatter(const Graph& g, const Table<T>& tb, const double* C,
                                 const T* alpha, double* hist_partial, int nw, hipStream_t st) {
    const size_t lds = dense_scatter_lds(tb);
    const int n = (int)g.n0;
    const T scale = (T)g.scale;
    if (tb.global) launch_fill<double>(hist_partial, 0.0, (int64_t)nw * tb.P.nb, st);
#define GGP_SCAT(DD, HG)                                                                       \
    hipLaunchKernelGGL((k_dense_scatter<T, DD, MODE, HG>), dim3(nw), dim3(256), lds, st,        \
                       g.coords, n, scale, tb.tab, tb.acc, tb.params, C, alpha, hist_partial)
#define GGP_SCAT_D(DD)                                                                         \
    do {                                                                                       \
        if (tb.global) GGP_SCAT(DD, true);                                                     \
        else GGP_SCAT(DD, false);                                                              \
    } while (0)
    switch (g.D) {
        case 2: GGP_SCAT_D(2); break;
        case 3: GGP_SCAT_D(3); break;
        case 4: GGP_SCAT_D(4); break;
        default: break;
    }
#undef GGP_SCAT_D
#undef GGP_SCAT
}


// d(sum log diag L)/dvals: Kinv = W^T W, diagonal halved (src/dense.jl:153-183).
template <typename T>
void dense_grad_logdet(const Graph& g, const Table<T>& tb, const T* L, double* W, double* C,
                       double* hist_partial, int nw, hipStream_t st) {
    const int n = (int)g.n0;
    dense_inverse64(L, n, W, C, st);  // C is the inversion's scratch, then K^-1 (lower)
    launch_gemm<double>({gemm_job(W, n, 1, W, n, C, n, n, n, n, GK_FROM_I | GK_FROM_J | GK_LOWER, 1.0)}, st);
    launch_dense_scatter<T, DM_LOGDET>(g, tb, C, nullptr, hist_partial, nw, st);
}

// d<vb, L xi>/dvals through the Cholesky adjoint with Lbar = tril(vb xi^T)
// (src/grad_generate_vals.jl:188-211): S = W^T P W with P = Phi(L^T Lbar), P[a][b] = u[a]xi[b]
// (a > b), u[a]xi[a]/2 (a = b), u = L^T vb; Abar[i][j] = S[i][j] + S[j][i], Abar[j][j] = S[j][j].
template <typename T>
void dense_inverse(const T* L, int n, double* W, double* S, hipStream_t st) {
    dense_inverse64(L, n, W, S, st);
}

template <typename T>
void dense_grad_generate(const Graph& g, const Table<T>& tb, const T* L, const T* vb,
                         const T* xi, double* W, double* C, double* Q, double* u,
                         double* hist_partial, int nw, bool inverse_ready, hipStream_t st) {
    const int n = (int)g.n0;
    if (!inverse_ready) dense_inverse64(L, n, W, C, st);
    // u = L^T vb in double (rows i >= a, increasing i)
    hipLaunchKernelGGL((k_trmv_t<T, double, double>), dim3(cdiv(n, kTvRows)), dim3(256), 0, st, L,
                       n, vb, u, (double*)nullptr, (const int32_t*)nullptr);
    hipLaunchKernelGGL((k_qprefix<T>), dim3(cdiv(n, 32)), dim3(256), 0, st, W, n, xi, u, Q);
    launch_gemm<double>({gemm_job(W, n, 1, Q, n, C, n, n, n, n, GK_FROM_I | GK_FROM_J, 1.0)}, st);
    launch_dense_scatter<T, DM_GENERATE>(g, tb, C, nullptr, hist_partial, nw, st);
}

// d(0.5 y^T K^-1 y)/dvals: -alpha_a alpha_b, diagonal -alpha_a^2/2 (src/dense.jl:244-252).
template <typename T>
void dense_grad_invloss(const Graph& g, const Table<T>& tb, const T* alpha, double* hist_partial,
                        int nw, hipStream_t st) {
    launch_dense_scatter<T, DM_INVLOSS>(g, tb, nullptr, alpha, hist_partial, nw, st);
}

// ---- d/dpoints of the dense layer (src/dense.jl:185-222, 268-300) -----------------------------
// One workgroup per point p sums, over every other point q, the pair cotangent G[p][q] through
// k'(r) dr/dx_p. The reference visits each pair (a > b) once and adds c to a and -c to b; the
// term p receives from (p, q) is the same c (or its exact negation) evaluated from p's side, so
// each row is a plain sum and dpd (n x D) is written without atomics.
// G = K^-1 (C, full symmetric) for the logdet; G = -alpha_p alpha_q for the inverse loss.
template <typename T, int D, int MODE>
__global__ void __launch_bounds__(256) k_dense_pts(const uint32_t* __restrict__ coords, int n,
                                                   T scale, const TabEnt<T>* __restrict__ tab,
                                                   const uint16_t* __restrict__ acc,
                                                   const TabParams<T>* __restrict__ Pp,
                                                   const double* __restrict__ C,
                                                   const T* __restrict__ alpha,
                                                   double* __restrict__ dpd) {
    const TabParams<T> P = *Pp;
    __shared__ double s_red[4][D];
    const int p = blockIdx.x;
    uint32_t cp[D];
#pragma unroll
    for (int d = 0; d < D; ++d) cp[d] = coords[(int64_t)p * D + d];
    const T ap = MODE == DM_INVLOSS ? alpha[p] : T(0);
    double g[D];
#pragma unroll
    for (int d = 0; d < D; ++d) g[d] = 0.0;
    for (int q = threadIdx.x; q < n; q += blockDim.x) {
        if (q == p) continue;
        uint32_t cq[D];
#pragma unroll
        for (int d = 0; d < D; ++d) cq[d] = coords[(int64_t)q * D + d];
        const T gv = MODE == DM_LOGDET ? (T)C[(int64_t)p * n + q] : -ap * alpha[q];
        T c[D];
        if (pair_pts<T, D>(cp, cq, gv, scale, tab, acc, P, c)) {
#pragma unroll
            for (int d = 0; d < D; ++d) g[d] += (double)c[d];
        }
    }
    const int l = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int d = 0; d < D; ++d) {
        double v = g[d];
        for (int o = 32; o > 0; o >>= 1) v += __shfl_down(v, o, 64);
        if (l == 0) s_red[w][d] = v;
    }
    __syncthreads();
    if (threadIdx.x < D) {
        const int d = threadIdx.x;
        dpd[(int64_t)p * D + d] = s_red[0][d] + s_red[1][d] + s_red[2][d] + s_red[3][d];
    }
}

template <typename T, int MODE>
static void launch_dense_pts(const Graph& g, const Table<T>& tb, const double* C, const T* alpha,
                             double* dpd, hipStream_t st) {
    const int n = (int)g.n0;
    const T scale = (T)g.scale;
    switch (g.D) {
        case 2: hipLaunchKernelGGL((k_dense_pts<T, 2, MODE>), dim3(n), dim3(256), 0, st, g.coords, n, scale, tb.tab, tb.acc, tb.params, C, alpha, dpd); break;
        case 3: hipLaunchKernelGGL((k_dense_pts<T, 3, MODE>), dim3(n), dim3(256), 0, st, g.coords, n, scale, tb.tab, tb.acc, tb.params, C, alpha, dpd); break;
        case 4: hipLaunchKernelGGL((k_dense_pts<T, 4, MODE>), dim3(n), dim3(256), 0, st, g.coords, n, scale, tb.tab, tb.acc, tb.params, C, alpha, dpd); break;
        default: break;
    }
}

// d(sum log diag L)/dpoints: K^-1 = W^T W in full (both triangles).
template <typename T>
void dense_grad_points_logdet(const Graph& g, const Table<T>& tb, const T* L, double* W,
                              double* C, double* dpd, hipStream_t st) {
    const int n = (int)g.n0;
    dense_inverse64(L, n, W, C, st);
    launch_gemm<double>({gemm_job(W, n, 1, W, n, C, n, n, n, n, GK_FROM_I | GK_FROM_J, 1.0)}, st);
    launch_dense_pts<T, DM_LOGDET>(g, tb, C, nullptr, dpd, st);
}

// d(0.5 y^T K^-1 y)/dpoints with alpha = K^-1 y.
template <typename T>
void dense_grad_points_invloss(const Graph& g, const Table<T>& tb, const T* alpha, double* dpd,
                               hipStream_t st) {
    launch_dense_pts<T, DM_INVLOSS>(g, tb, nullptr, alpha, dpd, st);
}

#define GGP_DENSE_INST(T)                                                                      \
    template void dense_assemble<T>(const Graph&, const Table<T>&, T*, T, hipStream_t, int*,   \
                                    int*);                                                     \
    template void dense_potrf<T>(T*, int, int*, int*, int, hipStream_t, bool);                            \
    template void dense_trmv<T>(const T*, int, const T*, T*, hipStream_t, T*, const int32_t*); \
    template void dense_trmv_t<T>(const T*, int, const T*, T*, hipStream_t, T*,                \
                                  const int32_t*);                                             \
    template void dense_trsv<T>(const T*, int, const T*, T*, int*, int*, hipStream_t);         \
    template void dense_trsv_t<T>(const T*, int, const T*, T*, int*, int*, hipStream_t);       \
    template void dense_logdiag<T>(const T*, int, double*, hipStream_t);                       \
    template void dense_grad_logdet<T>(const Graph&, const Table<T>&, const T*, double*,       \
                                       double*, double*, int, hipStream_t);                    \
    template void dense_grad_generate<T>(const Graph&, const Table<T>&, const T*, const T*,    \
                                         const T*, double*, double*, double*, double*,         \
                                         double*, int, bool, hipStream_t);                     \
    template void dense_inverse<T>(const T*, int, double*, double*, hipStream_t);              \
    template void dense_grad_invloss<T>(const Graph&, const Table<T>&, const T*, double*, int, \
                                        hipStream_t);                                          \
    template void dense_grad_points_logdet<T>(const Graph&, const Table<T>&, const T*,         \
                                              double*, double*, double*, hipStream_t);         \
    template void dense_grad_points_invloss<T>(const Graph&, const Table<T>&, const T*,        \
                                               double*, hipStream_t);                          \
    template size_t dense_scatter_lds<T>(const Table<T>&);
GGP_DENSE_INST(float)
GGP_DENSE_INST(double)

}  // namespace ggp
