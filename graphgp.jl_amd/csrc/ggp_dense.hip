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
#include "ggp_internal.h"

namespace ggp {

static inline unsigned cdiv(int64_t a, int64_t b) { return (unsigned)((a + b - 1) / b); }

// ---- assembly (src/dense.jl:15-40) ----------------------------------------------------------
template <typename T, int D, bool ANISO>
__global__ void k_dense_assemble(T* __restrict__ A, const uint32_t* __restrict__ coords, int n,
                                 T scale, const TabEnt<T>* __restrict__ tab,
                                 const uint16_t* __restrict__ acc, const TabParams<T>* __restrict__ Pp, T diag_add,
                                 AnisoArgs<T> an) {
    const int j = blockIdx.x * 16 + threadIdx.x;
    const int i = blockIdx.y * 16 + threadIdx.y;
    if (i >= n || j > i) return;
    TabParams<T> P{};
    if (!ANISO) P = *Pp;
    if (i == j) {
        const T d0 = ANISO ? aniso_lookup(T(0), T(0), an) : P.v0;
        A[(int64_t)i * n + i] = diag_add == T(0) ? d0 : d0 + diag_add;
        return;
    }
    uint32_t ci[D], cj[D];
#pragma unroll
    for (int d = 0; d < D; ++d) { ci[d] = coords[(int64_t)i * D + d]; cj[d] = coords[(int64_t)j * D + d]; }
    const T v = ANISO ? aniso_pair<T, D>(ci, cj, scale, an)
                      : cov_lookup(radius<T>(sqdist<D>(ci, cj), scale), tab, acc, P);
    A[(int64_t)i * n + j] = v;
    A[(int64_t)j * n + i] = v;
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

int dense_sync_ints(int n) {
    const int nt = (n + kTile - 1) / kTile;
    return nt * nt + 1;
}

template <typename T>
void dense_potrf(T* A, int n, int* info, int* sync, int max_wg, hipStream_t st) {
    if (n <= 0) return;
    const int nt = (n + kTile - 1) / kTile;
    const int ntiles = nt * (nt + 1) / 2;
    launch_fill<int>(sync, 0, dense_sync_ints(n), st);
    const int nwg = std::max(1, std::min(ntiles, max_wg));
    hipLaunchKernelGGL((k_potrf_tiles<T>), dim3(nwg), dim3(kDfThreads), 0, st, A, n, nt, sync, info);
}

// ---- triangular products and solves ---------------------------------------------------------
// y = L x (src/dense.jl:118): row i accumulates j = 0..i.
template <typename T>
__global__ void k_trmv(const T* __restrict__ L, int n, const T* __restrict__ x, T* __restrict__ y) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const T* row = L + (int64_t)i * n;
    T acc = T(0);
#pragma unroll 16
    for (int j = 0; j <= i; ++j) acc = num<T>::fma(row[j], x[j], acc);
    y[i] = acc;
}
// y = L^T x (src/grad.jl:457, 493): entry i accumulates j = i..n-1.
template <typename T>
__global__ void k_trmv_t(const T* __restrict__ L, int n, const T* __restrict__ x, T* __restrict__ y) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    T acc = T(0);
#pragma unroll 16
    for (int j = i; j < n; ++j) acc = num<T>::fma(L[(int64_t)j * n + i], x[j], acc);
    y[i] = acc;
}

// x = L \ b (src/dense.jl:134), one workgroup: 32-row diagonal blocks solved by wave 0 with
// broadcasts, the rows below updated by all threads; per entry the same fma chain as the
// row-by-row substitution.
template <typename T>
__global__ void __launch_bounds__(256) k_trsv(const T* __restrict__ L, int n,
                                              const T* __restrict__ b, T* __restrict__ x) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) x[i] = b[i];
    __syncthreads();
    for (int k0 = 0; k0 < n; k0 += kTile) {
        const int nk = min(kTile, n - k0);
        if (threadIdx.x < 64) {
            const int lane = threadIdx.x;
            T v = lane < nk ? x[k0 + lane] : T(0);
            for (int jj = 0; jj < nk; ++jj) {
                const T xj = bcast(v, jj) / L[(int64_t)(k0 + jj) * n + k0 + jj];
                if (lane == jj) v = xj;
                else if (lane > jj && lane < nk)
                    v = num<T>::fma(-L[(int64_t)(k0 + lane) * n + k0 + jj], xj, v);
            }
            if (lane < nk) x[k0 + lane] = v;
        }
        __syncthreads();
        for (int i = k0 + nk + threadIdx.x; i < n; i += blockDim.x) {
            T s = x[i];
            const T* row = L + (int64_t)i * n + k0;
            for (int p = 0; p < nk; ++p) s = num<T>::fma(-row[p], x[k0 + p], s);
            x[i] = s;
        }
        __syncthreads();
    }
}

// x = L^T \ b (src/dense.jl:236), blocked backward substitution.
template <typename T>
__global__ void __launch_bounds__(256) k_trsv_t(const T* __restrict__ L, int n,
                                                const T* __restrict__ b, T* __restrict__ x) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) x[i] = b[i];
    __syncthreads();
    const int nt = (n + kTile - 1) / kTile;
    for (int kb = nt - 1; kb >= 0; --kb) {
        const int k0 = kb * kTile, nk = min(kTile, n - k0);
        if (threadIdx.x < 64) {
            const int lane = threadIdx.x;
            T v = lane < nk ? x[k0 + lane] : T(0);
            for (int jj = nk - 1; jj >= 0; --jj) {
                const T xj = bcast(v, jj) / L[(int64_t)(k0 + jj) * n + k0 + jj];
                if (lane == jj) v = xj;
                else if (lane < jj) v = num<T>::fma(-L[(int64_t)(k0 + jj) * n + k0 + lane], xj, v);
            }
            if (lane < nk) x[k0 + lane] = v;
        }
        __syncthreads();
        for (int i = threadIdx.x; i < k0; i += blockDim.x) {
            T s = x[i];
            for (int p = 0; p < nk; ++p) s = num<T>::fma(-L[(int64_t)(k0 + p) * n + i], x[k0 + p], s);
            x[i] = s;
        }
        __syncthreads();
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
void dense_trmv(const T* L, int n, const T* x, T* y, hipStream_t st) {
    hipLaunchKernelGGL((k_trmv<T>), dim3(cdiv(n, 64)), dim3(64), 0, st, L, n, x, y);
}
template <typename T>
void dense_trmv_t(const T* L, int n, const T* x, T* y, hipStream_t st) {
    hipLaunchKernelGGL((k_trmv_t<T>), dim3(cdiv(n, 64)), dim3(64), 0, st, L, n, x, y);
}
template <typename T>
void dense_trsv(const T* L, int n, const T* b, T* x, hipStream_t st) {
    hipLaunchKernelGGL((k_trsv<T>), dim3(1), dim3(256), 0, st, L, n, b, x);
}
template <typename T>
void dense_trsv_t(const T* L, int n, const T* b, T* x, hipStream_t st) {
    hipLaunchKernelGGL((k_trsv_t<T>), dim3(1), dim3(256), 0, st, L, n, b, x);
}
template <typename T>
void dense_logdiag(const T* L, int n, double* out, hipStream_t st) {
    hipLaunchKernelGGL((k_logdiag<T>), dim3(1), dim3(256), 0, st, L, n, out);
}

template <typename T>
void dense_assemble(const Graph& g, const Table<T>& tb, T* A, T diag_add, hipStream_t st) {
    const int n = (int)g.n0;
    const dim3 grid(cdiv(n, 16), cdiv(n, 16)), blk(16, 16);
    const T scale = (T)g.scale;
    const bool an = tb.aniso.grid != nullptr;
#define GGP_ASM(DD)                                                                             \
    do {                                                                                        \
        if (an) hipLaunchKernelGGL((k_dense_assemble<T, DD, true>), grid, blk, 0, st, A, g.coords, n, scale, tb.tab, tb.acc, tb.params, diag_add, tb.aniso); \
        else hipLaunchKernelGGL((k_dense_assemble<T, DD, false>), grid, blk, 0, st, A, g.coords, n, scale, tb.tab, tb.acc, tb.params, diag_add, tb.aniso); \
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
// W = L^-1 in double. One wave solves kInvCols consecutive columns c0.. (so each row of L it reads
// serves all of them), left-looking over 64-row blocks: lane l of block r0 first forms
// acc_c = e_c[r] - sum_{c0<=p<r0} L[r][p] x_c[p] along its own row r = r0+l of L (contiguous
// reads; x in LDS), then the 64 x 64 diagonal block is solved from registers with the pivots
// broadcast by readlane.
constexpr int kInvCols = 1;

// lr[lane] of a 64-entry register row, selected by the lane's own index (a select chain, since
// registers cannot be indexed at run time).
__device__ inline double bcast_lane_diag(const double (&lr)[64], int lane) {
    double v = 1.0;
#pragma unroll
    for (int jj = 0; jj < 64; ++jj) v = lane == jj ? lr[jj] : v;
    return v;
}

template <typename T>
__global__ void __launch_bounds__(64) k_trinv(const T* __restrict__ L, int n,
                                              double* __restrict__ W) {
    extern __shared__ double sx[];  // kInvCols x n
    const int c0 = blockIdx.x * kInvCols, lane = threadIdx.x;
    for (int r0 = c0; r0 < n; r0 += 64) {
        const int r = r0 + lane;
        const bool live = r < n;
        const T* row = L + (int64_t)(live ? r : 0) * n;
        double acc[kInvCols];
#pragma unroll
        for (int q = 0; q < kInvCols; ++q) acc[q] = (r == c0 + q) ? 1.0 : 0.0;
        if (live) {
#pragma unroll 4
            for (int p = c0; p < r0; ++p) {
                const double lp = (double)row[p];
#pragma unroll
                for (int q = 0; q < kInvCols; ++q) acc[q] = __builtin_fma(-lp, sx[q * n + p], acc[q]);
            }
        }
        double lr[64];
#pragma unroll
        for (int jj = 0; jj < 64; ++jj) lr[jj] = (live && r0 + jj < n) ? (double)row[r0 + jj] : 1.0;
        // one reciprocal per row: lane l holds 1 / L[r0+l][r0+l]
        const double rinv = 1.0 / bcast_lane_diag(lr, lane);
#pragma unroll
        for (int jj = 0; jj < 64; ++jj) {
            if (r0 + jj < n) {
                const double rp = bcast(rinv, jj);
#pragma unroll
                for (int q = 0; q < kInvCols; ++q) {
                    const double xj = bcast(acc[q], jj) * rp;
                    if (lane == jj) acc[q] = xj;
                    else if (lane > jj) acc[q] = __builtin_fma(-lr[jj], xj, acc[q]);
                }
            }
        }
        if (live)
#pragma unroll
            for (int q = 0; q < kInvCols; ++q) sx[q * n + r] = acc[q];
        __syncthreads();
    }
    for (int q = 0; q < kInvCols; ++q) {
        const int c = c0 + q;
        if (c >= n) break;
        for (int r = lane; r < n; r += 64) W[(int64_t)r * n + c] = r < c ? 0.0 : sx[q * n + r];
    }
}

// C[i][j] = sum_{a >= max(i, j)} W[a][i] X[a][j] for lower-triangular W, X (n x n, row-major):
// 64 x 64 output tiles, 4 x 4 outputs per thread, 16-row slabs of W and X staged in LDS.
// lower_only: only tiles with i >= j.
constexpr int kWT = 64, kWK = 16;
__global__ void __launch_bounds__(256) k_wtx(const double* __restrict__ W,
                                             const double* __restrict__ X, int n,
                                             double* __restrict__ C, int lower_only) {
    __shared__ double sW[kWK][kWT + 1];
    __shared__ double sX[kWK][kWT + 1];
    const int bi = blockIdx.y, bj = blockIdx.x;
    if (lower_only && bj > bi) return;
    const int i0 = bi * kWT, j0 = bj * kWT;
    const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
    double acc[4][4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[u][v] = 0.0;
    const int a_start = (max(i0, j0) / kWK) * kWK;
    for (int a0 = a_start; a0 < n; a0 += kWK) {
        for (int e = threadIdx.x; e < kWK * kWT; e += blockDim.x) {
            const int rr = e / kWT, cc = e % kWT;
            const int a = a0 + rr;
            sW[rr][cc] = (a < n && i0 + cc < n) ? W[(int64_t)a * n + i0 + cc] : 0.0;
            sX[rr][cc] = (a < n && j0 + cc < n) ? X[(int64_t)a * n + j0 + cc] : 0.0;
        }
        __syncthreads();
#pragma unroll
        for (int rr = 0; rr < kWK; ++rr) {
            double w[4], x[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) w[u] = sW[rr][ty + 16 * u];
#pragma unroll
            for (int v = 0; v < 4; ++v) x[v] = sX[rr][tx + 16 * v];
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[u][v] = __builtin_fma(w[u], x[v], acc[u][v]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int i = i0 + ty + 16 * u, j = j0 + tx + 16 * v;
            if (i < n && j < n) C[(int64_t)i * n + j] = acc[u][v];
        }
}

// u = L^T vb (double), h/Q prefix pass: Q[a][j] = u[a] (sum_{j<=b<a} xi[b] W[b][j] + xi[a]W[a][j]/2)
template <typename T>
__global__ void k_ltv64(const T* __restrict__ L, int n, const T* __restrict__ vb,
                        double* __restrict__ u) {
    const int a = blockIdx.x * blockDim.x + threadIdx.x;
    if (a >= n) return;
    double s = 0.0;
#pragma unroll 16
    for (int i = a; i < n; ++i) s = __builtin_fma((double)L[(int64_t)i * n + a], (double)vb[i], s);
    u[a] = s;
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
// hist_partial.
template <typename T, int D, int MODE>
__global__ void __launch_bounds__(256) k_dense_scatter(const uint32_t* __restrict__ coords,
                                                       int n, T scale,
                                                       const TabEnt<T>* __restrict__ tab,
                                                       const uint16_t* __restrict__ acc,
                                                       const TabParams<T>* __restrict__ Pp,
                                                       const double* __restrict__ C,
                                                       const T* __restrict__ alpha,
                                                       double* __restrict__ hist_partial) {
    const TabParams<T> P = *Pp;
    extern __shared__ double s_hist[];
    for (int i = threadIdx.x; i < P.nb; i += blockDim.x) s_hist[i] = 0.0;
    __syncthreads();
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
    __syncthreads();
    double* out = hist_partial + (size_t)blockIdx.x * P.nb;
    for (int i = threadIdx.x; i < P.nb; i += blockDim.x) out[i] = s_hist[i];
}

template <typename T>
size_t dense_scatter_lds(const Table<T>& tb) { return (size_t)tb.P.nb * sizeof(double); }

template <typename T, int MODE>
static void launch_dense_scatter(const Graph& g, const Table<T>& tb, const double* C,
                                 const T* alpha, double* hist_partial, int nw, hipStream_t st) {
    const size_t lds = dense_scatter_lds(tb);
    const int n = (int)g.n0;
    const T scale = (T)g.scale;
    switch (g.D) {
        case 2: hipLaunchKernelGGL((k_dense_scatter<T, 2, MODE>), dim3(nw), dim3(256), lds, st, g.coords, n, scale, tb.tab, tb.acc, tb.params, C, alpha, hist_partial); break;
        case 3: hipLaunchKernelGGL((k_dense_scatter<T, 3, MODE>), dim3(nw), dim3(256), lds, st, g.coords, n, scale, tb.tab, tb.acc, tb.params, C, alpha, hist_partial); break;
        case 4: hipLaunchKernelGGL((k_dense_scatter<T, 4, MODE>), dim3(nw), dim3(256), lds, st, g.coords, n, scale, tb.tab, tb.acc, tb.params, C, alpha, hist_partial); break;
        default: break;
    }
}

template <typename T>
static void dense_inverse64(const T* L, int n, double* W, double* /*scratch*/, hipStream_t st) {
    hipLaunchKernelGGL((k_trinv<T>), dim3(cdiv(n, kInvCols)), dim3(64),
                       (size_t)kInvCols * n * sizeof(double), st, L, n, W);
}

// d(sum log diag L)/dvals: Kinv = W^T W, diagonal halved (src/dense.jl:153-183).
template <typename T>
void dense_grad_logdet(const Graph& g, const Table<T>& tb, const T* L, double* W, double* C,
                       double* hist_partial, int nw, hipStream_t st) {
    const int n = (int)g.n0;
    dense_inverse64(L, n, W, C, st);  // C doubles as the L^T scratch
    const dim3 grid(cdiv(n, kWT), cdiv(n, kWT));
    hipLaunchKernelGGL(k_wtx, grid, dim3(256), 0, st, W, W, n, C, 1);
    launch_dense_scatter<T, DM_LOGDET>(g, tb, C, nullptr, hist_partial, nw, st);
}

// d<vb, L xi>/dvals through the Cholesky adjoint with Lbar = tril(vb xi^T)
// (src/grad_generate_vals.jl:188-211): S = W^T P W with P = Phi(L^T Lbar), P[a][b] = u[a]xi[b]
// (a > b), u[a]xi[a]/2 (a = b), u = L^T vb; Abar[i][j] = S[i][j] + S[j][i], Abar[j][j] = S[j][j].
template <typename T>
void dense_grad_generate(const Graph& g, const Table<T>& tb, const T* L, const T* vb,
                         const T* xi, double* W, double* C, double* Q, double* u,
                         double* hist_partial, int nw, hipStream_t st) {
    const int n = (int)g.n0;
    dense_inverse64(L, n, W, C, st);
    hipLaunchKernelGGL((k_ltv64<T>), dim3(cdiv(n, 64)), dim3(64), 0, st, L, n, vb, u);
    hipLaunchKernelGGL((k_qprefix<T>), dim3(cdiv(n, 32)), dim3(256), 0, st, W, n, xi, u, Q);
    const dim3 grid(cdiv(n, kWT), cdiv(n, kWT));
    hipLaunchKernelGGL(k_wtx, grid, dim3(256), 0, st, W, Q, n, C, 0);
    launch_dense_scatter<T, DM_GENERATE>(g, tb, C, nullptr, hist_partial, nw, st);
}

// d(0.5 y^T K^-1 y)/dvals: -alpha_a alpha_b, diagonal -alpha_a^2/2 (src/dense.jl:244-252).
template <typename T>
void dense_grad_invloss(const Graph& g, const Table<T>& tb, const T* alpha, double* hist_partial,
                        int nw, hipStream_t st) {
    launch_dense_scatter<T, DM_INVLOSS>(g, tb, nullptr, alpha, hist_partial, nw, st);
}

#define GGP_DENSE_INST(T)                                                                      \
    template void dense_assemble<T>(const Graph&, const Table<T>&, T*, T, hipStream_t);        \
    template void dense_potrf<T>(T*, int, int*, int*, int, hipStream_t);                                  \
    template void dense_trmv<T>(const T*, int, const T*, T*, hipStream_t);                     \
    template void dense_trmv_t<T>(const T*, int, const T*, T*, hipStream_t);                   \
    template void dense_trsv<T>(const T*, int, const T*, T*, hipStream_t);                     \
    template void dense_trsv_t<T>(const T*, int, const T*, T*, hipStream_t);                   \
    template void dense_logdiag<T>(const T*, int, double*, hipStream_t);                       \
    template void dense_grad_logdet<T>(const Graph&, const Table<T>&, const T*, double*,       \
                                       double*, double*, int, hipStream_t);                    \
    template void dense_grad_generate<T>(const Graph&, const Table<T>&, const T*, const T*,    \
                                         const T*, double*, double*, double*, double*,         \
                                         double*, int, hipStream_t);                           \
    template void dense_grad_invloss<T>(const Graph&, const Table<T>&, const T*, double*, int, \
                                        hipStream_t);                                          \
    template size_t dense_scatter_lds<T>(const Table<T>&);
GGP_DENSE_INST(float)
GGP_DENSE_INST(double)

}  // namespace ggp
