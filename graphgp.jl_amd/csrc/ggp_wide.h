// ggp_wide.h — per-point kernels for any neighbour count k <= 31 (one wavefront per point).
//
// The register-block kernels (ggp_point_kernels.h) give each lane a whole point and unroll
// every loop over the (k+1)^2 block at compile time; they exist for the common k (4, 8, 10, 16).
// Here a wavefront owns one point and lane r owns ROW r of the block, so the per-lane state is
// one row (at most 32 entries) and k is a run-time value:
//
//   * Cholesky (src/linalg.jl:38-73) right-looking, lane-parallel over rows. At step j the
//     pivot comes from lane j (readlane) and every row subtracts L_rj * L_cj from its entry c in
//     increasing j, which is the reference's left-looking fma chain for that entry, term by
//     term, so the factor is bit-identical to the serial loop.
//   * mean_vec_solve (src/linalg.jl:85-103) and the seed substitutions of the adjoints are
//     order-dependent serial recurrences; they run wave-uniformly (every lane computes the same
//     chain from readlane'd operands), in the reference's order.
//   * chol_pullback (src/linalg.jl:112-137) keeps L and Lbar as COLUMNS (lane c owns column c):
//     in step j the updates of row j of Lbar are chains over i on the lane of each column p, and
//     those of rows i > j touch one entry per (i, p); both keep the reference's per-entry order.
//     Column j of Lbar and of L reaches the row lanes through a 64-entry LDS slot per wave.
//
// Lanes beyond k compute on copies and never publish anything; entries above a lane's
// diagonal are scratch that no result reads.
#pragma once
#include "ggp_point_kernels.h"  // tab_bytes, block_sum, the shared LDS table layout

namespace ggp {

constexpr int kWideN = 32;       // largest k+1 handled here
constexpr int kWideWaves = kWideBlock / 64;  // points per workgroup pass

// Orders the LDS accesses of one wavefront around a cross-lane exchange (no workgroup barrier:
// the exchange is private to the wavefront).
__device__ inline void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Sum over the 64 lanes of the wavefront, returned to every lane.
__device__ inline double wave_sum(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Joint coordinates of row `lane`: neighbour `lane` for lane < k, the point itself otherwise
// (_gather_joint!, src/kernels.jl:9-23). Returns the neighbour index (-1 for the point row).
// nbr64 (optional): the neighbours in the reference's layout, int64 nbr64[m*K + j].
template <int D>
__device__ inline int32_t wide_gather(uint32_t (&x)[D], const uint32_t* __restrict__ coords,
                                      const int32_t* __restrict__ nbr, int64_t M, int64_t m,
                                      int64_t n0, int K, int lane,
                                      const int64_t* __restrict__ nbr64 = nullptr) {
    int32_t nb = -1;
    int64_t row = n0 + m;
    if (lane < K) {
        if (nbr64) {  // not validated on the host: an index that does not precede the point
            const int64_t q = nbr64[m * K + lane];  // is read as the point itself
            nb = (int32_t)(q >= 0 && q < n0 + m ? q : n0 + m);
        } else {
            nb = nbr[(int64_t)lane * M + m];
        }
        row = nb;
    }
    const uint32_t* c = coords + row * D;
#pragma unroll
    for (int d = 0; d < D; ++d) x[d] = c[d];
    return nb;
}

// Row `lane` of the covariance (assemble_cov!, src/linalg.jl:15-29; anisotropic form
// src/aniso.jl:88-108): a[c] for c <= lane.
template <typename T, int D, bool ANISO>
__device__ inline void wide_assemble(T (&a)[kWideN], const uint32_t (&x)[D], int n, int lane,
                                     T scale, const TabEnt<T>* tab, const uint16_t* acc,
                                     const TabParams<T>& P, const AnisoArgs<T>& an) {
    const T diag = ANISO ? aniso_lookup(T(0), T(0), an) : P.v0;
#pragma unroll
    for (int c = 0; c < kWideN; ++c) {
        if (c < n) {
            uint32_t xc[D];
#pragma unroll
            for (int d = 0; d < D; ++d) xc[d] = bcast(x[d], c);
            T v = diag;
            if (c < lane && lane < n) {
                if (ANISO) v = aniso_pair<T, D>(x, xc, scale, an);
                else v = cov_lookup(radius<T>(sqdist<D>(x, xc), scale), tab, acc, P);
            }
            a[c] = v;
        }
    }
}

// chol_lower! (src/linalg.jl:38-73) on rows held one per lane. Returns L[k][k] (the std).
// COLS: also gather the factor by columns into lc (lane c: lc[i] = L[i][c], i >= c).
template <typename T, bool COLS>
__device__ inline T wide_cholesky(T (&a)[kWideN], T (&lc)[kWideN], int n, int K, int lane) {
    const T pivmin = num<T>::eps() * bcast(a[0], 0);
    const T dmin = num<T>::sqrt(pivmin);
    T sdev = T(0);
#pragma unroll
    for (int j = 0; j < kWideN; ++j) {
        if (j < n) {
            const T s = bcast(a[j], j);
            const bool ok = s > pivmin;  // false for NaN, as in the reference
            const T d = ok ? num<T>::sqrt(s) : dmin;
            const T q = a[j] / d;
            a[j] = lane == j ? d : (lane > j ? (ok ? q : T(0)) : a[j]);
            if (j == K) sdev = d;
            if (COLS) lc[j] = put(lc[j], d, j, lane);
#pragma unroll
            for (int c = j + 1; c < kWideN; ++c) {
                if (c < n) {
                    const T lcj = bcast(a[j], c);
                    if (COLS) lc[c] = put(lc[c], lcj, j, lane);
                    a[c] = num<T>::fma(-a[j], lcj, a[c]);
                }
            }
        }
    }
    return sdev;
}

// mean_vec_solve! (src/linalg.jl:85-103) as one wave-uniform chain; lane i receives x_i.
// Rows of L are in a (lane r = row r).
template <typename T>
__device__ inline T wide_mean_vec(const T (&a)[kWideN], int K, int lane) {
    const T pivfloor = T(1.5) * num<T>::sqrt(num<T>::eps()) * bcast(a[0], 0);
    T xs[kWideN];
    T mine = T(0);
#pragma unroll
    for (int i = kWideN - 2; i >= 0; --i) {
        if (i < K) {
            const T d = bcast(a[i], i);
            T s = bcast(a[i], K);
#pragma unroll
            for (int j = i + 1; j < kWideN - 1; ++j)
                if (j < K) s = num<T>::fma(-bcast(a[i], j), xs[j], s);
            xs[i] = d > pivfloor ? s / d : T(0);
            mine = lane == i ? xs[i] : mine;
        }
    }
    return mine;
}

// ---- factor pass (k_factor's twin) ----------------------------------------------------------
// TG: the table is read from global memory (too large for LDS) instead of being staged. MODE = -1:
// the mode is the run-time rt_mode (one instantiation serves every mode; used for TG, whose
// speed matters less than its build time).
template <typename T, int D, int MODE, bool ANISO, bool TG>
__global__ void __launch_bounds__(kWideBlock)
k_factor_w(const uint32_t* __restrict__ coords, const int32_t* __restrict__ nbr, int64_t M,
           int64_t n0, int K, T scale, const TabEnt<T>* __restrict__ g_tab,
           const uint16_t* __restrict__ g_acc, const TabParams<T>* __restrict__ Pp,
           T* __restrict__ mv, T* __restrict__ sd, T* __restrict__ terms,
           double* __restrict__ partial, const T* __restrict__ values, T* __restrict__ xi_out,
           AnisoArgs<T> an, const int64_t* __restrict__ nbr64, int rt_mode) {
    const int mode = MODE >= 0 ? MODE : rt_mode;
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ double s_red[kWideWaves];
    TabParams<T> P{};
    TabEnt<T>* s_tab = nullptr;
    uint16_t* s_acc = nullptr;
    if (!ANISO) {
        P = *Pp;
        if (TG) {
            s_tab = const_cast<TabEnt<T>*>(g_tab);
            s_acc = const_cast<uint16_t*>(g_acc);
        } else {
            s_tab = reinterpret_cast<TabEnt<T>*>(smem);
            s_acc = reinterpret_cast<uint16_t*>(smem + (size_t)(P.nb - 1) * sizeof(TabEnt<T>));
            stage_table(s_tab, s_acc, g_tab, g_acc, P);
        }
    }
    AnisoArgs<T> av{};
    if (ANISO) av = aniso_stage(an, smem);
    const int lane = threadIdx.x & 63;
    const int n = K + 1;
    double lsum = 0.0;
    const int64_t wstride = (int64_t)gridDim.x * kWideWaves;
    for (int64_t m = (int64_t)blockIdx.x * kWideWaves + (threadIdx.x >> 6); m < M; m += wstride) {
        uint32_t x[D];
        const int32_t nb = wide_gather<D>(x, coords, nbr, M, m, n0, K, lane, nbr64);
        T a[kWideN], unused[kWideN];
        wide_assemble<T, D, ANISO>(a, x, n, lane, scale, s_tab, s_acc, P, av);
        const T s = wide_cholesky<T, false>(a, unused, n, K, lane);
        if (mode & F_TERMS) {
            const T t = num<T>::log(s);
            if (lane == 0) {
                if (terms) terms[m] = t;
                lsum += (double)t;
            }
        }
        if (mode & (F_MV | F_INV)) {
            const T xm = wide_mean_vec(a, K, lane);
            if (mode & F_MV) {
                if (lane < K) mv[m * K + lane] = xm;
                if (lane == 0) sd[m] = s;
            }
            if (mode & F_INV) {  // src/kernels.jl:48-55
                const T prod = lane < K ? xm * values[nb] : T(0);
                T mean = T(0);
#pragma unroll
                for (int j = 0; j < kWideN - 1; ++j)
                    if (j < K) mean = mean + bcast(prod, j);
                if (lane == 0) xi_out[m] = (values[n0 + m] - mean) / s;
            }
        }
    }
    if (mode & F_TERMS) {
        const double t = block_sum(lsum, s_red);
        if (threadIdx.x == 0) partial[blockIdx.x] = t;
    }
}

// ---- adjoint pullback (k_pullback's twin) ---------------------------------------------------
// TG: the table is read from global memory and the histogram is accumulated with f64 atomics
// directly in this workgroup's row of hist_partial (zeroed by the host before the launch).
// MODE = -1: the mode is the run-time rt_mode (as for k_factor_w).
template <typename T, int D, int MODE, bool TG>
__global__ void __launch_bounds__(kWideBlock)
k_pullback_w(const uint32_t* __restrict__ coords, const int32_t* __restrict__ nbr, int64_t M,
             int64_t n0, int K, T scale, const TabEnt<T>* __restrict__ g_tab,
             const uint16_t* __restrict__ g_acc, const TabParams<T>* __restrict__ Pp,
             const T* __restrict__ v, const T* __restrict__ xi, const T* __restrict__ vb,
             double* __restrict__ hist_partial, double* __restrict__ scalar_partial,
             int rt_mode) {
    const int mode = MODE >= 0 ? MODE : rt_mode;
    const int SEED = mode & 3;
    const bool PTS = (mode & P_PTS) != 0;
    const TabParams<T> P = *Pp;
    extern __shared__ __align__(16) unsigned char smem[];
    TabEnt<T>* s_tab = TG ? const_cast<TabEnt<T>*>(g_tab) : reinterpret_cast<TabEnt<T>*>(smem);
    uint16_t* s_acc = TG ? const_cast<uint16_t*>(g_acc)
                         : reinterpret_cast<uint16_t*>(smem + (size_t)(P.nb - 1) * sizeof(TabEnt<T>));
    double* s_hist = TG ? hist_partial + (size_t)blockIdx.x * P.nb
                        : reinterpret_cast<double*>(smem + tab_bytes<T>(P.nb, P.ucells));
    __shared__ double s_red[kWideWaves];
    __shared__ T s_xch[kWideWaves][2][64];
    if (!TG) {
        if (!PTS)
            for (int i = threadIdx.x; i < P.nb; i += blockDim.x) s_hist[i] = 0.0;
        stage_table(s_tab, s_acc, g_tab, g_acc, P);
    }

    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    T* xb = s_xch[w][0];  // column j of Lbar, by row
    T* xl = s_xch[w][1];  // column j of L, by row
    const int n = K + 1;
    const AnisoArgs<T> no_aniso{};
    double ssum = 0.0;
    const int64_t wstride = (int64_t)gridDim.x * kWideWaves;
    for (int64_t m = (int64_t)blockIdx.x * kWideWaves + w; m < M; m += wstride) {
        uint32_t x[D];
        const int32_t nb = wide_gather<D>(x, coords, nbr, M, m, n0, K, lane);
        T a[kWideN], lc[kWideN], bc[kWideN];
        wide_assemble<T, D, false>(a, x, n, lane, scale, s_tab, s_acc, P, no_aniso);
#pragma unroll
        for (int i = 0; i < kWideN; ++i) lc[i] = T(0);
        const T s = wide_cholesky<T, true>(a, lc, n, K, lane);

        // ---- seeds: bc[i] = Lbar[i][lane] ----
#pragma unroll
        for (int i = 0; i < kWideN; ++i) bc[i] = T(0);
        if (SEED == P_LOGDET) {
            // src/linalg.jl:140-146 with seed 1; the term itself for the fused logdet.
            if (lane == 0) ssum += (double)num<T>::log(s);
            const T seed = T(1) / s;
#pragma unroll
            for (int i = 0; i < kWideN; ++i)
                if (i == K) bc[i] = lane == K ? seed : T(0);
        } else {
            const T xm = wide_mean_vec(a, K, lane);
            const T vnb = lane < K ? v[nb] : T(0);
            T seed, z0;
            if (SEED == P_INVLOSS) {
                // src/kernels_adjoint.jl:183-211 (no @fastmath there).
                const T prod = lane < K ? xm * vnb : T(0);
                T mean = T(0);
#pragma unroll
                for (int j = 0; j < kWideN - 1; ++j)
                    if (j < K) mean = mean + bcast(prod, j);
                const T xim = (v[n0 + m] - mean) / s;
                if (lane == 0) ssum += (double)(xim * xim / T(2));
                seed = -xim * xim / s;
                z0 = -xim * vnb / s;
            } else {
                // src/kernels_adjoint.jl:509-538.
                const T vbp = vb[n0 + m];
                seed = vbp * xi[n0 + m];
                z0 = vbp * vnb;
            }
            // Forward substitution L[0:k,0:k] zbar = z0 as one uniform chain (unguarded for the
            // inverse loss, guarded like mean_vec_solve! for generate_grad_vals).
            const T pivfloor = T(1.5) * num<T>::sqrt(num<T>::eps()) * bcast(a[0], 0);
            T zs[kWideN];
            T zm = T(0);
#pragma unroll
            for (int i = 0; i < kWideN - 1; ++i) {
                if (i < K) {
                    T t = bcast(z0, i);
#pragma unroll
                    for (int p = 0; p < i; ++p) t = t - bcast(a[p], i) * zs[p];
                    const T dii = bcast(a[i], i);
                    if (SEED == P_INVLOSS) zs[i] = t / dii;
                    else zs[i] = dii > pivfloor ? t / dii : T(0);
                    zm = lane == i ? zs[i] : zm;
                }
            }
            // Lbar[k][j] = zbar_j; Lbar[j][i] = -(zbar_i x_j) for i <= j < k; Lbar[k][k] = seed.
#pragma unroll
            for (int i = 0; i < kWideN; ++i) {
                if (i <= K) {
                    const T xi_i = i < K ? bcast(xm, i) : T(0);
                    T val = T(0);
                    if (i == K) val = lane < K ? T(0) + zm : (lane == K ? seed : T(0));
                    else if (lane <= i) val = T(0) - zm * xi_i;
                    bc[i] = val;
                }
            }
        }

        // ---- chol_pullback! (src/linalg.jl:112-137), columns on lanes ----
        T sbar_mine = T(0);
        double gpt[D];  // P_PTS: this row's point gradient
#pragma unroll
        for (int d = 0; d < D; ++d) gpt[d] = 0.0;
#pragma unroll
        for (int j = kWideN - 1; j >= 0; --j) {
            if (j < n) {
                const T ljj = bcast(lc[j], j);
                // column j of Lbar and of L from lane j to the row lanes
                if (lane == j) {
#pragma unroll
                    for (int i = j + 1; i < kWideN; ++i)
                        if (i < n) { xb[i] = bc[i]; xl[i] = lc[i]; }
                }
                wave_sync();
                const bool row = lane > j && lane < n;
                const T lb = row ? xb[lane] : T(0);
                const T lij = row ? xl[lane] : T(0);
                wave_sync();
                const T tbar = lb / ljj;
                const T qv = lb * lij / ljj;
                // Abar[lane][j] = tbar through the lookup weights (src/kernels_adjoint.jl:47-74),
                // or through k'(r) dr/dx into points lane and j (src/kernels_adjoint.jl:223-252)
                if (PTS) {
                    uint32_t xj[D];
#pragma unroll
                    for (int d = 0; d < D; ++d) xj[d] = bcast(x[d], j);
                    T c[D];
#pragma unroll
                    for (int d = 0; d < D; ++d) c[d] = T(0);
                    if (row) (void)pair_pts<T, D>(x, xj, tbar, scale, s_tab, s_acc, P, c);
#pragma unroll
                    for (int d = 0; d < D; ++d) {
                        gpt[d] += (double)c[d];
                        const double cs = wave_sum((double)c[d]);
                        if (lane == j) gpt[d] -= cs;
                    }
                } else {
                    uint32_t xj[D];
#pragma unroll
                    for (int d = 0; d < D; ++d) xj[d] = bcast(x[d], j);
                    if (row) {
                        const T r = radius<T>(sqdist<D>(x, xj), scale);
                        T wlo, whi;
                        const int lo = cov_weights(r, s_tab, s_acc, P, wlo, whi);
                        atomicAdd(&s_hist[lo], (double)(tbar * wlo));
                        atomicAdd(&s_hist[lo + 1], (double)(tbar * whi));
                    }
                }
                T t = bcast(bc[j], j);  // Lbar[j][j]
#pragma unroll
                for (int i = kWideN - 1; i > j; --i) {
                    if (i < n) {
                        t = t - bcast(qv, i);
                        const T tb = bcast(tbar, i);
                        bc[i] = num<T>::fma(-tb, lc[j], bc[i]);  // Lbar[i][lane], lane < j
                        bc[j] = num<T>::fma(-tb, lc[i], bc[j]);  // Lbar[j][lane], lane < j
                    }
                }
                const T sbar = t / (T(2) * ljj);
                sbar_mine = lane == j ? sbar : sbar_mine;
                bc[j] = num<T>::fma(-(T(2) * sbar), lc[j], bc[j]);
            }
        }
        if (PTS) {
            if (lane < n) {
                const int64_t gp = lane < K ? (int64_t)nb : n0 + m;
#pragma unroll
                for (int d = 0; d < D; ++d) atomicAdd(&hist_partial[gp * D + d], gpt[d]);
            }
        } else {
            // diagonal of Abar: one add per row into bin 0, summed in row order
            T diag = T(0);
#pragma unroll
            for (int j = 0; j < kWideN; ++j)
                if (j < n) diag += bcast(sbar_mine, j);
            if (lane == 0) atomicAdd(&s_hist[0], (double)diag);
        }
    }
    __syncthreads();
    if (!PTS && !TG) {
        double* out = hist_partial + (size_t)blockIdx.x * P.nb;
        for (int i = threadIdx.x; i < P.nb; i += blockDim.x) out[i] = s_hist[i];
    }
    if (scalar_partial) {
        const double t = block_sum(ssum, s_red);
        if (threadIdx.x == 0) scalar_partial[blockIdx.x] = t;
    }
}

}  // namespace ggp
