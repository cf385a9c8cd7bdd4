// ggp_wide.h — per-point kernels for any neighbour count k <= 31: a group of 32 lanes per point,
// two points per wavefront.
//
// The register-block kernels (ggp_point_kernels.h) give each lane a whole point and unroll every
// loop over the (k+1)^2 block at compile time; they exist for the common k (4, 8, 10, 16). Here a
// 32-lane group owns one point and lane r owns ROW r of a padded 32 x 32 block, so the per-lane
// state is one row and k is a run-time value:
//   * rows 0..k-1 hold the neighbours, row 31 the point itself and rows k..30 are padding (zero
//     off the diagonal, one on it). The factor of a padding row stays exactly +0 off the diagonal,
//     so a real entry's chain only ever meets terms fma(-(+0), +0, s) == s after its real terms,
//     and padding columns are skipped: every chain, and so the factor, is the reference's;
//   * Cholesky (src/linalg.jl:38-73) right-looking by columns on the rows' lanes: the pivot comes
//     from its lane (readlane), the finished column goes through LDS and every row reads it back
//     with 16-byte broadcast reads, so each entry takes its fma chain in the left-looking order;
//   * mean_vec_solve (src/linalg.jl:85-103) and the seed substitutions of the adjoints are
//     order-dependent serial recurrences; each group runs them group-uniformly in the reference's
//     order, from a column of L in LDS or from each lane's own row;
//   * chol_pullback (src/linalg.jl:112-137) keeps L and Lbar by COLUMNS (lane c owns column c,
//     after one transpose through LDS). Step j sends column j of Lbar and L to the row lanes, which
//     form tbar = Abar[i][j] and the Lbar[j][j] terms, and get them back to every lane as one LDS
//     vector; each column lane then updates its entries in the reference's per-entry order.
// Each group has LDS for its rows' coordinates, a seed vector and one exchange area. Both
// halves of a wavefront run the same instruction stream; a half past the last point computes a
// copy of the last point and publishes nothing.
#pragma once
#include <type_traits>

#include "ggp_point_kernels.h"  // tab_bytes, block_sum, the shared LDS table layout

namespace ggp {

constexpr int kGrp = 32;                     // lanes per point = rows of the padded block
constexpr int kGrpPt = kGrp - 1;             // the point's row
constexpr int kWideWaves = kWideBlock / 64;  // wavefronts per workgroup

// 16 bytes of T (one LDS vector access).
template <typename T>
struct alignas(16) Q16 {
    T e[16 / sizeof(T)];
};
struct alignas(16) QU {
    uint32_t e[4];
};

// The value of x in lane j of the calling lane's group.
template <typename T>
__device__ __forceinline__ T gbcast(T x, int j, bool hi) {
    const T lo = bcast(x, j), up = bcast(x, kGrp + j);
    return hi ? up : lo;
}

// Sum over the 32 lanes of the group, returned to all of them.
__device__ __forceinline__ double grp_sum(double v) {
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) v += __shfl_xor(v, o, 32);
    return v;
}

// v[c] = src[c] for the 16-byte chunks of src (16-byte aligned, kGrp elements) that hold an
// index >= lo; the others are left alone.
template <typename T>
__device__ __forceinline__ void lds_tail(T (&v)[kGrp], const T* src, int lo) {
    constexpr int V = 16 / sizeof(T);
#pragma unroll
    for (int c0 = 0; c0 < kGrp; c0 += V) {
        if (c0 + V > lo) {
            const Q16<T> q = *reinterpret_cast<const Q16<T>*>(src + c0);
#pragma unroll
            for (int u = 0; u < V; ++u) v[c0 + u] = q.e[u];
        }
    }
}

// Joint coordinates of row r: neighbour r for r < k, the point itself otherwise
// (_gather_joint!, src/kernels.jl:9-23); published to xc (this group's rows, 4 words each).
// Returns the neighbour index (-1 for the point and the padding rows).
// nbr64 (optional): the neighbours in the reference's layout, int64 nbr64[m*K + j].
template <int D>
__device__ __forceinline__ int32_t grp_gather(uint32_t (&x)[D], uint32_t* xc,
                                              const uint32_t* __restrict__ coords,
                                              const int32_t* __restrict__ nbr, int64_t M,
                                              int64_t m, int64_t n0, int K, int r,
                                              const int64_t* __restrict__ nbr64) {
    int32_t nb = -1;
    int64_t row = n0 + m;
    if (r < K) {
        if (nbr64) {  // not validated on the host: an index that does not precede the point
            const int64_t q = nbr64[m * K + r];  // is read as the point itself
            nb = (int32_t)(q >= 0 && q < n0 + m ? q : n0 + m);
        } else {
            nb = nbr[(int64_t)r * M + m];
        }
        row = nb;
    }
    const uint32_t* c = coords + row * D;
    QU w{};
#pragma unroll
    for (int d = 0; d < D; ++d) {
        x[d] = c[d];
        w.e[d] = x[d];
    }
    *reinterpret_cast<QU*>(xc + 4 * r) = w;
    wave_sync_lds();
    return nb;
}

template <int D>
__device__ __forceinline__ void grp_coords(uint32_t (&y)[D], const uint32_t* xc, int j) {
    const QU w = *reinterpret_cast<const QU*>(xc + 4 * j);
#pragma unroll
    for (int d = 0; d < D; ++d) y[d] = w.e[d];
}

// Row r of the covariance (assemble_cov!, src/linalg.jl:15-29; anisotropic form
// src/aniso.jl:88-108): a[c] for c <= r; padding rows get their unit diagonal, entries above
// the diagonal are scratch (0).
template <typename T, int D, bool ANISO>
__device__ __forceinline__ void grp_assemble(T (&a)[kGrp], const uint32_t (&x)[D],
                                             const uint32_t* xc, int K, int r, T scale,
                                             const TabEnt<T>* tab, const uint16_t* acc,
                                             const TabParams<T>& P, const AnisoArgs<T>& an) {
    const bool real = r < K || r == kGrpPt;
    const T diag = ANISO ? aniso_lookup(T(0), T(0), an) : P.v0;
#pragma unroll
    for (int c = 0; c < kGrp - 1; ++c) {
        T v = T(0);
        if (c < K) {  // a real column: its pairs with the real rows below it
            uint32_t y[D];
            grp_coords<D>(y, xc, c);
            if (c < r && real) {
                if (ANISO) v = aniso_pair<T, D>(x, y, scale, an);
                else v = cov_lookup(radius<T>(sqdist<D>(x, y), scale), tab, acc, P);
            }
        }
        a[c] = c == r ? (real ? diag : T(1)) : v;
    }
    a[kGrpPt] = r == kGrpPt ? diag : T(0);
}

// chol_lower! (src/linalg.jl:38-73) on the rows of the group; xv: the group's exchange area.
// rd (LDS): RN(1 / L[j][j]) by column, with which the column and every later division by L[j][j]
// take div_rcp (the IEEE quotient). Returns L[31][31] (the point's conditional standard
// deviation), group-uniform.
template <typename T>
__device__ __forceinline__ T grp_cholesky(T (&a)[kGrp], T* xv, T* rd, int K, int r, bool hi) {
    const T pivmin = num<T>::eps() * gbcast(a[0], 0, hi);
    const T dmin = num<T>::sqrt(pivmin);
    T col[kGrp];
#pragma unroll
    for (int j = 0; j < kGrp; ++j) {
        if (j < K || j == kGrpPt) {
            const T s = gbcast(a[j], j, hi);
            const bool ok = s > pivmin;  // false for NaN, as in the reference
            const T d = ok ? num<T>::sqrt(s) : dmin;
            const T y = rcp_rn(d);
            if (r == 0) rd[j] = y;
            const T q = div_rcp(a[j], d, y);
            a[j] = r == j ? d : (r > j ? (ok ? q : T(0)) : a[j]);
            if (j < kGrpPt) {
                xv[r] = a[j];
                wave_sync_lds();
                lds_tail(col, xv, j + 1);
#pragma unroll
                for (int c = 0; c < kGrp; ++c)
                    if (c > j) a[c] = num<T>::fma(-a[j], col[c], a[c]);
                __builtin_amdgcn_wave_barrier();
            }
        }
    }
    return gbcast(a[kGrpPt], kGrpPt, hi);
}

// mean_vec_solve! (src/linalg.jl:85-103): x_i = (L[P][i] - sum_{j>i} L[j][i] x_j) / L[i][i] for
// i = k-1 .. 0 (P the point's row), the sum in increasing j, from column i of L put in LDS;
// x_i = 0 where L[i][i] is at the clamp floor. Group-uniform; lane i receives x_i. xs (LDS,
// optional): every x_i by index (0 for the padding rows).
template <typename T>
__device__ __forceinline__ T grp_mean_vec(const T (&a)[kGrp], int K, int r, bool hi, T* xv,
                                          const T* rd, T* xs_out) {
    const T pivfloor = T(1.5) * num<T>::sqrt(num<T>::eps()) * gbcast(a[0], 0, hi);
    T xs[kGrp - 1];
    T col[kGrp];
    T mine = T(0);
#pragma unroll
    for (int i = kGrp - 2; i >= 0; --i) {
        T xi = T(0);
        if (i < K) {
            xv[r] = a[i];
            wave_sync_lds();
            lds_tail(col, xv, i);
            T s = col[kGrpPt];
#pragma unroll
            for (int j = 0; j < kGrp - 1; ++j)
                if (j > i) s = num<T>::fma(-col[j], xs[j], s);
            const T d = col[i];
            xi = d > pivfloor ? div_rcp(s, d, rd[i]) : T(0);
            mine = r == i ? xi : mine;
            __builtin_amdgcn_wave_barrier();
        }
        xs[i] = xi;
        if (xs_out && r == 0) xs_out[i] = xi;
    }
    return mine;
}

// Forward substitution L[0:k,0:k] zbar = z0 (z0 of row r in lane r), in the reference's order:
// at step i every lane runs the chain of its own row over p < i, and lane i's is zbar_i.
// GUARD: zero where the pivot is at the clamp floor (as mean_vec_solve! does). Lane i receives
// zbar_i.
template <typename T, bool GUARD>
__device__ __forceinline__ T grp_zbar(const T (&a)[kGrp], T z0, int K, int r, bool hi,
                                      const T* rd) {
    const T pivfloor = T(1.5) * num<T>::sqrt(num<T>::eps()) * gbcast(a[0], 0, hi);
    T zs[kGrp - 1];
    T zm = T(0);
#pragma unroll
    for (int i = 0; i < kGrp - 1; ++i) {
        T zi = T(0);
        if (i < K) {
            T t = z0;
#pragma unroll
            for (int p = 0; p < kGrp - 1; ++p)
                if (p < i) t = t - a[p] * zs[p];
            const T ti = gbcast(t, i, hi);
            const T dii = gbcast(a[i], i, hi);
            const T q = div_rcp(ti, dii, rd[i]);
            zi = GUARD ? (dii > pivfloor ? q : T(0)) : q;
            zm = r == i ? zi : zm;
        }
        zs[i] = zi;
    }
    return zm;
}

// lc[i] = L[i][r] for i >= r and 0 above the diagonal (column r of L), four columns at a time
// through LDS.
template <typename T>
__device__ __forceinline__ void grp_columns(const T (&a)[kGrp], T (&lc)[kGrp], T* xv, int r) {
    constexpr int S = kGrp + 16 / (int)sizeof(T);  // row stride: the four rows in distinct banks
#pragma unroll
    for (int i = 0; i < kGrp; ++i) lc[i] = T(0);
#pragma unroll
    for (int q = 0; q < kGrp / 4; ++q) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int c = 4 * q + u;
            xv[u * S + r] = c <= r ? a[c] : T(0);
        }
        wave_sync_lds();
        if ((r >> 2) == q) lds_tail(lc, xv + (r & 3) * S, 0);
        __builtin_amdgcn_wave_barrier();
    }
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
    __shared__ __align__(16) uint32_t s_xc[kWidePts][kGrp * 4];
    __shared__ __align__(16) T s_rd[kWidePts][kGrp];
    __shared__ __align__(16) T s_xv[kWidePts][kWideXch];
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
    const int lane = threadIdx.x & 63, r = lane & (kGrp - 1);
    const bool hi = lane >= kGrp;
    const int grp = threadIdx.x >> 5;
    uint32_t* xc = s_xc[grp];
    T* rd = s_rd[grp];
    T* xv = s_xv[grp];
    double lsum = 0.0;
    const int64_t stride = (int64_t)gridDim.x * kWidePts;
    auto points = [&](const AnisoArgs<T>& av) __attribute__((always_inline)) {
    for (int64_t b = (int64_t)blockIdx.x * kWidePts + 2 * (threadIdx.x >> 6); b < M; b += stride) {
        const bool live = b + hi < M;
        const int64_t m = live ? b + hi : M - 1;
        uint32_t x[D];
        const int32_t nb = grp_gather<D>(x, xc, coords, nbr, M, m, n0, K, r, nbr64);
        T a[kGrp];
        grp_assemble<T, D, ANISO>(a, x, xc, K, r, scale, s_tab, s_acc, P, av);
        const T s = grp_cholesky(a, xv, rd, K, r, hi);
        if (mode & F_TERMS) {
            const T t = num<T>::log(s);
            if (live && r == 0) {
                if (terms) terms[m] = t;
                lsum += (double)t;
            }
        }
        if (mode & (F_MV | F_INV)) {
            const T xm = grp_mean_vec(a, K, r, hi, xv, rd, (T*)nullptr);
            if (mode & F_MV) {
                if (live && r < K) mv[m * K + r] = xm;
                if (live && r == 0) sd[m] = s;
            }
            if (mode & F_INV) {  // src/kernels.jl:48-55: the mean in neighbour order
                xv[r] = r < K ? xm * values[nb] : T(0);
                wave_sync_lds();
                T pv[kGrp];
                lds_tail(pv, xv, 0);
                T mean = T(0);
#pragma unroll
                for (int j = 0; j < kGrp - 1; ++j) mean = mean + pv[j];  // padding: + (+0)
                if (live && r == 0) xi_out[m] = (values[n0 + m] - mean) / s;
                __builtin_amdgcn_wave_barrier();
            }
        }
    }
    };
    // staged axes (the whole workgroup stages them) are read from LDS on that side only
    if (ANISO && an.lds != 0) points(aniso_stage_lds(an, smem));
    else points(an);
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
__global__ void __launch_bounds__(kWideBlock) __attribute__((amdgpu_waves_per_eu(2)))
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
    __shared__ __align__(16) uint32_t s_xc[kWidePts][kGrp * 4];
    __shared__ __align__(16) T s_sv[kWidePts][2 * kGrp];
    __shared__ __align__(16) T s_xv[kWidePts][kWideXch];
    if (!TG) {
        if (!PTS)
            for (int i = threadIdx.x; i < P.nb; i += blockDim.x) s_hist[i] = 0.0;
        stage_table(s_tab, s_acc, g_tab, g_acc, P);
    }

    const int lane = threadIdx.x & 63, r = lane & (kGrp - 1);
    const bool hi = lane >= kGrp;
    const int grp = threadIdx.x >> 5;
    uint32_t* xc = s_xc[grp];
    T* xs = s_sv[grp];         // seeds: x (mean vector); the loop: sbar by row
    T* rd = s_sv[grp] + kGrp;  // RN(1 / L[j][j]) by column
    T* xv = s_xv[grp];
    const AnisoArgs<T> no_aniso{};
    double ssum = 0.0;
    const int64_t stride = (int64_t)gridDim.x * kWidePts;
    for (int64_t b = (int64_t)blockIdx.x * kWidePts + 2 * (threadIdx.x >> 6); b < M; b += stride) {
        const bool live = b + hi < M;
        const int64_t m = live ? b + hi : M - 1;
        uint32_t x[D];
        const int32_t nb = grp_gather<D>(x, xc, coords, nbr, M, m, n0, K, r, nullptr);
        T a[kGrp];
        grp_assemble<T, D, false>(a, x, xc, K, r, scale, s_tab, s_acc, P, no_aniso);
        const T s = grp_cholesky(a, xv, rd, K, r, hi);

        // ---- seeds: bc[i] = Lbar[i][r] ----
        T lc[kGrp], bc[kGrp];
        if (SEED == P_LOGDET) {
            // src/linalg.jl:140-146 with seed 1; the term itself for the fused logdet.
            if (live && r == 0) ssum += (double)num<T>::log(s);
            grp_columns(a, lc, xv, r);
            const T seed = T(1) / s;
#pragma unroll
            for (int i = 0; i < kGrp; ++i) bc[i] = T(0);
            bc[kGrpPt] = r == kGrpPt ? seed : T(0);
        } else {
            const T xm = grp_mean_vec(a, K, r, hi, xv, rd, xs);
            const T vnb = r < K ? v[nb] : T(0);
            T seed, z0;
            if (SEED == P_INVLOSS) {
                // src/kernels_adjoint.jl:183-211 (no @fastmath there): the mean in neighbour order
                xv[r] = r < K ? xm * vnb : T(0);
                wave_sync_lds();
                T pv[kGrp];
                lds_tail(pv, xv, 0);
                T mean = T(0);
#pragma unroll
                for (int j = 0; j < kGrp - 1; ++j) mean = mean + pv[j];
                __builtin_amdgcn_wave_barrier();
                const T xim = (v[n0 + m] - mean) / s;
                if (live && r == 0) ssum += (double)(xim * xim / T(2));
                seed = -xim * xim / s;
                z0 = -xim * vnb / s;
            } else {
                // src/kernels_adjoint.jl:509-538.
                const T vbp = vb[n0 + m];
                seed = vbp * xi[n0 + m];
                z0 = vbp * vnb;
            }
            // unguarded for the inverse loss, guarded like mean_vec_solve! for generate_grad_vals
            const T zm = SEED == P_INVLOSS ? grp_zbar<T, false>(a, z0, K, r, hi, rd)
                                           : grp_zbar<T, true>(a, z0, K, r, hi, rd);
            grp_columns(a, lc, xv, r);
            wave_sync_lds();
            T xsv[kGrp];
            lds_tail(xsv, xs, 0);
            // Lbar[P][j] = zbar_j; Lbar[j][i] = -(zbar_i x_j) for i <= j < k; Lbar[P][P] = seed.
#pragma unroll
            for (int i = 0; i < kGrp - 1; ++i) bc[i] = (i < K && r <= i) ? T(0) - zm * xsv[i] : T(0);
            bc[kGrpPt] = r < K ? T(0) + zm : (r == kGrpPt ? seed : T(0));
        }

        // ---- chol_pullback! (src/linalg.jl:112-137), columns on lanes ----
        double gpt[D];  // P_PTS: this row's point gradient
#pragma unroll
        for (int d = 0; d < D; ++d) gpt[d] = 0.0;
        const bool real_r = r < K || r == kGrpPt;
        T* pb = xv;              // column j of Lbar by row
        T* pl = xv + kGrp;       // column j of L by row
        T* tv = xv + 2 * kGrp;   // (tbar_i, Lbar[i][j] L[i][j] / L[j][j]) by row i
        static_for<0, kGrp>([&](auto J) __attribute__((always_inline)) {
            constexpr int j = kGrp - 1 - decltype(J)::value;
            if (j < K || j == kGrpPt) {
                if (r == j) {
#pragma unroll
                    for (int i = 0; i < kGrp; ++i) {
                        if (i >= j) {
                            pb[i] = bc[i];
                            pl[i] = lc[i];
                        }
                    }
                }
                wave_sync_lds();
                const T lbjj = pb[j], ljj = pl[j], y = rd[j];
                const bool row = r > j && real_r;
                const T lb = row ? pb[r] : T(0);
                const T lij = row ? pl[r] : T(0);
                const T tbar = div_rcp(lb, ljj, y);
                const T qv = div_rcp(lb * lij, ljj, y);
                // Abar[r][j] = tbar through the lookup weights (src/kernels_adjoint.jl:47-74), or
                // through k'(r) dr/dx into points r and j (src/kernels_adjoint.jl:223-252)
                uint32_t xj[D];
                grp_coords<D>(xj, xc, j);
                if (PTS) {
                    T c[D];
#pragma unroll
                    for (int d = 0; d < D; ++d) c[d] = T(0);
                    if (row) (void)pair_pts<T, D>(x, xj, tbar, scale, s_tab, s_acc, P, c);
#pragma unroll
                    for (int d = 0; d < D; ++d) {
                        gpt[d] += (double)c[d];
                        const double cs = grp_sum((double)c[d]);
                        if (r == j) gpt[d] -= cs;
                    }
                } else if (row && live) {
                    const T rr = radius<T>(sqdist<D>(x, xj), scale);
                    T wlo, whi;
                    const int lo = cov_weights(rr, s_tab, s_acc, P, wlo, whi);
                    atomicAdd(&s_hist[lo], (double)(tbar * wlo));
                    atomicAdd(&s_hist[lo + 1], (double)(tbar * whi));
                }
                tv[2 * r] = tbar;
                tv[2 * r + 1] = qv;
                wave_sync_lds();
                T t = lbjj;  // Lbar[j][j]
#pragma unroll
                for (int i = kGrp - 1; i >= 0; --i) {
                    if (i > j) {
                        const T tb = tv[2 * i];
                        t = t - tv[2 * i + 1];
                        bc[i] = num<T>::fma(-tb, lc[j], bc[i]);  // Lbar[i][r], r < j
                        bc[j] = num<T>::fma(-tb, lc[i], bc[j]);  // Lbar[j][r], r < j
                    }
                }
                const T sbar = div_rcp(t, T(2) * ljj, y * T(0.5));
                if (r == 0) xs[j] = sbar;
                bc[j] = num<T>::fma(-(T(2) * sbar), lc[j], bc[j]);
                __builtin_amdgcn_wave_barrier();
            } else if (r == 0) {
                xs[j] = T(0);
            }
        });
        if (PTS) {
            if (live && real_r) {
                const int64_t gp = r < K ? (int64_t)nb : n0 + m;
#pragma unroll
                for (int d = 0; d < D; ++d) atomicAdd(&hist_partial[gp * D + d], gpt[d]);
            }
        } else {
            // diagonal of Abar: one add per row into bin 0, summed in row order
            wave_sync_lds();
            T sb[kGrp];
            lds_tail(sb, xs, 0);
            T diag = T(0);
#pragma unroll
            for (int j = 0; j < kGrp; ++j) diag += sb[j];  // padding rows: + (+0)
            if (live && r == 0) atomicAdd(&s_hist[0], (double)diag);
        }
        __builtin_amdgcn_wave_barrier();
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
