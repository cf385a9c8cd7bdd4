// ggp_point_kernels.h — per-point kernels of the Vecchia refinement for gfx950.
//
// Kernel map (reference kernel each replaces):
//   k_factor<MV>      refine_meanvec_std_kernel! (src/kernels.jl:61-78): mean_vec and std for
//                     ALL refined points in one launch, independent of the field values
//   k_factor<TERMS>   refine_logdet_kernel! (src/kernels.jl:25-35) + the host sum (src/api.jl:24-27)
//   k_factor<INV>     refine_inv_kernel! (src/kernels.jl:37-56)
//   k_sweep_fwd       refine_apply_fused_kernel! (src/kernels.jl:101-119) split: the factor
//                     pass above + this gather-only level apply
//   k_sweep_rev       refine_reverse_apply_fused_kernel! (src/kernels_adjoint.jl:453-474) as a
//                     deterministic gather over the reverse neighbour list instead of atomics
//   k_pullback<...>   refine_logdet_grad_hist_kernel! / refine_logdet_and_grad_hist_kernel! /
//                     refine_inv_loss_grad_hist_kernel! / generate_grad_vals_rev_kernel!
//                     (src/kernels_adjoint.jl:80-221, 484-553): the per-point Cholesky pullback,
//                     with the d_vals histogram accumulated in f64 in LDS and flushed per
//                     workgroup to a partials buffer (no global atomics)
//
// Layout in HBM: coords point-major uint32 (D per point); neighbours int32 SoA nbr[j*M + m];
// mean_vec SoA mv[j*M + m]; std sd[m]; field arrays in tree order.
//
// Included only by ggp_inst.hip, which is compiled once per (element type, k) so the heavy,
// fully unrolled instantiations build in parallel; ggp_kernels.hip dispatches to them.
#pragma once
#include "ggp_internal.h"


namespace ggp {

// Dynamic LDS layout shared by the table-using kernels: [TabEnt x (nb-1)] [uint16 x (U+1)]
// [double hist x nb (adjoints only)].
template <typename T>
__host__ __device__ inline size_t tab_bytes(int nb, int ucells) {
    size_t a = (size_t)(nb - 1) * sizeof(TabEnt<T>);
    size_t b = ((size_t)(ucells + 1) * sizeof(uint16_t) + 15) & ~(size_t)15;
    return a + b;
}

// Block-wide double sum of one value per thread; result valid in thread 0.
__device__ inline double block_sum(double v, double* s_red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_down(v, o, 64);
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    if (l == 0) s_red[w] = v;
    __syncthreads();
    double t = 0.0;
    if (threadIdx.x == 0)
        for (int i = 0; i < (int)(blockDim.x >> 6); ++i) t += s_red[i];
    return t;
}

// ---- factor pass ----------------------------------------------------------------------------
// ANISO: the covariance comes from the anisotropic grid (src/aniso.jl) instead of (bins, vals).
template <typename T, int K, int D, int MODE, bool ANISO>
__global__ void __launch_bounds__(kBlock)
k_factor(const uint32_t* __restrict__ coords, const int32_t* __restrict__ nbr, int64_t M,
         int64_t n0, T scale, const TabEnt<T>* __restrict__ g_tab,
         const uint16_t* __restrict__ g_acc, const TabParams<T>* __restrict__ Pp, T* __restrict__ mv,
         T* __restrict__ sd, T* __restrict__ terms, double* __restrict__ partial,
         const T* __restrict__ values, T* __restrict__ xi_out, AnisoArgs<T> an) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ double s_red[kBlock / 64];
    TabParams<T> P{};
    TabEnt<T>* s_tab = nullptr;
    uint16_t* s_acc = nullptr;
    if (!ANISO) {
        P = *Pp;
        s_tab = reinterpret_cast<TabEnt<T>*>(smem);
        s_acc = reinterpret_cast<uint16_t*>(smem + (size_t)(P.nb - 1) * sizeof(TabEnt<T>));
        stage_table(s_tab, s_acc, g_tab, g_acc, P);
    }

    double lsum = 0.0;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t m = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; m < M; m += stride) {
        Block<T, K, D> blk;
        int32_t nb[K];
        blk.gather(coords, nbr, M, m, n0, nb);
        if (ANISO) blk.assemble_aniso(scale, an);
        else blk.assemble(scale, s_tab, s_acc, P);
        blk.cholesky();
        const T s = blk.stddev();
        if (MODE & F_TERMS) {
            const T t = num<T>::log(s);
            if (terms) terms[m] = t;
            lsum += (double)t;
        }
        if (MODE & (F_MV | F_INV)) {
            T x[K];
            blk.mean_vec(x);
            if (MODE & F_MV) {
#pragma unroll
                for (int j = 0; j < K; ++j) mv[(int64_t)j * M + m] = x[j];
                sd[m] = s;
            }
            if (MODE & F_INV) {  // src/kernels.jl:48-55
                T mean = T(0);
#pragma unroll
                for (int j = 0; j < K; ++j) mean += x[j] * values[nb[j]];
                xi_out[m] = (values[n0 + m] - mean) / s;
            }
        }
    }
    if (MODE & F_TERMS) {
        const double t = block_sum(lsum, s_red);
        if (threadIdx.x == 0) partial[blockIdx.x] = t;
    }
}

// ---- level sweeps ---------------------------------------------------------------------------
// Forward apply of one depth level (src/kernels.jl:113-118): std*xi first, then + mv_j*v_j in
// neighbour order, each product rounded before the add (that code is not under @fastmath).
// TWO_PASS: the anisotropic apply order (src/kernels.jl:89-92): sum mv_j*v_j first, then
// + std*xi.
// K = 0: k is the run-time Krt (the wavefront-per-point path); otherwise Krt == K.
template <typename T, int K, bool TWO_PASS>
__global__ void __launch_bounds__(kBlock)
k_sweep_fwd(T* __restrict__ v, const T* __restrict__ xi, int64_t xi_off,
            const T* __restrict__ mv, const T* __restrict__ sd, const int32_t* __restrict__ nbr,
            int64_t M, int64_t n0, int64_t m_lo, int64_t len, int Krt) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= len) return;
    const int64_t m = m_lo + t;
    if constexpr (K == 0) {
        T acc = TWO_PASS ? T(0) : sd[m] * xi[xi_off + m];
        for (int j = 0; j < Krt; ++j)
            acc = acc + mv[(int64_t)j * M + m] * v[nbr[(int64_t)j * M + m]];
        v[n0 + m] = TWO_PASS ? acc + sd[m] * xi[xi_off + m] : acc;
        return;
    }
    constexpr int KA = K > 0 ? K : 1;
    int32_t nb[KA];
    T w[KA];
#pragma unroll
    for (int j = 0; j < K; ++j) {
        nb[j] = nbr[(int64_t)j * M + m];
        w[j] = mv[(int64_t)j * M + m];
    }
    if (TWO_PASS) {
        T acc = T(0);
#pragma unroll
        for (int j = 0; j < K; ++j) acc = acc + w[j] * v[nb[j]];
        v[n0 + m] = acc + sd[m] * xi[xi_off + m];
    } else {
        T acc = sd[m] * xi[xi_off + m];
#pragma unroll
        for (int j = 0; j < K; ++j) acc = acc + w[j] * v[nb[j]];
        v[n0 + m] = acc;
    }
}

// Reverse sweep of one depth level, positions [q_lo, q_hi): vb[q] = vbar[q] + sum over the
// consumers (p, j) of q of mv_j(p)*vb[p], the consumers listed by decreasing p — exactly the
// order in which the reference's serial host sweep (src/grad.jl:433-445) adds them — and
// xg[q] = std_q*vb[q] for refined q. Every consumer lies in a later level, so vb[p] is final.
//
// A group of G lanes (G a power of two <= 64, sized to the level's largest fan-in) serves one
// point: each lane loads one consumer's product mv*vb per round, so the dependent memory round
// trips per point drop from the fan-in to fan-in/G; the products are then added one by one in
// list order (shuffled from their lanes), which keeps every rounding of the serial sum.
template <typename T, int K>
__global__ void __launch_bounds__(kBlock)
k_sweep_rev(T* __restrict__ vb, const T* __restrict__ vbar, T* __restrict__ xg,
            const T* __restrict__ mv, const T* __restrict__ sd,
            const int64_t* __restrict__ rev_ptr, const uint32_t* __restrict__ rev,
            int64_t M, int64_t n0, int64_t q_lo, int64_t q_hi, int G, int Krt) {
    const uint32_t KK = K > 0 ? (uint32_t)K : (uint32_t)Krt;
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int lane = threadIdx.x & 63;
    const int gl = lane & (G - 1);          // lane within the group
    const int gbase = lane - gl;            // first lane of the group
    const int64_t q = q_lo + tid / G;
    const bool live = q < q_hi;
    int64_t e0 = 0, cnt = 0;
    T acc = T(0);
    if (live) {
        e0 = rev_ptr[q];
        cnt = rev_ptr[q + 1] - e0;
        acc = vbar[q];
    }
    for (int64_t base = 0; base < cnt; base += G) {
        T prod = T(0);
        if (base + gl < cnt) {
            const uint32_t c = rev[e0 + base + gl];
            const uint32_t m = c / KK, j = c - m * KK;
            prod = mv[(int64_t)j * M + m] * vb[n0 + m];
        }
        const int64_t take = cnt - base < G ? cnt - base : G;
        for (int i = 0; i < take; ++i) acc = acc + __shfl(prod, gbase + i, 64);
    }
    if (live && gl == 0) {
        vb[q] = acc;
        if (xg && q >= n0) xg[q] = sd[q - n0] * acc;
    }
}

// ---- adjoint pullback -----------------------------------------------------------------------
// Histogram scatter of one point's Abar through the lookup weights (src/kernels_adjoint.jl:47-74).
template <typename T, int K, int D>
__device__ inline void scatter_hist(double* hist, const Block<T, K, D>& blk,
                                    const T (&Abar)[(K + 1) * (K + 2) / 2], T scale,
                                    const TabEnt<T>* tab, const uint16_t* acc,
                                    const TabParams<T>& P) {
    constexpr int N = K + 1;
    T diag = T(0);
#pragma unroll
    for (int a = 0; a < N; ++a) diag += Abar[tri(a, a)];
    atomicAdd(&hist[0], (double)diag);
#pragma unroll
    for (int a = 1; a < N; ++a)
#pragma unroll
        for (int b = 0; b < a; ++b) {
            const T r = radius<T>(sqdist<D>(blk.jc[a], blk.jc[b]), scale);
            T wlo, whi;
            const int lo = cov_weights(r, tab, acc, P, wlo, whi);
            const T g = Abar[tri(a, b)];
            atomicAdd(&hist[lo], (double)(g * wlo));
            atomicAdd(&hist[lo + 1], (double)(g * whi));
        }
}

template <typename T, int K, int D, int MODE>
__global__ void __launch_bounds__(kBlock)
k_pullback(const uint32_t* __restrict__ coords, const int32_t* __restrict__ nbr, int64_t M,
           int64_t n0, T scale, const TabEnt<T>* __restrict__ g_tab,
           const uint16_t* __restrict__ g_acc, const TabParams<T>* __restrict__ Pp,
           const T* __restrict__ v,     // INVLOSS: values (tree order); GENVALS: forward field
           const T* __restrict__ xi,    // GENVALS: xi (tree order)
           const T* __restrict__ vb,    // GENVALS: field cotangent after the reverse sweep
           double* __restrict__ hist_partial, double* __restrict__ scalar_partial) {
    const TabParams<T> P = *Pp;
    extern __shared__ __align__(16) unsigned char smem[];
    TabEnt<T>* s_tab = reinterpret_cast<TabEnt<T>*>(smem);
    uint16_t* s_acc = reinterpret_cast<uint16_t*>(smem + (size_t)(P.nb - 1) * sizeof(TabEnt<T>));
    double* s_hist = reinterpret_cast<double*>(smem + tab_bytes<T>(P.nb, P.ucells));
    __shared__ double s_red[kBlock / 64];
    for (int i = threadIdx.x; i < P.nb; i += blockDim.x) s_hist[i] = 0.0;
    stage_table(s_tab, s_acc, g_tab, g_acc, P);

    constexpr int N = K + 1;
    constexpr int NT = N * (N + 1) / 2;
    double ssum = 0.0;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t m = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; m < M; m += stride) {
        Block<T, K, D> blk;
        int32_t nb[K];
        blk.gather(coords, nbr, M, m, n0, nb);
        blk.assemble(scale, s_tab, s_acc, P);
        blk.cholesky();
        const T s = blk.stddev();
        T Lbar[NT], Abar[NT];
#pragma unroll
        for (int i = 0; i < NT; ++i) { Lbar[i] = T(0); Abar[i] = T(0); }
        if (MODE == P_LOGDET) {
            // src/linalg.jl:140-146 with seed 1; the term itself for the fused logdet.
            ssum += (double)num<T>::log(s);
            Lbar[tri(K, K)] = T(1) / s;
        } else {
            T x[K], zbar[K];
            blk.mean_vec(x);
            if (MODE == P_INVLOSS) {
                // src/kernels_adjoint.jl:183-211 (no @fastmath there).
                T mean = T(0);
#pragma unroll
                for (int j = 0; j < K; ++j) mean += x[j] * v[nb[j]];
                const T xim = (v[n0 + m] - mean) / s;
                ssum += (double)(xim * xim / T(2));
                Lbar[tri(K, K)] = -xim * xim / s;
#pragma unroll
                for (int j = 0; j < K; ++j) zbar[j] = -xim * v[nb[j]] / s;
#pragma unroll
                for (int i = 0; i < K; ++i) {
                    T t = zbar[i];
#pragma unroll
                    for (int p = 0; p < i; ++p) t -= blk.A[tri(i, p)] * zbar[p];
                    zbar[i] = t / blk.A[tri(i, i)];
                }
            } else {
                // src/kernels_adjoint.jl:509-538: seeds from vb[p], xi[p], v[neighbours], with
                // the forward substitution guarded like mean_vec_solve!.
                const T vbp = vb[n0 + m];
                Lbar[tri(K, K)] = vbp * xi[n0 + m];
                const T pivfloor = T(1.5) * num<T>::sqrt(num<T>::eps()) * blk.A[0];
#pragma unroll
                for (int j = 0; j < K; ++j) zbar[j] = vbp * v[nb[j]];
#pragma unroll
                for (int i = 0; i < K; ++i) {
                    T t = zbar[i];
#pragma unroll
                    for (int p = 0; p < i; ++p) t -= blk.A[tri(i, p)] * zbar[p];
                    zbar[i] = blk.A[tri(i, i)] > pivfloor ? t / blk.A[tri(i, i)] : T(0);
                }
            }
#pragma unroll
            for (int j = 0; j < K; ++j) {
                Lbar[tri(K, j)] += zbar[j];
#pragma unroll
                for (int i = 0; i <= j; ++i) Lbar[tri(j, i)] -= zbar[i] * x[j];
            }
        }
        chol_pullback<T, N>(Abar, Lbar, blk.A);
        scatter_hist<T, K, D>(s_hist, blk, Abar, scale, s_tab, s_acc, P);
    }
    __syncthreads();
    double* out = hist_partial + (size_t)blockIdx.x * P.nb;
    for (int i = threadIdx.x; i < P.nb; i += blockDim.x) out[i] = s_hist[i];
    if (scalar_partial) {
        const double t = block_sum(ssum, s_red);
        if (threadIdx.x == 0) scalar_partial[blockIdx.x] = t;
    }
}

static inline unsigned grid_for_pt(int64_t n) { return (unsigned)((n + kBlock - 1) / kBlock); }

template <typename T, int K>
void PointK<T, K>::factor(const Graph& g, const Table<T>& tb, int mode, T* mv, T* sd, T* terms,
                          double* partial, const T* values, T* xi_out, unsigned nblk,
                          hipStream_t st) {
    const bool aniso = tb.aniso.grid != nullptr;
    const size_t lds = aniso ? 0 : tab_bytes<T>(tb.P.nb, tb.P.ucells);
    const T scale = (T)g.scale;
#define GGP_FACTOR(DD, MODEV)                                                                  \
    do {                                                                                       \
        if (aniso)                                                                             \
            hipLaunchKernelGGL((k_factor<T, K, DD, MODEV, true>), dim3(nblk), dim3(kBlock), 0,  \
                               st, g.coords, g.nbr, g.M, g.n0, scale, tb.tab, tb.acc,           \
                               tb.params, mv, sd, terms, partial, values, xi_out, tb.aniso);    \
        else                                                                                   \
            hipLaunchKernelGGL((k_factor<T, K, DD, MODEV, false>), dim3(nblk), dim3(kBlock),    \
                               lds, st, g.coords, g.nbr, g.M, g.n0, scale, tb.tab, tb.acc,      \
                               tb.params, mv, sd, terms, partial, values, xi_out, tb.aniso);    \
    } while (0)
#define GGP_FACTOR_D(DD)                                                                       \
    switch (mode) {                                                                            \
        case F_MV: GGP_FACTOR(DD, F_MV); break;                                                \
        case F_TERMS: GGP_FACTOR(DD, F_TERMS); break;                                          \
        case F_INV: GGP_FACTOR(DD, F_INV); break;                                              \
        default: break;                                                                        \
    }
    switch (g.D) {
        case 2: GGP_FACTOR_D(2); break;
        case 3: GGP_FACTOR_D(3); break;
        case 4: GGP_FACTOR_D(4); break;
        default: break;
    }
#undef GGP_FACTOR_D
#undef GGP_FACTOR
}

template <typename T, int K>
void PointK<T, K>::pullback(const Graph& g, const Table<T>& tb, int mode, const T* v,
                            const T* xi, const T* vb, double* hist_partial,
                            double* scalar_partial, unsigned nblk, hipStream_t st) {
    const size_t lds = tab_bytes<T>(tb.P.nb, tb.P.ucells) + (size_t)tb.P.nb * sizeof(double);
    const T scale = (T)g.scale;
#define GGP_PULL(DD, MODEV)                                                                    \
    hipLaunchKernelGGL((k_pullback<T, K, DD, MODEV>), dim3(nblk), dim3(kBlock), lds, st,        \
                       g.coords, g.nbr, g.M, g.n0, scale, tb.tab, tb.acc, tb.params, v, xi, vb, \
                       hist_partial, scalar_partial)
#define GGP_PULL_D(DD)                                                                         \
    switch (mode) {                                                                            \
        case P_LOGDET: GGP_PULL(DD, P_LOGDET); break;                                          \
        case P_INVLOSS: GGP_PULL(DD, P_INVLOSS); break;                                        \
        case P_GENVALS: GGP_PULL(DD, P_GENVALS); break;                                        \
        default: break;                                                                        \
    }
    switch (g.D) {
        case 2: GGP_PULL_D(2); break;
        case 3: GGP_PULL_D(3); break;
        case 4: GGP_PULL_D(4); break;
        default: break;
    }
#undef GGP_PULL_D
#undef GGP_PULL
}

template <typename T, int K>
void PointK<T, K>::sweep_fwd(const Graph& g, T* v, const T* xi, int64_t xi_off, const T* mv,
                             const T* sd, int64_t m_lo, int64_t len, bool two_pass,
                             hipStream_t st) {
    if (two_pass)
        hipLaunchKernelGGL((k_sweep_fwd<T, K, true>), dim3(grid_for_pt(len)), dim3(kBlock), 0, st,
                           v, xi, xi_off, mv, sd, g.nbr, g.M, g.n0, m_lo, len, (int)g.K);
    else
        hipLaunchKernelGGL((k_sweep_fwd<T, K, false>), dim3(grid_for_pt(len)), dim3(kBlock), 0,
                           st, v, xi, xi_off, mv, sd, g.nbr, g.M, g.n0, m_lo, len, (int)g.K);
}

template <typename T, int K>
void PointK<T, K>::sweep_rev(const Graph& g, T* vb, const T* vbar, T* xg, const T* mv,
                             const T* sd, int64_t q_lo, int64_t q_hi, int G, hipStream_t st) {
    hipLaunchKernelGGL((k_sweep_rev<T, K>), dim3(grid_for_pt((q_hi - q_lo) * G)), dim3(kBlock), 0,
                       st, vb, vbar, xg, mv, sd, g.rev_ptr, g.rev, g.M, g.n0, q_lo, q_hi, G,
                       (int)g.K);
}

}  // namespace ggp
