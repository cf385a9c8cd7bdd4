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
// mean_vec point-major mv[m*k + j] (a consumer's k weights share a cache line: the reverse
// sweep gathers them by list entry m*k + j); std sd[m]; field arrays in tree order.
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
// The grid-stride loop of k_factor over the refined points; returns this lane's sum of the
// logdet terms. ONE: the single-step table search (P.steps <= 1).
template <typename T, int K, int D, int MODE, bool ANISO, bool ONE>
__device__ inline double factor_points(const uint32_t* __restrict__ coords,
                                       const int32_t* __restrict__ nbr, int64_t M, int64_t n0,
                                       T scale, const TabEnt<T>* s_tab, const uint16_t* s_acc,
                                       const TabParams<T>& P, T* __restrict__ mv,
                                       T* __restrict__ sd, T* __restrict__ terms,
                                       const T* __restrict__ values, T* __restrict__ xi_out,
                                       const AnisoArgs<T>& an,
                                       const int64_t* __restrict__ nbr64) {
    double lsum = 0.0;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t m = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; m < M; m += stride) {
        Block<T, K, D> blk;
        int32_t nb[K];
        blk.gather(coords, nbr, M, m, n0, nb, nbr64);
        if (ANISO) blk.assemble_aniso(scale, an);
        else blk.template assemble<ONE, true>(scale, s_tab, s_acc, P);
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
                for (int j = 0; j < K; ++j) mv[m * K + j] = x[j];
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
    return lsum;
}

// ANISO: the covariance comes from the anisotropic grid (src/aniso.jl) instead of (bins, vals).
// nbr64 (optional): the neighbours in the reference's layout (int64, point-major) instead of nbr.
template <typename T, int K, int D, int MODE, bool ANISO>
__global__ void __launch_bounds__(kBlock)
k_factor(const uint32_t* __restrict__ coords, const int32_t* __restrict__ nbr, int64_t M,
         int64_t n0, T scale, const TabEnt<T>* __restrict__ g_tab,
         const uint16_t* __restrict__ g_acc, const TabParams<T>* __restrict__ Pp, T* __restrict__ mv,
         T* __restrict__ sd, T* __restrict__ terms, double* __restrict__ partial,
         const T* __restrict__ values, T* __restrict__ xi_out, AnisoArgs<T> an,
         const int64_t* __restrict__ nbr64) {
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
    if (ANISO && an.lds != 0)  // axes staged: their reads are LDS reads
        lsum = factor_points<T, K, D, MODE, ANISO, true>(coords, nbr, M, n0, scale, s_tab, s_acc,
                                                         P, mv, sd, terms, values, xi_out,
                                                         aniso_stage_lds(an, smem), nbr64);
    else if (ANISO || P.steps <= 1)
        lsum = factor_points<T, K, D, MODE, ANISO, true>(coords, nbr, M, n0, scale, s_tab, s_acc,
                                                         P, mv, sd, terms, values,
                                                         xi_out, an, nbr64);
    else
        lsum = factor_points<T, K, D, MODE, ANISO, false>(coords, nbr, M, n0, scale, s_tab, s_acc,
                                                          P, mv, sd, terms, values,
                                                          xi_out, an, nbr64);
    if (MODE & F_TERMS) {
        const double t = block_sum(lsum, s_red);
        if (threadIdx.x == 0) partial[blockIdx.x] = t;
    }
}


// ---- level sweeps: one persistent launch per sweep ----------------------------------------
// Every value a sweep produces starts as a pending marker (a NaN no arithmetic produces) and is
// published once, with an agent-scope store. A reader takes its inputs with plain loads and
// polls with agent-scope loads only those it still sees pending: a published value never
// changes, so a plain load returns either the marker or the final value.
//
// Workgroups take chunks from an atomic ticket counter; the chunks lie inside one level each
// and are listed in topological order (a point's inputs sit in strictly earlier chunks), so a
// chunk only waits for chunks already taken by running workgroups, whatever the residency,
// and no wavefront ever waits for a lane of its own. Every wait is bounded: past
// kSweepSpinLimit polls it sets bit 2 of *err and goes on, so every workgroup exits; the host
// reports that as an error. The arithmetic per point is the per-level kernels', unchanged.
// Next chunk for the workgroup; the value is made wave-uniform for the compiler (readfirstlane)
// so the loop test is a uniform branch and the loop keeps its shape.
__device__ inline int sweep_next(int* ticket, int* s_c) {
    __syncthreads();
    if (threadIdx.x == 0) *s_c = atomicAdd(ticket, 1);
    __syncthreads();
    return __builtin_amdgcn_readfirstlane(*s_c);
}

// Forward apply (src/kernels.jl:113-118): std*xi first, then + mv_j*v_j in neighbour order, each
// product rounded before the add (that code is not under @fastmath). TWO_PASS: the anisotropic
// order (src/kernels.jl:89-92): sum mv_j*v_j first, then + std*xi. K = 0: k is the run-time Krt.
template <typename T, int K, bool TWO_PASS>
__global__ void __launch_bounds__(kBlock)
k_sweep_fwd(T* __restrict__ v, const T* __restrict__ xi, int64_t xi_off,
            const T* __restrict__ mv, const T* __restrict__ sd, const int32_t* __restrict__ nbr,
            int64_t M, int64_t n0, int Krt, const int4* __restrict__ chunks, int nchunks,
            int* __restrict__ ticket, int* __restrict__ err, T* __restrict__ out,
            const int32_t* __restrict__ oidx) {
    __shared__ int s_c;
    constexpr int KA = K > 0 ? K : 1;
    for (int c = sweep_next(ticket, &s_c); c < nchunks; c = sweep_next(ticket, &s_c)) {
        const int4 ch = chunks[c];
        if ((int)threadIdx.x >= ch.y) continue;
        const int64_t m = ch.x + threadIdx.x;
        const T s_xi = sd[m] * xi[xi_off + m];
        T acc = TWO_PASS ? T(0) : s_xi;
        if constexpr (K == 0) {
            constexpr int B = 8;
            for (int j0 = 0; j0 < Krt; j0 += B) {
                int64_t q[B];
                bool live[B];
                T w[B], x[B];
#pragma unroll
                for (int u = 0; u < B; ++u) {
                    live[u] = j0 + u < Krt;
                    q[u] = live[u] ? nbr[(int64_t)(j0 + u) * M + m] : 0;
                    w[u] = live[u] ? mv[m * Krt + j0 + u] : T(0);
                }
                sweep_read_all<T, B>(x, v, q, live, err);
#pragma unroll
                for (int u = 0; u < B; ++u)
                    if (live[u]) acc = acc + w[u] * x[u];
            }
        } else {
            int64_t q[KA];
            bool live[KA];
            T w[KA], x[KA];
#pragma unroll
            for (int j = 0; j < K; ++j) {
                q[j] = nbr[(int64_t)j * M + m];
                w[j] = mv[m * K + j];
                live[j] = true;
            }
            sweep_read_all<T, KA>(x, v, q, live, err);
#pragma unroll
            for (int j = 0; j < K; ++j) acc = acc + w[j] * x[j];
        }
        if (TWO_PASS) acc = acc + s_xi;
        sweep_publish(v + n0 + m, acc);
        if (out) out[oidx ? (int64_t)oidx[n0 + m] : n0 + m] = acc;  // null map: identity
    }
}

// Reverse gather (the transpose of the forward apply): vb[q] = vbar[q] + sum over the consumers
// (p, j) of q of mv_j(p)*vb[p], the consumers listed by decreasing p — exactly the order in
// which the reference's serial host sweep (src/grad.jl:433-445) adds them — and
// xg[q] = std_q*vb[q] for refined q.
// A point feeds about k*ln(N/q) later points, so early levels have long lists and few points.
// Each chunk therefore gives a point 2^lg lanes (lg chosen per chunk when the graph is built so
// that a lane holds at most kRevSlots entries): the lanes fetch their entries and the consumer
// values together (one round trip for the list, one for the values), form the products, and
// the point's first lane adds them in list order from LDS, which keeps every rounding of the
// serial sum. The list layout is lane-major per chunk, so every fetch is coalesced. The next
// chunk's ticket is taken while this one runs.
template <typename T, int K>
__global__ void __launch_bounds__(kBlock)
k_sweep_rev(T* __restrict__ vb, const T* __restrict__ vbar, T* __restrict__ xg,
            const T* __restrict__ mv, const T* __restrict__ sd, const uint32_t* __restrict__ rcnt,
            const uint32_t* __restrict__ rev, int64_t M, int64_t n0, int Krt,
            const int4* __restrict__ chunks, int nchunks, int* __restrict__ ticket,
            int* __restrict__ err, T* __restrict__ xout, const int32_t* __restrict__ oidx) {
    constexpr int B = kRevSlots;
    __shared__ int s_c;
    __shared__ T s_prod[B][kBlock];
    const int tid = threadIdx.x;
    const uint32_t KK = K > 0 ? (uint32_t)K : (uint32_t)Krt;
    if (tid == 0) s_c = atomicAdd(ticket, 1);
    __syncthreads();
    int c = __builtin_amdgcn_readfirstlane(s_c);
    while (c < nchunks) {
        const int4 ch = chunks[c];
        __syncthreads();  // every lane has read s_c
        int next = 0;
        if (tid == 0) next = atomicAdd(ticket, 1);
        const int lg = ch.y >> 16, np = ch.y & 0xffff, nslots = ch.w;
        const int i = tid >> lg, sub = tid & ((1 << lg) - 1);
        const bool pt = i < np;
        const int64_t q = (int64_t)ch.x + i;
        const int cnt = pt ? (int)rcnt[q] : 0;
        T acc = (pt && sub == 0) ? vbar[q] : T(0);
        // std of the point, fetched with the list counts (off the chunk's tail)
        const T sdq = (xg && pt && sub == 0 && q >= n0) ? sd[q - n0] : T(0);
        for (int t0 = 0; t0 < nslots; t0 += B) {
            int64_t p[B];
            bool live[B];
            T w[B], x[B];
#pragma unroll
            for (int u = 0; u < B; ++u) {
                const int t = t0 + u;
                live[u] = pt && ((t << lg) + sub) < cnt;
                // the chunk owns nslots * kBlock entries from ch.z * kBlock (unused ones hold
                // kRevNone), so the entries are fetched with the counts, not after them; live
                // implies t < nslots (a point's count is at most nslots << lg)
                const uint32_t e = t < nslots ? rev[((int64_t)ch.z + t) * kBlock + tid] : kRevNone;
                const uint32_t m = e / KK, j = e - m * KK;
                p[u] = n0 + m;
                w[u] = live[u] ? mv[(int64_t)m * KK + j] : T(0);
            }
            sweep_read_all<T, B>(x, vb, p, live, err);
            if (lg == 0) {
#pragma unroll
                for (int u = 0; u < B; ++u)
                    if (live[u]) acc = acc + w[u] * x[u];
            } else {
#pragma unroll
                for (int u = 0; u < B; ++u) s_prod[u][tid] = w[u] * x[u];
                wave_sync_lds();
                if (pt && sub == 0) {
                    const int mask = (1 << lg) - 1;
                    const int uhi = min(cnt, (t0 + B) << lg);
                    for (int uu = t0 << lg; uu < uhi; ++uu)
                        acc = acc + s_prod[(uu >> lg) - t0][(i << lg) + (uu & mask)];
                }
                wave_sync_lds();
            }
        }
        if (pt && sub == 0) {
            sweep_publish(vb + q, acc);
            if (xg && q >= n0) {
                const T x = sdq * acc;
                xg[q] = x;
                if (xout) xout[oidx ? (int64_t)oidx[q] : q] = x;  // null map: identity
            }
        }
        if (tid == 0) s_c = next;
        __syncthreads();
        c = __builtin_amdgcn_readfirstlane(s_c);
    }
}

// ---- adjoint pullback -----------------------------------------------------------------------
// d/dpoints scatter of one point's Abar (src/kernels_adjoint.jl:223-252): each pair's term is
// summed per block row in double, then one f64 atomic add per row and coordinate into dp
// (N x D, tree order).
template <typename T, int K, int D, bool ONE>
__device__ inline void scatter_pts(double* dp, const Block<T, K, D>& blk, const int32_t (&nb)[K],
                                   int64_t m, int64_t n0,
                                   const T (&Abar)[(K + 1) * (K + 2) / 2], T scale,
                                   const TabEnt<T>* tab, const uint16_t* acc,
                                   const TabParams<T>& P) {
    constexpr int N = K + 1;
    double g[N][D];
#pragma unroll
    for (int a = 0; a < N; ++a)
#pragma unroll
        for (int d = 0; d < D; ++d) g[a][d] = 0.0;
#pragma unroll
    for (int a = 1; a < N; ++a)
#pragma unroll
        for (int b = 0; b < a; ++b) {
            T c[D];
            if (pair_pts<T, D, ONE>(blk.jc[a], blk.jc[b], Abar[tri(a, b)], scale, tab, acc, P, c)) {
#pragma unroll
                for (int d = 0; d < D; ++d) {
                    g[a][d] += (double)c[d];
                    g[b][d] -= (double)c[d];
                }
            }
        }
#pragma unroll
    for (int a = 0; a < N; ++a) {
        const int64_t ga = a < K ? (int64_t)nb[a] : n0 + m;
#pragma unroll
        for (int d = 0; d < D; ++d) atomicAdd(&dp[ga * D + d], g[a][d]);
    }
}

// The grid-stride loop of k_pullback over the refined points; returns this lane's sum of the
// scalar terms. ONE: the single-step table search (P.steps <= 1).
template <typename T, int K, int D, int MODE, bool ONE>
__device__ inline double pullback_points(const uint32_t* __restrict__ coords,
                                         const int32_t* __restrict__ nbr, int64_t M, int64_t n0,
                                         T scale, const TabEnt<T>* s_tab, const uint16_t* s_acc,
                                         const TabParams<T>& P, const T* __restrict__ v,
                                         const T* __restrict__ xi, const T* __restrict__ vb,
                                         double* __restrict__ hist_partial, double* s_hist) {
    constexpr int SEED = MODE & 3;
    constexpr bool PTS = (MODE & P_PTS) != 0;
    constexpr int N = K + 1;
    constexpr int NT = N * (N + 1) / 2;
    double ssum = 0.0;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t m = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; m < M; m += stride) {
        Block<T, K, D> blk;
        int32_t nb[K];
        blk.gather(coords, nbr, M, m, n0, nb);
        blk.template assemble<ONE>(scale, s_tab, s_acc, P);
        blk.cholesky();
        const T s = blk.stddev();
        T Lbar[NT];
#pragma unroll
        for (int i = 0; i < NT; ++i) Lbar[i] = T(0);
        if (SEED == P_LOGDET) {
            // src/linalg.jl:140-146 with seed 1; the term itself for the fused logdet.
            ssum += (double)num<T>::log(s);
            Lbar[tri(K, K)] = T(1) / s;
        } else {
            T x[K], zbar[K];
            blk.mean_vec(x);
            if (SEED == P_INVLOSS) {
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
                    zbar[i] = div_rcp(t, blk.A[tri(i, i)], blk.rd[i]);
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
                    zbar[i] = blk.A[tri(i, i)] > pivfloor ? div_rcp(t, blk.A[tri(i, i)], blk.rd[i]) : T(0);
                }
            }
#pragma unroll
            for (int j = 0; j < K; ++j) {
                Lbar[tri(K, j)] += zbar[j];
#pragma unroll
                for (int i = 0; i <= j; ++i) Lbar[tri(j, i)] -= zbar[i] * x[j];
            }
        }
        if (PTS) {
            T Abar[NT];
#pragma unroll
            for (int i = 0; i < NT; ++i) Abar[i] = T(0);
            chol_pullback<T, N>(Abar, Lbar, blk.A, blk.rd);
            scatter_pts<T, K, D, ONE>(hist_partial, blk, nb, m, n0, Abar, scale, s_tab, s_acc, P);
        } else {
            // Abar[i][j] goes through the lookup weights as it is formed (src/kernels_adjoint.jl:
            // 47-74); the diagonal, summed in row order, into bin 0
            T sdiag[N];
            chol_pullback_each<T, N>(Lbar, blk.A, blk.rd, sdiag, [&](int i, int j, T g) {
                const T r = radius<T>(sqdist<D>(blk.jc[i], blk.jc[j]), scale);
                T wlo, whi;
                const int lo = cov_weights<T, ONE>(r, s_tab, s_acc, P, wlo, whi);
                atomicAdd(&s_hist[lo], (double)(g * wlo));
                atomicAdd(&s_hist[lo + 1], (double)(g * whi));
            });
            T diag = T(0);
#pragma unroll
            for (int a = 0; a < N; ++a) diag += sdiag[a];
            atomicAdd(&s_hist[0], (double)diag);
        }
    }
    return ssum;
}

// MODE: P_LOGDET / P_INVLOSS / P_GENVALS seeds the factor cotangents; with P_PTS added, Abar goes
// to the point positions (hist_partial is then dp, N x D) instead of the table histogram.
template <typename T, int K, int D, int MODE>
__global__ void __launch_bounds__(kBlock)
k_pullback(const uint32_t* __restrict__ coords, const int32_t* __restrict__ nbr, int64_t M,
           int64_t n0, T scale, const TabEnt<T>* __restrict__ g_tab,
           const uint16_t* __restrict__ g_acc, const TabParams<T>* __restrict__ Pp,
           const T* __restrict__ v,     // INVLOSS: values (tree order); GENVALS: forward field
           const T* __restrict__ xi,    // GENVALS: xi (tree order)
           const T* __restrict__ vb,    // GENVALS: field cotangent after the reverse sweep
           double* __restrict__ hist_partial, double* __restrict__ scalar_partial) {
    constexpr bool PTS = (MODE & P_PTS) != 0;
    const TabParams<T> P = *Pp;
    extern __shared__ __align__(16) unsigned char smem[];
    TabEnt<T>* s_tab = reinterpret_cast<TabEnt<T>*>(smem);
    uint16_t* s_acc = reinterpret_cast<uint16_t*>(smem + (size_t)(P.nb - 1) * sizeof(TabEnt<T>));
    double* s_hist = reinterpret_cast<double*>(smem + tab_bytes<T>(P.nb, P.ucells));
    __shared__ double s_red[kBlock / 64];
    if (!PTS)
        for (int i = threadIdx.x; i < P.nb; i += blockDim.x) s_hist[i] = 0.0;
    stage_table(s_tab, s_acc, g_tab, g_acc, P);

    // The branch-free single-step lookups raise this kernel's register count past three
    // wavefronts per SIMD, which costs more than they save: the general search throughout.
    const double ssum = pullback_points<T, K, D, MODE, false>(coords, nbr, M, n0, scale, s_tab,
                                                              s_acc, P, v, xi, vb, hist_partial,
                                                              s_hist);
    __syncthreads();
    if (!PTS) {
        double* out = hist_partial + (size_t)blockIdx.x * P.nb;
        for (int i = threadIdx.x; i < P.nb; i += blockDim.x) out[i] = s_hist[i];
    }
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
    const size_t lds = aniso ? (size_t)tb.aniso.lds : tab_bytes<T>(tb.P.nb, tb.P.ucells);
    const T scale = (T)g.scale;
#define GGP_FACTOR(DD, MODEV)                                                                  \
    do {                                                                                       \
        if (aniso)                                                                             \
            hipLaunchKernelGGL((k_factor<T, K, DD, MODEV, true>), dim3(nblk), dim3(kBlock), lds,\
                               st, g.coords, g.nbr, g.M, g.n0, scale, tb.tab, tb.acc,           \
                               tb.params, mv, sd, terms, partial, values, xi_out, tb.aniso,     \
                               g.nbr64);                                                        \
        else                                                                                   \
            hipLaunchKernelGGL((k_factor<T, K, DD, MODEV, false>), dim3(nblk), dim3(kBlock),    \
                               lds, st, g.coords, g.nbr, g.M, g.n0, scale, tb.tab, tb.acc,      \
                               tb.params, mv, sd, terms, partial, values, xi_out, tb.aniso,     \
                               g.nbr64);                                                        \
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
    const size_t lds = tab_bytes<T>(tb.P.nb, tb.P.ucells) +
                       ((mode & P_PTS) ? 0 : (size_t)tb.P.nb * sizeof(double));
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
        case P_LOGDET | P_PTS: GGP_PULL(DD, P_LOGDET | P_PTS); break;                          \
        case P_INVLOSS | P_PTS: GGP_PULL(DD, P_INVLOSS | P_PTS); break;                        \
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
                             const T* sd, bool two_pass, T* out, const int32_t* oidx,
                             hipStream_t st) {
    const unsigned nwg = (unsigned)std::max(1, std::min(g.n_fwd_chunks, g.sweep_wgs));
    if (two_pass)
        hipLaunchKernelGGL((k_sweep_fwd<T, K, true>), dim3(nwg), dim3(kBlock), 0, st, v, xi,
                           xi_off, mv, sd, g.nbr, g.M, g.n0, (int)g.K, g.fwd_chunks,
                           g.n_fwd_chunks, g.sweep_ticket, g.sweep_err, out, oidx);
    else
        hipLaunchKernelGGL((k_sweep_fwd<T, K, false>), dim3(nwg), dim3(kBlock), 0, st, v, xi,
                           xi_off, mv, sd, g.nbr, g.M, g.n0, (int)g.K, g.fwd_chunks,
                           g.n_fwd_chunks, g.sweep_ticket, g.sweep_err, out, oidx);
}

template <typename T, int K>
void PointK<T, K>::sweep_rev(const Graph& g, T* vb, const T* vbar, T* xg, const T* mv,
                             const T* sd, T* xout, const int32_t* oidx, hipStream_t st) {
    const unsigned nwg = (unsigned)std::max(1, std::min(g.n_rev_chunks, g.sweep_wgs));
    hipLaunchKernelGGL((k_sweep_rev<T, K>), dim3(nwg), dim3(kBlock), 0, st, vb, vbar, xg, mv, sd,
                       g.rcnt, g.rev, g.M, g.n0, (int)g.K, g.rev_chunks, g.n_rev_chunks,
                       g.sweep_ticket + 1, g.sweep_err, xout, oidx);
}

}  // namespace ggp
