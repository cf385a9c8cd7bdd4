// ggp_kernels.hip — element-wise and reduction kernels, and the (k)-dispatch to the per-point
// kernel instantiations (ggp_point_kernels.h, compiled per (T, k) from ggp_inst.hip).
#include "ggp_point_kernels.h"

namespace ggp {

// Block-wide double sum of one value per thread; result valid in thread 0.
__device__ inline double block_sum_g(double v, double* s_red) {
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

// d_out[i] = T(sum_w partial[w][i] + extra[i]). One wave per bin: lane l sums rows l, l+64, ...
// in order, then the 64 lane sums are combined by a fixed shuffle tree (deterministic).
template <typename T>
__global__ void __launch_bounds__(256) k_reduce_hist(T* __restrict__ d_out,
                                                     const double* __restrict__ partial, int nw,
                                                     int nb, const double* __restrict__ extra) {
    const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int l = threadIdx.x & 63;
    double s = 0.0;
    if (i < nb)
        for (int w = l; w < nw; w += 64) s += partial[(size_t)w * nb + i];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_down(s, o, 64);
    if (i < nb && l == 0) {
        if (extra) s += extra[i];
        d_out[i] = (T)s;
    }
}

// out[0] = sum of n doubles (single block, fixed order per thread then tree).
__global__ void k_reduce_scalar(double* __restrict__ out, const double* __restrict__ in, int n,
                                const double* __restrict__ add) {
    __shared__ double s_red[kBlock / 64];
    double t = 0.0;
    for (int i = threadIdx.x; i < n; i += blockDim.x) t += in[i];
    t = block_sum_g(t, s_red);
    if (threadIdx.x == 0) out[0] = t + (add ? add[0] : 0.0);
}

// out[0] = sum_i x_i^2 / 2 in double (the dense part of the inverse loss, src/grad.jl:521).
template <typename T>
__global__ void k_sumsq_half(const T* __restrict__ x, int64_t n, double* __restrict__ out) {
    __shared__ double s_red[kBlock / 64];
    double t = 0.0;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) t += (double)x[i] * (double)x[i];
    t = block_sum_g(t, s_red);
    if (threadIdx.x == 0) out[0] = 0.5 * t;
}
template <typename T>
void launch_sumsq_half(const T* x, int64_t n, double* out, hipStream_t st) {
    hipLaunchKernelGGL((k_sumsq_half<T>), dim3(1), dim3(kBlock), 0, st, x, n, out);
}

// ---- permutations (src/orchestrate.jl:24, 38) -----------------------------------------------
template <typename T>
__global__ void k_gather(T* __restrict__ out, const T* __restrict__ in,
                         const int32_t* __restrict__ idx, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = idx ? in[idx[i]] : in[i];
}
template <typename T>
__global__ void k_scatter(T* __restrict__ out, const T* __restrict__ in,
                          const int32_t* __restrict__ idx, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        if (idx) out[idx[i]] = in[i]; else out[i] = in[i];
    }
}
template <typename T>
__global__ void k_fill(T* __restrict__ p, T v, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}
template <typename T>
__global__ void k_copy(T* __restrict__ dst, const T* __restrict__ src, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = src[i];
}
// ---- the group-per-point path (k not in the register-block set) ---------------------------
template <typename T>
void WideK<T>::factor(const Graph& g, const Table<T>& tb, int mode, T* mv, T* sd, T* terms,
                      double* partial, const T* values, T* xi_out, unsigned nblk,
                      hipStream_t st) {
    switch (g.D) {
        case 2: WideD<T, 2>::factor(g, tb, mode, mv, sd, terms, partial, values, xi_out, nblk, st); break;
        case 3: WideD<T, 3>::factor(g, tb, mode, mv, sd, terms, partial, values, xi_out, nblk, st); break;
        case 4: WideD<T, 4>::factor(g, tb, mode, mv, sd, terms, partial, values, xi_out, nblk, st); break;
        default: break;
    }
}

template <typename T>
void WideK<T>::pullback(const Graph& g, const Table<T>& tb, int mode, const T* v, const T* xi,
                        const T* vb, double* hist_partial, double* scalar_partial,
                        unsigned nblk, hipStream_t st) {
    switch (g.D) {
        case 2: WideD<T, 2>::pullback(g, tb, mode, v, xi, vb, hist_partial, scalar_partial, nblk, st); break;
        case 3: WideD<T, 3>::pullback(g, tb, mode, v, xi, vb, hist_partial, scalar_partial, nblk, st); break;
        case 4: WideD<T, 4>::pullback(g, tb, mode, v, xi, vb, hist_partial, scalar_partial, nblk, st); break;
        default: break;
    }
}

template <typename T>
void WideK<T>::sweep_fwd(const Graph& g, T* v, const T* xi, int64_t xi_off, const T* mv,
                         const T* sd, bool two_pass, T* out, const int32_t* oidx,
                         hipStream_t st) {
    PointK<T, 0>::sweep_fwd(g, v, xi, xi_off, mv, sd, two_pass, out, oidx, st);
}

template <typename T>
void WideK<T>::sweep_rev(const Graph& g, T* vb, const T* vbar, T* xg, const T* mv, const T* sd,
                         T* xout, const int32_t* oidx, hipStream_t st) {
    PointK<T, 0>::sweep_rev(g, vb, vbar, xg, mv, sd, xout, oidx, st);
}

template struct WideK<float>;
template struct WideK<double>;

// ================================ launchers ===================================================
static inline unsigned grid_for(int64_t n, int block = kBlock) {
    return (unsigned)((n + block - 1) / block);
}

// K = 0 selects the group-per-point kernels (every other k up to kMaxK).
template <typename T, int K> struct LaunchSel { using type = PointK<T, K>; };
template <typename T> struct LaunchSel<T, 0> { using type = WideK<T>; };
template <typename T, int K> using Launch = typename LaunchSel<T, K>::type;

#define GGP_FOR_K(CALL)                              \
    do {                                             \
        switch (g.K) {                               \
            case 4: CALL(4); break;                  \
            case 8: CALL(8); break;                  \
            case 10: CALL(10); break;                \
            case 16: CALL(16); break;                \
            default: CALL(0); break;                 \
        }                                            \
    } while (0)

// A table in global memory (too large for LDS) runs on the group-per-point kernels for
// every k: they have the global-table form, and give the same IEEE results.
template <typename T>
void launch_factor(const Graph& g, const Table<T>& tb, int mode, T* mv, T* sd, T* terms,
                   double* partial, const T* values, T* xi_out, unsigned nblk, hipStream_t st) {
#define CALLF(KK) Launch<T, KK>::factor(g, tb, mode, mv, sd, terms, partial, values, xi_out, nblk, st)
    if (tb.global) CALLF(0);
    else GGP_FOR_K(CALLF);
#undef CALLF
}

template <typename T>
void launch_pullback(const Graph& g, const Table<T>& tb, int mode, const T* v, const T* xi,
                     const T* vb, double* hist_partial, double* scalar_partial, unsigned nblk,
                     hipStream_t st) {
#define CALLP(KK) Launch<T, KK>::pullback(g, tb, mode, v, xi, vb, hist_partial, scalar_partial, nblk, st)
    if (tb.global) CALLP(0);
    else GGP_FOR_K(CALLP);
#undef CALLP
}

// Pending markers over the swept range of v and/or vb, and both tickets zeroed: one launch an
// op issues early, off its critical path, instead of one fill before each sweep.
template <typename U>
__global__ void k_sweep_prep(U* __restrict__ a, U* __restrict__ b, U mark, int64_t n,
                             int* __restrict__ tickets) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < 2 && blockIdx.x == 0) tickets[i] = 0;
    if (i < n) {
        if (a) a[i] = mark;
        if (b) b[i] = mark;
    }
}
template <typename T>
void launch_sweep_prep(const Graph& g, T* v, T* vb, hipStream_t st) {
    using U = typename num<T>::bits_t;
    const int64_t n = std::max<int64_t>(g.offsets.back() - g.n0, 1);
    hipLaunchKernelGGL((k_sweep_prep<U>), dim3(grid_for(n)), dim3(kBlock), 0, st,
                       v ? reinterpret_cast<U*>(v + g.n0) : nullptr,
                       vb ? reinterpret_cast<U*>(vb + g.n0) : nullptr, (U)Pending<T>::bits,
                       g.offsets.back() - g.n0, g.sweep_ticket);
}

template <typename T>
void launch_sweep_fwd(const Graph& g, T* v, const T* xi, int64_t xi_off, const T* mv,
                      const T* sd, bool two_pass, bool prepared, hipStream_t st, T* out,
                      const int32_t* oidx) {
    if (g.n_fwd_chunks == 0) return;
    if (!prepared) launch_sweep_prep<T>(g, v, (T*)nullptr, st);
#define CALLS(KK) Launch<T, KK>::sweep_fwd(g, v, xi, xi_off, mv, sd, two_pass, out, oidx, st)
    GGP_FOR_K(CALLS);
#undef CALLS
}

template <typename T>
void launch_sweep_rev(const Graph& g, T* vb, const T* vbar, T* xg, const T* mv, const T* sd,
                      bool prepared, hipStream_t st, T* xout, const int32_t* oidx) {
    if (g.n_rev_chunks == 0) return;
    if (!prepared) launch_sweep_prep<T>(g, (T*)nullptr, vb, st);
#define CALLR(KK) Launch<T, KK>::sweep_rev(g, vb, vbar, xg, mv, sd, xout, oidx, st)
    GGP_FOR_K(CALLR);
#undef CALLR
}

template <typename U>
__global__ void k_fill_bits(U* __restrict__ p, U v, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}
template <typename T>
void launch_fill_pending(T* p, int64_t n, hipStream_t st) {
    using U = typename num<T>::bits_t;
    if (n > 0)
        hipLaunchKernelGGL((k_fill_bits<U>), dim3(grid_for(n)), dim3(kBlock), 0, st,
                           reinterpret_cast<U*>(p), (U)Pending<T>::bits, n);
}

template <typename T>
void launch_reduce_hist(T* d_out, const double* partial, int nw, int nb, const double* extra,
                        hipStream_t st) {
    hipLaunchKernelGGL((k_reduce_hist<T>), dim3((nb + 3) / 4), dim3(256), 0, st, d_out,
                       partial, nw, nb, extra);
}

void launch_reduce_scalar(double* out, const double* in, int n, const double* add,
                          hipStream_t st) {
    hipLaunchKernelGGL(k_reduce_scalar, dim3(1), dim3(kBlock), 0, st, out, in, n, add);
}

template <typename T>
void launch_gather(T* out, const T* in, const int32_t* idx, int64_t n, hipStream_t st) {
    if (n > 0) hipLaunchKernelGGL((k_gather<T>), dim3(grid_for(n)), dim3(kBlock), 0, st, out, in, idx, n);
}
template <typename T>
void launch_scatter(T* out, const T* in, const int32_t* idx, int64_t n, hipStream_t st) {
    if (n > 0) hipLaunchKernelGGL((k_scatter<T>), dim3(grid_for(n)), dim3(kBlock), 0, st, out, in, idx, n);
}
template <typename T>
void launch_fill(T* p, T v, int64_t n, hipStream_t st) {
    if (n > 0) hipLaunchKernelGGL((k_fill<T>), dim3(grid_for(n)), dim3(kBlock), 0, st, p, v, n);
}
template <typename T>
void launch_copy(T* dst, const T* src, int64_t n, hipStream_t st) {
    if (n > 0) hipLaunchKernelGGL((k_copy<T>), dim3(grid_for(n)), dim3(kBlock), 0, st, dst, src, n);
}

// out[row(r)][d] = dp[r][d] (+ dpd[r][d] for the first n_dense entries), rounded to T once;
// row = map[r] (internal -> tree position) or r.
template <typename T>
__global__ void k_points_out(T* __restrict__ out, const double* __restrict__ dp,
                             const double* __restrict__ dpd, int64_t N, int D, int64_t n_dense,
                             const int32_t* __restrict__ map) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N * D) return;
    const int64_t r = i / D, d = i - r * D;
    const int64_t row = map ? (int64_t)map[r] : r;
    out[row * D + d] = (T)(i < n_dense ? dp[i] + dpd[i] : dp[i]);
}
template <typename T>
void launch_points_out(T* out, const double* dp, const double* dpd, int64_t N, int D,
                       int64_t n_dense, const int32_t* map, hipStream_t st) {
    if (N > 0)
        hipLaunchKernelGGL((k_points_out<T>), dim3(grid_for(N * D)), dim3(kBlock), 0, st, out, dp,
                           dpd, N, D, n_dense, map);
}

// Self-check of div_rcp against the IEEE division. f32: every divisor bit pattern in
// [b0, b0 + count), each with `per` numerators; f64: `count` random divisors in [2^-60, 2^60).
// Numerators: random sign and significand, exponent uniform over 2^-100 .. 2^100 (f32) or
// 2^-900 .. 2^900 (f64), and zero.
__device__ inline uint64_t mix64(uint64_t x) {
    x += 0x9e3779b97f4a7c15ull;
    x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
    x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
    return x ^ (x >> 31);
}
__global__ void __launch_bounds__(256) k_div_check(int f64, uint64_t b0, uint64_t count,
                                                   uint32_t per, uint64_t seed,
                                                   unsigned long long* bad) {
    unsigned long long nbad = 0;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride) {
        if (!f64) {
            const float d = __uint_as_float((uint32_t)(b0 + i));
            const float y = 1.0f / d;
            // the reciprocal the kernels use (equal to 1/d on [2^-126, 2^126) and at 0, inf, NaN)
            const float yr = ggp::rcp_rn(d);
            const bool in = __builtin_fabsf(d) >= 0x1p-126f && __builtin_fabsf(d) < 0x1p126f;
            if (in || d == 0.f || __builtin_isinf(d)) nbad += __float_as_uint(yr) != __float_as_uint(y);
            else if (d != d) nbad += yr == yr;
            for (uint32_t u = 0; u < per; ++u) {
                const uint64_t h = mix64(seed ^ (i * 0x100000001b3ull + u));
                const uint32_t e = 27u + (uint32_t)((h >> 32) % 201u);  // 2^-100 .. 2^100
                const uint32_t bits = (uint32_t)(h & 0x807fffffu) | (e << 23);
                const float t = u == 0 ? 0.0f : __uint_as_float(bits);
                nbad += __float_as_uint(ggp::div_rcp(t, d, y)) != __float_as_uint(t / d);
            }
        } else {
            const uint64_t hd = mix64(seed + i);
            const uint64_t ed = 963u + (hd >> 52) % 121u;  // 2^-60 .. 2^60
            const double d = __longlong_as_double((long long)((hd & 0x000fffffffffffffull) | (ed << 52)));
            const double y = 1.0 / d;
            for (uint32_t u = 0; u < per; ++u) {
                const uint64_t h = mix64(hd ^ (u * 0x9e3779b97f4a7c15ull));
                const uint64_t e = 123u + (h >> 52) % 1801u;  // 2^-900 .. 2^900
                const uint64_t bits = (h & 0x800fffffffffffffull) | (e << 52);
                const double t = u == 0 ? 0.0 : __longlong_as_double((long long)bits);
                nbad += __double_as_longlong(ggp::div_rcp(t, d, y)) != __double_as_longlong(t / d);
            }
        }
    }
    if (nbad) atomicAdd(bad, nbad);
}
void launch_div_check(int f64, uint64_t b0, uint64_t count, uint32_t per, uint64_t seed,
                      unsigned long long* bad, hipStream_t st) {
    hipLaunchKernelGGL(k_div_check, dim3(4096), dim3(256), 0, st, f64, b0, count, per, seed, bad);
}

// Self-check of the square roots against the correctly rounded sqrtf over `count` consecutive
// bit patterns from b0: sqrt_rn_any_f32 everywhere (NaN results match any NaN), sqrt_rn_f32 on 0
// and [1e-30, 2^64]; *bad receives the number of differing results.
__global__ void __launch_bounds__(256) k_sqrt_check(uint32_t b0, uint32_t count,
                                                    unsigned long long* __restrict__ bad) {
    const uint32_t stride = gridDim.x * blockDim.x;
    unsigned long long nbad = 0;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride) {
        const float x = __uint_as_float(b0 + i);
        const float ref = __builtin_sqrtf(x);
        const float any = sqrt_rn_any_f32(x);
        nbad += ref != ref ? any == any : __float_as_uint(any) != __float_as_uint(ref);
        if (x == 0.f || (x >= 1e-30f && x <= 0x1p64f))
            nbad += __float_as_uint(sqrt_rn_f32(x)) != __float_as_uint(ref);
    }
    if (nbad) atomicAdd(bad, nbad);
}
void launch_sqrt_check(uint32_t b0, uint32_t count, unsigned long long* bad, hipStream_t st) {
    hipLaunchKernelGGL(k_sqrt_check, dim3(4096), dim3(256), 0, st, b0, count, bad);
}

#define GGP_INST(T)                                                                            \
    template void launch_factor<T>(const Graph&, const Table<T>&, int, T*, T*, T*, double*,    \
                                   const T*, T*, unsigned, hipStream_t);                       \
    template void launch_pullback<T>(const Graph&, const Table<T>&, int, const T*, const T*,   \
                                     const T*, double*, double*, unsigned, hipStream_t);       \
    template void launch_sweep_fwd<T>(const Graph&, T*, const T*, int64_t, const T*, const T*, \
                                      bool, bool, hipStream_t, T*, const int32_t*);            \
    template void launch_sweep_rev<T>(const Graph&, T*, const T*, T*, const T*, const T*,      \
                                      bool, hipStream_t, T*, const int32_t*);                  \
    template void launch_sweep_prep<T>(const Graph&, T*, T*, hipStream_t);                     \
    template void launch_fill_pending<T>(T*, int64_t, hipStream_t);                            \
    template void launch_reduce_hist<T>(T*, const double*, int, int, const double*,            \
                                        hipStream_t);                                          \
    template void launch_gather<T>(T*, const T*, const int32_t*, int64_t, hipStream_t);        \
    template void launch_scatter<T>(T*, const T*, const int32_t*, int64_t, hipStream_t);       \
    template void launch_fill<T>(T*, T, int64_t, hipStream_t);                                 \
    template void launch_sumsq_half<T>(const T*, int64_t, double*, hipStream_t);               \
    template void launch_copy<T>(T*, const T*, int64_t, hipStream_t);                          \
    template void launch_points_out<T>(T*, const double*, const double*, int64_t, int,        \
                                       int64_t, const int32_t*, hipStream_t);
GGP_INST(float)
GGP_INST(double)
template void launch_fill<int>(int*, int, int64_t, hipStream_t);

}  // namespace ggp
