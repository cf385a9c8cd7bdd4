// ggp_point.h — per-point device primitives of the Vecchia refinement, for gfx950.
//
// One lane owns one refined point. The (k+1)x(k+1) covariance block, its Cholesky factor and
// (in the adjoints) the factor/covariance cotangents live in VGPRs as packed lower triangles;
// every loop over the block is unrolled at compile time (K, D are template parameters), so no
// private array is ever indexed at run time and nothing goes to scratch for k <= 10.
//
// Arithmetic follows the reference expression by expression (file:line cited per function):
// a multiply feeding an add/sub is a single fma exactly where the reference evaluates it under
// @fastmath, and a separate multiply and add everywhere else. The library is compiled with
// -ffp-contract=off, so the compiler fuses nothing by itself; division and square root are the
// correctly rounded IEEE operations (HIP's defaults for f32 and f64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace ggp {

template <typename T> struct num;
template <> struct num<float> {
    using bits_t = uint32_t;
    using sbits_t = int32_t;
    __device__ __host__ static constexpr float eps() { return 1.1920928955078125e-7f; }
    __device__ static inline float fma(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
    __device__ static inline float sqrt(float a) { return __builtin_sqrtf(a); }
    __device__ static inline float log(float a) { return ::logf(a); }
    __device__ static inline bits_t bits(float a) { return __float_as_uint(a); }
};
template <> struct num<double> {
    using bits_t = uint64_t;
    using sbits_t = int64_t;
    __device__ __host__ static constexpr double eps() { return 2.220446049250313e-16; }
    __device__ static inline double fma(double a, double b, double c) { return __builtin_fma(a, b, c); }
    __device__ static inline double sqrt(double a) { return __builtin_sqrt(a); }
    __device__ static inline double log(double a) { return ::log(a); }
    __device__ static inline bits_t bits(double a) { return (bits_t)__double_as_longlong(a); }
};

// t / d rounded once, given y = RN(1/d) (rcp_rn, one per divisor): q0 = t*y lies within
// an ulp of t/d, the remainder t - d*q0 is exact in one fma, and q0 + (t - d*q0)*y rounded once
// is the correctly rounded quotient (Markstein's correction step, as in the IA-64 division
// sequences). It equals the IEEE division whenever the remainder is representable and nothing
// overflows: t = 0, or |t| >= 2^-103 (f32; 2^-970 in f64) with a normal quotient. A nonzero
// |t| below that (reachable only by cancelling covariance entries to 2^-100 of their size) may
// differ in the last bit of a subnormal-range quotient. ggp_selftest_div checks it on the device.
template <typename T>
__device__ inline T div_rcp(T t, T d, T y) {
    const T q0 = t * y;
    return num<T>::fma(num<T>::fma(-q0, d, t), y, q0);
}

// f(integral_constant<int, I>) for I = B .. E-1, each call its own inlined copy (a loop whose
// body is too large for the unroller's budget would otherwise keep a run-time index into the
// lanes' register arrays and send them to scratch memory).
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// RN(1/d), the IEEE quotient: f32 through v_rcp_f32 (within 1 ulp) and one Newton step
// r + r(1 - d r) with the residual exact in one fma, which equals 1/d for every d in
// [2^-126, 2^126) (ggp_selftest_div compares the two for each divisor it takes); zeros,
// infinities and NaN (whose residual is NaN) keep v_rcp_f32's result, which is 1/d there.
// Subnormal and larger d never reach it (it divides by square roots of positive floats).
template <typename T>
__device__ inline T rcp_rn(T d) {
    return T(1) / d;
}
template <>
__device__ inline float rcp_rn<float>(float d) {
    const float r = __builtin_amdgcn_rcpf(d);
    const float e = __builtin_fmaf(-d, r, 1.0f);
    return e == e ? __builtin_fmaf(e, r, r) : r;
}

// ---- values published one by one ----------------------------------------------------------
// A value that another workgroup waits for can carry its own readiness: the buffer starts as a
// pending marker (a NaN no arithmetic produces), the writer publishes each value once with an
// agent-scope store, and a reader takes the values with plain loads and polls with agent-scope
// loads only those it still sees pending (a published value never changes, so a plain load
// returns the marker or the final value). No flag and no release/acquire pair is needed: the
// values are the data. The level sweeps and the dense factor's hand-offs use it.
template <typename T> struct Pending;
template <> struct Pending<float> { static constexpr uint32_t bits = 0x7fc0feedu; };
template <> struct Pending<double> { static constexpr uint64_t bits = 0x7ff800000000feedull; };
constexpr int kSweepSpinLimit = 1 << 20;

__device__ inline float from_bits(uint32_t b) { return __uint_as_float(b); }
__device__ inline double from_bits(uint64_t b) { return __longlong_as_double((long long)b); }

// Values at p[idx[u]] for the live entries u < B (live[u] false: 0). All reads are issued
// together; the ones still pending are polled together, one back-off sleep per round.
template <typename T, int B>
__device__ inline void sweep_read_all(T (&out)[B], const T* p, const int64_t (&idx)[B],
                                      const bool (&live)[B], int* err, int err_bit = 4) {
    using U = typename num<T>::bits_t;
    const U* pu = reinterpret_cast<const U*>(p);
    U b[B];
#pragma unroll
    for (int u = 0; u < B; ++u) b[u] = live[u] ? pu[idx[u]] : U(0);
    for (int spins = 0;; ++spins) {
        bool pending = false;
#pragma unroll
        for (int u = 0; u < B; ++u) pending = pending || b[u] == Pending<T>::bits;
        if (!pending) break;
        if (spins > kSweepSpinLimit) {
            atomicOr(err, err_bit);
            break;
        }
        if (spins < 8) __builtin_amdgcn_s_sleep(1);
        else __builtin_amdgcn_s_sleep(4);
#pragma unroll
        for (int u = 0; u < B; ++u)
            if (b[u] == Pending<T>::bits)
                b[u] = __hip_atomic_load(pu + idx[u], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int u = 0; u < B; ++u) out[u] = live[u] ? from_bits(b[u]) : T(0);
}

template <typename T>
__device__ inline void sweep_publish(T* p, T x) {
    using U = typename num<T>::bits_t;
    __hip_atomic_store(reinterpret_cast<U*>(p), num<T>::bits(x), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// ---- cross-lane moves (wave-uniform lane index; call from wave-uniform control flow) --------
// bcast: the value of x in `lane`, for every lane. put: x with `lane`'s value replaced by v
// (me = the calling lane).
__device__ inline float bcast(float x, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}
__device__ inline double bcast(double x, int lane) {
    const long long v = __double_as_longlong(x);
    const int lo = __builtin_amdgcn_readlane((int)(v & 0xffffffffLL), lane);
    const int hi = __builtin_amdgcn_readlane((int)(v >> 32), lane);
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}
__device__ inline uint32_t bcast(uint32_t x, int lane) {
    return (uint32_t)__builtin_amdgcn_readlane((int)x, lane);
}
template <typename T>
__device__ inline T put(T x, T v, int lane, int me) {
    return me == lane ? v : x;
}

// Orders one wavefront's LDS writes before its later reads (no workgroup barrier).
__device__ inline void wave_sync_lds() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Index of (i, j), i >= j, in a packed lower triangle.
__host__ __device__ constexpr int tri(int i, int j) { return i * (i + 1) / 2 + j; }

// ---- covariance table -------------------------------------------------------------------------
// Entry `lo` of the interpolation table: the bracketing segment [bins[lo], bins[lo+1]).
// `slope` is (vals[lo+1]-vals[lo]) / (bins[lo+1]-bins[lo]) evaluated once in T, which is the
// same IEEE value the reference computes inline (src/interp.jl:30).
template <typename T> struct __attribute__((aligned(4 * sizeof(T)))) TabEnt {
    T x0, y0, slope, x1;
};

// Scalars that describe the table and its O(1) segment index.
//
// The reference finds `lo` (bins[lo] <= r < bins[lo+1]) by binary search (src/interp.jl:17-27).
// Here the segment is found from the IEEE bit pattern of r, which is monotone in r for r >= 0:
// cell c = (bits(r) - bits(bins[1])) >> shift, and acc[c+1] is the largest lo with bins[lo] <=
// the smallest value of cell c. Starting there and stepping forward while bins[lo+1] <= r gives
// the unique lo with bins[lo] <= r < bins[lo+1] — the binary search's answer — for any strictly
// increasing table; on log-spaced tables the forward step runs at most about once.
template <typename T> struct TabParams {
    T b0, b1, bl, v0, vl;          // bins[0], bins[1], bins[nb-1], vals[0], vals[nb-1]
    typename num<T>::bits_t base;  // bits(bins[1])
    int shift;                     // cell width in ulps = 2^shift
    int ucells;                    // number of cells U; acc has U+1 entries
    int nb;                        // number of bins
    int steps;                     // most forward steps any r in [b0, bl) needs from acc[cell]
};

// ONE: the table has steps <= 1 (every cell holds at most one bin edge, as on log-spaced tables),
// so the search is one unconditional step and the lookup has no branch: the out-of-range cases
// are selected afterwards, the lookup itself running on an in-range stand-in. The kernels choose
// ONE once per launch from P.steps; both forms return the same lo.
template <typename T, bool ONE>
__device__ inline int seg_index(T r, const TabEnt<T>* __restrict__ tab,
                                const uint16_t* __restrict__ acc, const TabParams<T>& P) {
    using S = typename num<T>::sbits_t;
    S d = (S)(num<T>::bits(r) - P.base);
    int cell = d < 0 ? 0 : (int)min((S)(d >> P.shift) + 1, (S)P.ucells);
    int lo = acc[cell];
    if (ONE) lo += r >= tab[lo].x1 ? 1 : 0;
    else while (r >= tab[lo].x1) ++lo;  // bounded: bins[nb-1] > r here
    return lo;
}

// cov_lookup (src/interp.jl:10-34).
template <typename T, bool ONE = false>
__device__ inline T cov_lookup(T r, const TabEnt<T>* __restrict__ tab,
                               const uint16_t* __restrict__ acc, const TabParams<T>& P) {
    if (ONE) {
        const T b0 = P.b0, bl = P.bl, v0 = P.v0, vl = P.vl;
        const bool below = r <= b0, above = r >= bl;
        const T rr = above ? b0 : r;
        const TabEnt<T> e = tab[seg_index<T, true>(rr, tab, acc, P)];
        T v = num<T>::fma(e.slope, rr - e.x0, e.y0);
        v = above ? vl : v;
        return below ? v0 : v;
    }
    if (r <= P.b0) return P.v0;
    if (r >= P.bl) return P.vl;
    const TabEnt<T> e = tab[seg_index<T, false>(r, tab, acc, P)];
    return num<T>::fma(e.slope, r - e.x0, e.y0);  // @fastmath y0 + slope*(r - x0)
}

// cov_lookup_dr (src/interp.jl:43-60): d cov / d r, the bracketing segment's slope; 0 at or
// beyond either end of the table.
template <typename T, bool ONE = false>
__device__ inline T cov_slope(T r, const TabEnt<T>* __restrict__ tab,
                              const uint16_t* __restrict__ acc, const TabParams<T>& P) {
    if (ONE) {
        const T b0 = P.b0, bl = P.bl;
        const bool out = r <= b0 || r >= bl;
        const T rr = r >= bl ? b0 : r;
        const T sl = tab[seg_index<T, true>(rr, tab, acc, P)].slope;
        return out ? T(0) : sl;
    }
    if (r <= P.b0 || r >= P.bl) return T(0);
    return tab[seg_index<T, false>(r, tab, acc, P)].slope;
}

// cov_lookup_weights (src/interp.jl:62-83): value = wlo*vals[lo] + whi*vals[lo+1].
template <typename T, bool ONE = false>
__device__ inline int cov_weights(T r, const TabEnt<T>* __restrict__ tab,
                                  const uint16_t* __restrict__ acc, const TabParams<T>& P,
                                  T& wlo, T& whi) {
    if (ONE) {
        const T b0 = P.b0, bl = P.bl;
        const int last = P.nb - 2;
        const bool below = r <= b0, above = r >= bl;
        const T rr = above ? b0 : r;
        const int lo = seg_index<T, true>(rr, tab, acc, P);
        const TabEnt<T> e = tab[lo];
        const T t = (rr - e.x0) / (e.x1 - e.x0);
        T wl = T(1) - t, wh = t;
        wl = above ? T(0) : wl;
        wh = above ? T(1) : wh;
        wlo = below ? T(1) : wl;
        whi = below ? T(0) : wh;
        const int l2 = above ? last : lo;
        return below ? 0 : l2;
    }
    if (r <= P.b0) { wlo = T(1); whi = T(0); return 0; }
    if (r >= P.bl) { wlo = T(0); whi = T(1); return P.nb - 2; }
    const int lo = seg_index<T, false>(r, tab, acc, P);
    const TabEnt<T> e = tab[lo];
    const T t = (r - e.x0) / (e.x1 - e.x0);
    wlo = T(1) - t;
    whi = t;
    return lo;
}

// Exact squared lattice distance. The reference accumulates Int64 (src/linalg.jl:19-23); the
// coordinates are < 2^21, so every term and the sum (< 2^46) are exact in double, and the
// conversion to T below rounds the same integer once, as T(sq) does.
template <int D>
__device__ inline double sqdist(const uint32_t (&a)[D], const uint32_t (&b)[D]) {
    double s = 0.0;
#pragma unroll
    for (int d = 0; d < D; ++d) {
        const double x = (double)((int32_t)a[d] - (int32_t)b[d]);
        s = __builtin_fma(x, x, s);  // exact: all operands and results are integers < 2^53
    }
    return s;
}

// Correctly rounded square root of x = 0 or x >= 1e-30 (f32), without the range scaling and
// special-value handling of the general sequence. v_sqrt_f32 is within 1 ulp of sqrt(x), so the
// correctly rounded result is s or one of its neighbours s-, s+; the exact residuals x - s-*s and
// x - s+*s (one fma each) decide which: no float lies strictly between s-*s and (s-1/2ulp)^2,
// nor between s*s+ and (s+1/2ulp)^2. Checked against sqrtf bit for bit over every float in
// [1e-30, 2^64] and 0 (selftest_sqrt).
__device__ inline float sqrt_rn_f32(float x) {
    const float s = __builtin_amdgcn_sqrtf(x);
    const float sdn = __uint_as_float(__float_as_uint(s) - 1u);
    const float sup = __uint_as_float(__float_as_uint(s) + 1u);
    const float rdn = __builtin_fmaf(-sdn, s, x);
    const float rup = __builtin_fmaf(-sup, s, x);
    const float y = rdn <= 0.f ? sdn : s;
    return rup > 0.f ? sup : y;
}
// Correctly rounded sqrtf(x) for every float x, from sqrt_rn_f32 by exact scaling: with e the
// exponent field of x and m = floor((e - 127) / 2), x 4^-m lies in [2^-23, 4) (subnormals
// included), inside sqrt_rn_f32's range, and sqrt(x) = sqrt(x 4^-m) 2^m with both scalings exact
// (the root of a positive float is normal); zeros, infinities and NaN pass through. For a
// wave-uniform x, m is scalar arithmetic and the sequence is shorter than the general one.
// Checked against sqrtf bit for bit over every float (selftest_sqrt; NaN results compared as
// NaN).
__device__ inline float sqrt_rn_any_f32(float x) {
    const int m = ((int)((__float_as_uint(x) >> 23) & 255u) - 127) >> 1;
    return __builtin_amdgcn_ldexpf(sqrt_rn_f32(__builtin_amdgcn_ldexpf(x, -2 * m)), m);
}
template <typename T> __device__ inline T sqrt_lattice(T x) { return num<T>::sqrt(x); }
template <> __device__ inline float sqrt_lattice<float>(float x) { return sqrt_rn_f32(x); }

// r = sqrt(T(sq)) * scale (src/linalg.jl:24; src/kernels_adjoint.jl:34). T(sq) is 0 or an
// integer >= 1, inside the fast square root's range.
template <typename T>
__device__ inline T radius(double sq, T scale) {
    return sqrt_lattice<T>((T)sq) * scale;
}

// One pair's contribution to d/dpoints (src/kernels_adjoint.jl:223-252): the off-diagonal
// cotangent g of the pair (a, b) through k'(r) dr/dx; c[d] is what point a gains and point b
// loses. Returns false (c untouched) for coincident points and radii outside the table.
template <typename T, int D, bool ONE = false>
__device__ inline bool pair_pts(const uint32_t (&ca)[D], const uint32_t (&cb)[D], T g, T scale,
                                const TabEnt<T>* __restrict__ tab,
                                const uint16_t* __restrict__ acc, const TabParams<T>& P,
                                T (&c)[D]) {
    const double sq = sqdist<D>(ca, cb);
    if (sq == 0.0) return false;
    const T r = radius<T>(sq, scale);
    const T dcov = cov_slope<T, ONE>(r, tab, acc, P);
    if (dcov == T(0)) return false;
    const T f = g * dcov / r;
#pragma unroll
    for (int d = 0; d < D; ++d) {
        const T diff = scale * ((T)ca[d] - (T)cb[d]);
        c[d] = f * diff;
    }
    return true;
}

// ---- anisotropic covariance K(d_spatial, d_z) (src/aniso.jl) ----------------------------------
// O(1) segment index of one axis of the grid: the cell index of TabParams over the IEEE bit
// patterns of [bins[1], bins[n-1]]; acc[c+1] is the largest lo <= n-2 with bins[lo] <= the
// smallest value of cell c.
template <typename T> struct AxisIdx {
    typename num<T>::bits_t base = 0;  // bits(bins[1])
    int shift = 0, ucells = 0;
};

// Device view of the table: axes sb (ns), zb (nz), grid[i*nz + j] = K(sb[i], zb[j]), alpha, and
// the axes' cell indices sacc (si.ucells + 1 entries) and zacc (zi.ucells + 1). The kernels that
// assemble anisotropic covariances stage the axes and their indices in LDS (aniso_stage) when
// `lds` bytes fit their budget; the grid is read from global memory (L2-resident).
template <typename T> struct AnisoArgs {
    const T* sb = nullptr;
    const T* zb = nullptr;
    const T* grid = nullptr;
    const uint16_t* sacc = nullptr;
    const uint16_t* zacc = nullptr;
    AxisIdx<T> si{}, zi{};
    int ns = 0, nz = 0;
    T alpha = T(1);
    int lds = 0;  // bytes of the staged axes and indices, 0: not staged
};

// _frac_index (src/aniso.jl:43-57): 0-based fractional position of d on an increasing axis,
// clamped to [0, n-1]. The bracketing segment is the binary search's (Julia tie rule: the
// largest lo with bins[lo] <= d), found from the cell index and forward steps.
template <typename T>
__device__ inline T frac_index(T d, const T* __restrict__ bins, int n,
                               const uint16_t* __restrict__ acc, const AxisIdx<T>& X) {
    if (d <= bins[0]) return T(0);
    if (d >= bins[n - 1]) return T(n - 1);
    using S = typename num<T>::sbits_t;
    const S dd = (S)(num<T>::bits(d) - X.base);
    const int cell = dd < 0 ? 0 : (int)min((S)(dd >> X.shift) + 1, (S)X.ucells);
    int lo = acc[cell];
    while (bins[lo + 1] <= d) ++lo;  // bounded: d < bins[n-1]
    const T x0 = bins[lo], x1 = bins[lo + 1];
    return T(lo) + (d - x0) / (x1 - x0);
}

// The axes and their cell indices copied into LDS at smem (an.lds bytes, nonzero) by the whole
// workgroup; returns the view whose axes are there. A caller that branches on an.lds and calls
// this on one side only keeps each side's pointers in one address space (LDS reads on this
// side, global reads on the other) instead of generic ones.
template <typename T>
__device__ inline AnisoArgs<T> aniso_stage_lds(const AnisoArgs<T>& an, unsigned char* smem) {
    AnisoArgs<T> s = an;
    T* sb = reinterpret_cast<T*>(smem);
    T* zb = sb + an.ns;
    uint16_t* sacc = reinterpret_cast<uint16_t*>(zb + an.nz);
    uint16_t* zacc = sacc + an.si.ucells + 1;
    const int t = (int)(threadIdx.x + blockDim.x * (threadIdx.y + blockDim.y * threadIdx.z));
    const int nth = (int)(blockDim.x * blockDim.y * blockDim.z);
    for (int i = t; i < an.ns; i += nth) sb[i] = an.sb[i];
    for (int i = t; i < an.nz; i += nth) zb[i] = an.zb[i];
    for (int i = t; i <= an.si.ucells; i += nth) sacc[i] = an.sacc[i];
    for (int i = t; i <= an.zi.ucells; i += nth) zacc[i] = an.zacc[i];
    __syncthreads();
    s.sb = sb;
    s.zb = zb;
    s.sacc = sacc;
    s.zacc = zacc;
    return s;
}

// aniso_stage_lds when the axes fit (an.lds != 0), else an itself.
template <typename T>
__device__ inline AnisoArgs<T> aniso_stage(const AnisoArgs<T>& an, unsigned char* smem) {
    return an.lds == 0 ? an : aniso_stage_lds(an, smem);
}

// Bytes aniso_stage needs: both axes, then both cell indices.
template <typename T>
__host__ __device__ inline size_t aniso_stage_bytes(int ns, int nz, int su, int zu) {
    return (size_t)(ns + nz) * sizeof(T) + (size_t)(su + 1 + zu + 1) * sizeof(uint16_t);
}

// aniso_lookup (src/aniso.jl:66-84): bilinear interpolation with edge clamping; no @fastmath.
template <typename T>
__device__ inline T aniso_lookup(T ds, T dz, const AnisoArgs<T>& a) {
    const T fx = frac_index(ds, a.sb, a.ns, a.sacc, a.si);
    const T fz = frac_index(dz, a.zb, a.nz, a.zacc, a.zi);
    const int i0 = (int)fx, j0 = (int)fz;
    const int i1 = i0 + 1 < a.ns ? i0 + 1 : a.ns - 1, j1 = j0 + 1 < a.nz ? j0 + 1 : a.nz - 1;
    const T tx = fx - T(i0), tz = fz - T(j0);
    const T g00 = a.grid[i0 * a.nz + j0], g10 = a.grid[i1 * a.nz + j0];
    const T g01 = a.grid[i0 * a.nz + j1], g11 = a.grid[i1 * a.nz + j1];
    return (g00 * (T(1) - tx) + g10 * tx) * (T(1) - tz) + (g01 * (T(1) - tx) + g11 * tx) * tz;
}

// Pair covariance of two lattice points (src/aniso.jl:96-106): spatial distance over the first
// D-1 dims, radial |dz| * scale / alpha over the last.
template <typename T, int D>
__device__ inline T aniso_pair(const uint32_t (&a)[D], const uint32_t (&b)[D], T scale,
                               const AnisoArgs<T>& an) {
    double sqs = 0.0;
#pragma unroll
    for (int d = 0; d < D - 1; ++d) {
        const double x = (double)((int32_t)a[d] - (int32_t)b[d]);
        sqs = __builtin_fma(x, x, sqs);  // exact integers
    }
    const T dz = (T)((int32_t)a[D - 1] - (int32_t)b[D - 1]);  // exact: |dz| < 2^24
    const T d_spatial = num<T>::sqrt((T)sqs) * scale;
    const T d_z = __builtin_fabs(dz) * scale / an.alpha;
    return aniso_lookup(d_spatial, d_z, an);
}

// ---- the per-point block ------------------------------------------------------------------
template <typename T, int K, int D>
struct Block {
    static constexpr int N = K + 1;
    static constexpr int NT = N * (N + 1) / 2;
    uint32_t jc[N][D];  // joint lattice coords: rows 0..K-1 the neighbours, row K the point
    T A[NT];            // covariance, then its Cholesky factor (packed lower)
    T rd[K];            // RN(1 / L[j][j]) for the columns with entries below the diagonal

    // _gather_joint! (src/kernels.jl:9-23). nbr is the int32 structure-of-arrays neighbour
    // table nbr[j*M + m]; with nbr64 set, the neighbours come from it instead, in the
    // reference's layout (int64, the K of a point contiguous: nbr64[m*K + j]). coords is
    // point-major.
    __device__ inline void gather(const uint32_t* __restrict__ coords,
                                  const int32_t* __restrict__ nbr, int64_t M, int64_t m,
                                  int64_t n0, int32_t (&nb)[K],
                                  const int64_t* __restrict__ nbr64 = nullptr) {
        if (nbr64) {
            // a caller's table is not validated on the host: an index that does not precede
            // the point is read as the point itself, so no access leaves the arrays
#pragma unroll
            for (int j = 0; j < K; ++j) {
                const int64_t q = nbr64[m * K + j];
                nb[j] = (int32_t)(q >= 0 && q < n0 + m ? q : n0 + m);
            }
        } else {
#pragma unroll
            for (int j = 0; j < K; ++j) nb[j] = nbr[(int64_t)j * M + m];
        }
#pragma unroll
        for (int j = 0; j < K; ++j) {
            const uint32_t* c = coords + (int64_t)nb[j] * D;
#pragma unroll
            for (int d = 0; d < D; ++d) jc[j][d] = c[d];
        }
        const uint32_t* c = coords + (n0 + m) * D;
#pragma unroll
        for (int d = 0; d < D; ++d) jc[K][d] = c[d];
    }

    // assemble_cov! (src/linalg.jl:15-29). With ROWS (single-step tables only) the lookups of
    // one row run phase by phase (radii, cell reads, step reads, entry reads), so their LDS round
    // trips overlap, at the cost of registers; each entry is the value cov_lookup returns.
    template <bool ONE = false, bool ROWS = false>
    __device__ inline void assemble(T scale, const TabEnt<T>* __restrict__ tab,
                                    const uint16_t* __restrict__ acc, const TabParams<T>& P) {
        if (!(ONE && ROWS)) {
#pragma unroll
            for (int a = 0; a < N; ++a) {
                A[tri(a, a)] = P.v0;  // cov_lookup(0) = vals[1] since bins[1] = 0 <= 0
#pragma unroll
                for (int b = 0; b < a; ++b)
                    A[tri(a, b)] = cov_lookup<T, ONE>(radius<T>(sqdist<D>(jc[a], jc[b]), scale),
                                                      tab, acc, P);
            }
            return;
        }
        using S = typename num<T>::sbits_t;
        const T b0 = P.b0, bl = P.bl, v0 = P.v0, vl = P.vl;
#pragma unroll
        for (int a = 0; a < N; ++a) {
            A[tri(a, a)] = v0;
            T r[N], rr[N];
            int lo[N];
#pragma unroll
            for (int b = 0; b < a; ++b) {
                r[b] = radius<T>(sqdist<D>(jc[a], jc[b]), scale);
                rr[b] = r[b] >= bl ? b0 : r[b];
                const S d = (S)(num<T>::bits(rr[b]) - P.base);
                const int cell = d < 0 ? 0 : (int)min((S)(d >> P.shift) + 1, (S)P.ucells);
                lo[b] = acc[cell];
            }
#pragma unroll
            for (int b = 0; b < a; ++b) lo[b] += rr[b] >= tab[lo[b]].x1 ? 1 : 0;
#pragma unroll
            for (int b = 0; b < a; ++b) {
                const TabEnt<T> e = tab[lo[b]];
                T v = num<T>::fma(e.slope, rr[b] - e.x0, e.y0);  // @fastmath y0 + slope*(r - x0)
                v = r[b] >= bl ? vl : v;
                A[tri(a, b)] = r[b] <= b0 ? v0 : v;
            }
        }
    }

    // anisotropic assemble_cov! (src/aniso.jl:88-108).
    __device__ inline void assemble_aniso(T scale, const AnisoArgs<T>& an) {
        const T diagv = aniso_lookup(T(0), T(0), an);
#pragma unroll
        for (int a = 0; a < N; ++a) {
            A[tri(a, a)] = diagv;
#pragma unroll
            for (int b = 0; b < a; ++b) A[tri(a, b)] = aniso_pair<T, D>(jc[a], jc[b], scale, an);
        }
    }

    // chol_lower! (src/linalg.jl:38-73), whole loop under @fastmath. The clamp branch is
    // evaluated as a select so the wave never diverges; both arms produce the reference's
    // values bit for bit.
    __device__ inline void cholesky() {
        const T pivmin = num<T>::eps() * A[0];
        const T dmin = num<T>::sqrt(pivmin);
#pragma unroll
        for (int j = 0; j < N; ++j) {
            T s = A[tri(j, j)];
#pragma unroll
            for (int p = 0; p < j; ++p) s = num<T>::fma(-A[tri(j, p)], A[tri(j, p)], s);
            const bool ok = s > pivmin;  // false for NaN, as in the reference
            const T d = ok ? num<T>::sqrt(s) : dmin;
            A[tri(j, j)] = d;
            if (j < K) rd[j] = rcp_rn(d);
#pragma unroll
            for (int i = j + 1; i < N; ++i) {
                T t = A[tri(i, j)];
#pragma unroll
                for (int p = 0; p < j; ++p) t = num<T>::fma(-A[tri(i, p)], A[tri(j, p)], t);
                A[tri(i, j)] = ok ? div_rcp(t, d, rd[j]) : T(0);
            }
        }
    }

    // mean_vec_solve! (src/linalg.jl:85-103), under @fastmath.
    __device__ inline void mean_vec(T (&x)[K]) const {
        const T pivfloor = T(1.5) * num<T>::sqrt(num<T>::eps()) * A[0];
#pragma unroll
        for (int i = K - 1; i >= 0; --i) {
            const T d = A[tri(i, i)];
            T s = A[tri(K, i)];
#pragma unroll
            for (int j = i + 1; j < K; ++j) s = num<T>::fma(-A[tri(j, i)], x[j], s);
            x[i] = d > pivfloor ? div_rcp(s, d, rd[i]) : T(0);
        }
    }

    __device__ inline T stddev() const { return A[tri(K, K)]; }
};

// chol_pullback! (src/linalg.jl:112-137), under @fastmath. Lbar holds the factor cotangents on
// entry and is consumed; Abar receives d/dA for the lower triangle. rd[j] = RN(1 / L[j][j]) for
// j < N - 1 (Block::rd): the divisions by L[j][j] and 2 L[j][j] use it (div_rcp, the IEEE
// quotient), the last column's one division is a plain division.
template <typename T, int N>
__device__ inline void chol_pullback(T (&Abar)[N * (N + 1) / 2], T (&Lbar)[N * (N + 1) / 2],
                                     const T (&L)[N * (N + 1) / 2], const T (&rd)[N - 1]) {
#pragma unroll
    for (int j = N - 1; j >= 0; --j) {
        const T ljj = L[tri(j, j)];
#pragma unroll
        for (int i = N - 1; i >= j + 1; --i) {
            const T lbij = Lbar[tri(i, j)];
            const T tbar = div_rcp(lbij, ljj, rd[j]);
            Lbar[tri(j, j)] -= div_rcp(lbij * L[tri(i, j)], ljj, rd[j]);
            Abar[tri(i, j)] = tbar;
#pragma unroll
            for (int p = 0; p < j; ++p) {
                Lbar[tri(i, p)] = num<T>::fma(-tbar, L[tri(j, p)], Lbar[tri(i, p)]);
                Lbar[tri(j, p)] = num<T>::fma(-tbar, L[tri(i, p)], Lbar[tri(j, p)]);
            }
        }
        const T sbar = j < N - 1 ? div_rcp(Lbar[tri(j, j)], T(2) * ljj, rd[j < N - 1 ? j : 0] * T(0.5))
                                 : Lbar[tri(j, j)] / (T(2) * ljj);
        Abar[tri(j, j)] = sbar;
#pragma unroll
        for (int p = 0; p < j; ++p)
            Lbar[tri(j, p)] = num<T>::fma(-(T(2) * sbar), L[tri(j, p)], Lbar[tri(j, p)]);
    }
}

// chol_pullback with each off-diagonal Abar[i][j] handed to pair(i, j, Abar[i][j]) when it is
// formed instead of stored, and the diagonal into sdiag; the same operations in the same order.
template <typename T, int N, typename F>
__device__ inline void chol_pullback_each(T (&Lbar)[N * (N + 1) / 2], const T (&L)[N * (N + 1) / 2],
                                          const T (&rd)[N - 1], T (&sdiag)[N], F&& pair) {
#pragma unroll
    for (int j = N - 1; j >= 0; --j) {
        const T ljj = L[tri(j, j)];
#pragma unroll
        for (int i = N - 1; i >= j + 1; --i) {
            const T lbij = Lbar[tri(i, j)];
            const T tbar = div_rcp(lbij, ljj, rd[j]);
            Lbar[tri(j, j)] -= div_rcp(lbij * L[tri(i, j)], ljj, rd[j]);
            pair(i, j, tbar);
#pragma unroll
            for (int p = 0; p < j; ++p) {
                Lbar[tri(i, p)] = num<T>::fma(-tbar, L[tri(j, p)], Lbar[tri(i, p)]);
                Lbar[tri(j, p)] = num<T>::fma(-tbar, L[tri(i, p)], Lbar[tri(j, p)]);
            }
        }
        const T sbar = j < N - 1 ? div_rcp(Lbar[tri(j, j)], T(2) * ljj, rd[j < N - 1 ? j : 0] * T(0.5))
                                 : Lbar[tri(j, j)] / (T(2) * ljj);
        sdiag[j] = sbar;
#pragma unroll
        for (int p = 0; p < j; ++p)
            Lbar[tri(j, p)] = num<T>::fma(-(T(2) * sbar), L[tri(j, p)], Lbar[tri(j, p)]);
    }
}

// ---- LDS staging of the table -----------------------------------------------------------
// Cooperative copy of the prepared table (entries + cell index) from global memory into LDS.
template <typename T>
__device__ inline void stage_table(TabEnt<T>* s_tab, uint16_t* s_acc,
                                   const TabEnt<T>* __restrict__ g_tab,
                                   const uint16_t* __restrict__ g_acc, const TabParams<T>& P) {
    for (int i = threadIdx.x; i < P.nb - 1; i += blockDim.x) s_tab[i] = g_tab[i];
    for (int i = threadIdx.x; i <= P.ucells; i += blockDim.x) s_acc[i] = g_acc[i];
    __syncthreads();
}

}  // namespace ggp
