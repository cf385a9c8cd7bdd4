// graphgp_oracle.cpp — TEST INFRASTRUCTURE ONLY.
//
// A CPU restatement of GraphGP.jl's fused per-point Vecchia refinement (the CPU dispatch path:
// src/cpu_native.jl, src/api.jl, src/orchestrate.jl, src/dense.jl, src/grad.jl,
// src/grad_generate_vals.jl and the primitives in src/interp.jl / src/linalg.jl). It is the
// parity checker for the HIP library and the CPU baseline timed beside it. Nothing in the
// product links or calls this file; only the tests, the smoke check and the benchmark's
// cpu_baseline leg load it.
//
// Arithmetic convention (what "the reference's arithmetic" means here): every expression that
// the reference evaluates under `@fastmath` with a multiply feeding an add/sub is written as an
// explicit fused multiply-add (LLVM contracts those); every other expression is evaluated as
// written, in IEEE arithmetic with correctly rounded division and square root. The file is
// compiled with -ffp-contract=off so the compiler adds no contraction of its own.
//
// Parity pinning of each function (checks live in tests/):
//   cov_lookup / cov_lookup_weights ... numpy.interp + exact-hit/clamp cases (test_interp.jl:7-18)
//   chol_lower / mean_vec_solve ........ numpy Cholesky + triangular solve (test_linalg.jl)
//   chol_pullback / chol_pullback_dyn .. finite differences + closed-form matrix adjoint
//   refine_* (logdet / inv / forward) .. small.npz and medium.npz f64/f32 JAX values
//   generate / generate_inv ............ generate_parity.npz (f64, non-identity permutation)
//   dense layer ........................ numpy Cholesky / slogdet on the same assembled matrix
//   refine_logdet_grad_vals ............ small.npz grad_logdet_vals64
//   refine_inv_loss_grad_vals .......... small.npz inv_loss64 / grad_inv_loss_vals64
//   generate_grad_xi ................... adjoint identity <vbar, G xi> = <G^T vbar, xi>,
//                                        and the dense matrix G built column by column
//   generate_grad_vals ................. central finite differences of <w, generate(vals)>
//
// Layouts (all 0-based): coords[p*D + d] (the reference's (D,N) column-major UInt32);
// neighbors[m*K + j] (the reference's (K,M) column-major, -1 = unset); offsets[b] exclusive
// ends with offsets[0] = n0 and offsets[last] = N; indices[tree_pos] = original_pos.

#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <vector>
#include <omp.h>

namespace {

struct Prob {
    const uint32_t* coords;
    const int64_t* neighbors;
    const int64_t* offsets;
    const int64_t* indices;
    int64_t n_offsets, n0, K, N, D, nbins;
    double scale;
    const void* bins;
    const void* vals;
    int nthreads;
    // anisotropic covariance (src/types.jl:15-20); aniso != 0 selects it over (bins, vals)
    int aniso;
    const void* sbins;  // spatial axis, ns entries
    const void* zbins;  // z axis, nz entries
    const void* grid;   // ns x nz, row-major: grid[i*nz + j] = K(sbins[i], zbins[j])
    int64_t ns, nz;
    double alpha;
    // Accumulate the d/dvals histograms in double instead of T, and evaluate the dense-layer
    // cotangents (the n0 x n0 Cholesky adjoint, K^-1, alpha) in double from the T factor. The
    // reference sums and evaluates both in T (src/grad.jl:32-87, src/dense.jl:153-252,
    // src/grad_generate_vals.jl:188-211), so the default mirrors it; the double mode removes
    // the rounding noise of very large point sets and of the O(n0^3) dense loops in T from
    // comparisons whose subject is the per-point arithmetic (the library evaluates the dense
    // cotangents in double).
    int acc64;
};

template <typename T> inline T eps_of();
template <> inline float eps_of<float>() { return std::numeric_limits<float>::epsilon(); }
template <> inline double eps_of<double>() { return std::numeric_limits<double>::epsilon(); }

// ---- src/interp.jl:10-34 -------------------------------------------------------------------
template <typename T>
inline int64_t search_lo(T r, const T* bins, int64_t n) {
    int64_t lo = 1, hi = n;  // 1-based, as the reference
    while (hi - lo > 1) {
        int64_t mid = (lo + hi) >> 1;
        if (bins[mid - 1] <= r) lo = mid; else hi = mid;
    }
    return lo - 1;  // 0-based
}

template <typename T>
inline T cov_lookup(T r, const T* bins, const T* vals, int64_t n) {
    if (r <= bins[0]) return vals[0];
    if (r >= bins[n - 1]) return vals[n - 1];
    int64_t lo = search_lo(r, bins, n);
    T x0 = bins[lo], x1 = bins[lo + 1], y0 = vals[lo], y1 = vals[lo + 1];
    T slope = (y1 - y0) / (x1 - x0);
    return std::fma(slope, r - x0, y0);  // @fastmath y0 + slope*(r - x0)
}

// ---- src/interp.jl:62-83 -------------------------------------------------------------------
template <typename T>
inline void cov_lookup_weights(T r, const T* bins, int64_t n, int64_t& lo, T& wlo, T& whi) {
    if (r <= bins[0]) { lo = 0; wlo = T(1); whi = T(0); return; }
    if (r >= bins[n - 1]) { lo = n - 2; wlo = T(0); whi = T(1); return; }
    lo = search_lo(r, bins, n);
    T x0 = bins[lo], x1 = bins[lo + 1];
    T t = (r - x0) / (x1 - x0);
    wlo = T(1) - t;
    whi = t;
}

// Lower triangle of an n x n row-major scratch: A[i*n + j], i >= j.
template <typename T>
struct Scratch {
    int64_t n, K, D;
    std::vector<T> A, Abar, Lbar, mv, zbar;
    std::vector<uint32_t> jc;
    Scratch(int64_t K_, int64_t D_)
        : n(K_ + 1), K(K_), D(D_), A((K_ + 1) * (K_ + 1)), Abar((K_ + 1) * (K_ + 1)),
          Lbar((K_ + 1) * (K_ + 1)), mv(K_), zbar(K_), jc((K_ + 1) * D_) {}
};

// ---- src/kernels.jl:9-23 --------------------------------------------------------------------
inline void gather_joint(uint32_t* jc, const Prob& p, int64_t m) {
    const int64_t K = p.K, D = p.D;
    for (int64_t j = 0; j < K; ++j) {
        int64_t nj = p.neighbors[m * K + j];
        for (int64_t d = 0; d < D; ++d) jc[j * D + d] = p.coords[nj * D + d];
    }
    int64_t fine = p.n0 + m;
    for (int64_t d = 0; d < D; ++d) jc[K * D + d] = p.coords[fine * D + d];
}

inline int64_t sqdist(const uint32_t* a, const uint32_t* b, int64_t D) {
    int64_t sq = 0;
    for (int64_t d = 0; d < D; ++d) {
        int64_t di = (int64_t)a[d] - (int64_t)b[d];
        sq += di * di;
    }
    return sq;
}

// ---- src/linalg.jl:15-29 --------------------------------------------------------------------
template <typename T>
inline void assemble_cov(T* A, const uint32_t* jc, int64_t n, int64_t D, T scale, const T* bins,
                         const T* vals, int64_t nb) {
    for (int64_t a = 0; a < n; ++a) {
        A[a * n + a] = cov_lookup(T(0), bins, vals, nb);
        for (int64_t b = 0; b < a; ++b) {
            int64_t sq = sqdist(jc + a * D, jc + b * D, D);
            T r = std::sqrt(T(sq)) * scale;
            A[a * n + b] = cov_lookup(r, bins, vals, nb);
        }
    }
}

// ---- src/aniso.jl:43-84 (no @fastmath in these functions) -------------------------------------
template <typename T>
inline T frac_index(T d, const T* bins, int64_t n) {
    if (d <= bins[0]) return T(0);
    if (d >= bins[n - 1]) return T(n - 1);
    const int64_t lo = search_lo(d, bins, n);
    const T x0 = bins[lo], x1 = bins[lo + 1];
    return T(lo) + (d - x0) / (x1 - x0);
}

template <typename T>
inline T aniso_lookup(T ds, T dz, const Prob& p) {
    const T* sb = (const T*)p.sbins; const T* zb = (const T*)p.zbins; const T* g = (const T*)p.grid;
    const int64_t ns = p.ns, nz = p.nz;
    const T fx = frac_index(ds, sb, ns), fz = frac_index(dz, zb, nz);
    const int64_t i0 = (int64_t)fx, j0 = (int64_t)fz;
    const int64_t i1 = i0 + 1 < ns ? i0 + 1 : ns - 1, j1 = j0 + 1 < nz ? j0 + 1 : nz - 1;
    const T tx = fx - T(i0), tz = fz - T(j0);
    const T g00 = g[i0 * nz + j0], g10 = g[i1 * nz + j0], g01 = g[i0 * nz + j1], g11 = g[i1 * nz + j1];
    return (g00 * (T(1) - tx) + g10 * tx) * (T(1) - tz) + (g01 * (T(1) - tx) + g11 * tx) * tz;
}

// Anisotropic pair covariance (src/aniso.jl:88-108): spatial distance over dims 0..D-2, radial
// |dz| * scale / alpha over the last dim.
template <typename T>
inline T aniso_pair(const uint32_t* a, const uint32_t* b, int64_t D, T scale, const Prob& p) {
    int64_t sqs = 0;
    for (int64_t d = 0; d < D - 1; ++d) {
        int64_t di = (int64_t)a[d] - (int64_t)b[d];
        sqs += di * di;
    }
    const int64_t dzi = (int64_t)a[D - 1] - (int64_t)b[D - 1];
    const T d_spatial = std::sqrt(T(sqs)) * scale;
    const T d_z = std::abs(T(dzi)) * scale / T(p.alpha);
    return aniso_lookup(d_spatial, d_z, p);
}

template <typename T>
inline void assemble_cov_aniso(T* A, const uint32_t* jc, int64_t n, int64_t D, T scale,
                               const Prob& p) {
    const T diagv = aniso_lookup(T(0), T(0), p);
    for (int64_t a = 0; a < n; ++a) {
        A[a * n + a] = diagv;
        for (int64_t b = 0; b < a; ++b) A[a * n + b] = aniso_pair(jc + a * D, jc + b * D, D, scale, p);
    }
}

// ---- src/linalg.jl:38-73 --------------------------------------------------------------------
template <typename T>
inline void chol_lower(T* A, int64_t n) {
    const T pivmin = eps_of<T>() * A[0];
    for (int64_t j = 0; j < n; ++j) {
        T s = A[j * n + j];
        for (int64_t p = 0; p < j; ++p) s = std::fma(-A[j * n + p], A[j * n + p], s);
        if (s > pivmin) {
            T d = std::sqrt(s);
            A[j * n + j] = d;
            for (int64_t i = j + 1; i < n; ++i) {
                T t = A[i * n + j];
                for (int64_t p = 0; p < j; ++p) t = std::fma(-A[i * n + p], A[j * n + p], t);
                A[i * n + j] = t / d;
            }
        } else {
            A[j * n + j] = std::sqrt(pivmin);
            for (int64_t i = j + 1; i < n; ++i) A[i * n + j] = T(0);
        }
    }
}

// ---- src/linalg.jl:85-103 -------------------------------------------------------------------
template <typename T>
inline void mean_vec_solve(T* x, const T* L, int64_t K) {
    const int64_t n = K + 1;
    const T pivfloor = T(1.5) * std::sqrt(eps_of<T>()) * L[0];
    for (int64_t i = K - 1; i >= 0; --i) {
        T d = L[i * n + i];
        if (d > pivfloor) {
            T s = L[K * n + i];
            for (int64_t j = i + 1; j < K; ++j) s = std::fma(-L[j * n + i], x[j], s);
            x[i] = s / d;
        } else {
            x[i] = T(0);
        }
    }
}

// ---- src/linalg.jl:112-137 (and the runtime-sized twin src/grad_generate_vals.jl:18-39, which
// is the same recurrence without @fastmath: `dyn` selects plain multiply-subtract). ------------
template <typename T, bool dyn>
inline void chol_pullback_impl(T* Abar, T* Lbar, const T* L, int64_t n) {
    for (int64_t j = n - 1; j >= 0; --j) {
        const T ljj = L[j * n + j];
        for (int64_t i = n - 1; i >= j + 1; --i) {
            const T lbij = Lbar[i * n + j];
            const T tbar = lbij / ljj;
            Lbar[j * n + j] -= lbij * L[i * n + j] / ljj;
            Abar[i * n + j] = tbar;
            for (int64_t p = 0; p < j; ++p) {
                if (dyn) {
                    Lbar[i * n + p] -= tbar * L[j * n + p];
                    Lbar[j * n + p] -= tbar * L[i * n + p];
                } else {
                    Lbar[i * n + p] = std::fma(-tbar, L[j * n + p], Lbar[i * n + p]);
                    Lbar[j * n + p] = std::fma(-tbar, L[i * n + p], Lbar[j * n + p]);
                }
            }
        }
        const T sbar = Lbar[j * n + j] / (T(2) * ljj);
        Abar[j * n + j] = sbar;
        for (int64_t p = 0; p < j; ++p) {
            if (dyn) Lbar[j * n + p] -= T(2) * sbar * L[j * n + p];
            else Lbar[j * n + p] = std::fma(-(T(2) * sbar), L[j * n + p], Lbar[j * n + p]);
        }
    }
}

template <typename T>
inline void zero_lbar(T* Lbar, int64_t n) {
    for (int64_t i = 0; i < n * n; ++i) Lbar[i] = T(0);
}

// Per-point forward pieces shared by every op (gather → assemble → factor).
template <typename T>
inline void factor_point(Scratch<T>& s, const Prob& p, int64_t m, T scale, const T* bins,
                         const T* vals) {
    gather_joint(s.jc.data(), p, m);
    if (p.aniso) assemble_cov_aniso(s.A.data(), s.jc.data(), s.n, p.D, scale, p);
    else assemble_cov(s.A.data(), s.jc.data(), s.n, p.D, scale, bins, vals, p.nbins);
    chol_lower(s.A.data(), s.n);
}

// Scatter a lower-triangle cotangent through the lookup weights into dv (dv[0] gets every
// diagonal, one add per row, as src/grad.jl:43-56). `r` without @fastmath there.
template <typename T, typename A>
inline void scatter_abar(A* dv, const Scratch<T>& s, T scale, const T* bins, int64_t nb, int64_t D) {
    const int64_t n = s.n;
    for (int64_t a = 0; a < n; ++a) {
        dv[0] += (A)s.Abar[a * n + a];
        for (int64_t b = 0; b < a; ++b) {
            int64_t sq = sqdist(s.jc.data() + a * D, s.jc.data() + b * D, D);
            T r = std::sqrt(T(sq)) * scale;
            int64_t lo; T wlo, whi;
            cov_lookup_weights(r, bins, nb, lo, wlo, whi);
            T g = s.Abar[a * n + b];
            dv[lo] += (A)(g * wlo);
            dv[lo + 1] += (A)(g * whi);
        }
    }
}

// Contiguous static chunks, one per thread (src/cpu_native.jl:18-31).
template <typename F>
void threaded_points(int64_t M, int nt, F&& body) {
    if (M <= 0) return;
    int64_t chunk = (M + nt - 1) / nt;
#pragma omp parallel num_threads(nt)
    {
        int t = omp_get_thread_num();
        int64_t lo = (int64_t)t * chunk, hi = std::min<int64_t>(lo + chunk, M);
        if (lo < hi) body(lo, hi);
    }
}

// ---- src/cpu_native.jl:33-44 ----------------------------------------------------------------
template <typename T>
void refine_logdet_terms(const Prob& p, T* terms) {
    const T* bins = (const T*)p.bins; const T* vals = (const T*)p.vals; const T scale = T(p.scale);
    const int64_t M = p.N - p.n0, K = p.K;
    threaded_points(M, p.nthreads, [&](int64_t lo, int64_t hi) {
        Scratch<T> s(K, p.D);
        for (int64_t m = lo; m < hi; ++m) {
            factor_point(s, p, m, scale, bins, vals);
            terms[m] = std::log(s.A[K * s.n + K]);
        }
    });
}

// ---- src/cpu_native.jl:46-63 ----------------------------------------------------------------
template <typename T>
void refine_inv(const Prob& p, const T* values, T* xi) {
    const T* bins = (const T*)p.bins; const T* vals = (const T*)p.vals; const T scale = T(p.scale);
    const int64_t M = p.N - p.n0, K = p.K, n0 = p.n0;
    threaded_points(M, p.nthreads, [&](int64_t lo, int64_t hi) {
        Scratch<T> s(K, p.D);
        for (int64_t m = lo; m < hi; ++m) {
            factor_point(s, p, m, scale, bins, vals);
            mean_vec_solve(s.mv.data(), s.A.data(), K);
            T mean = T(0);
            for (int64_t j = 0; j < K; ++j) mean += s.mv[j] * values[p.neighbors[m * K + j]];
            T sd = s.A[K * s.n + K];
            xi[m] = (values[n0 + m] - mean) / sd;
        }
    });
}

// ---- src/cpu_native.jl:65-84 ----------------------------------------------------------------
template <typename T>
void refine_meanvec_std(const Prob& p, T* mean_vec, T* sd) {
    const T* bins = (const T*)p.bins; const T* vals = (const T*)p.vals; const T scale = T(p.scale);
    const int64_t M = p.N - p.n0, K = p.K;
    threaded_points(M, p.nthreads, [&](int64_t lo, int64_t hi) {
        Scratch<T> s(K, p.D);
        for (int64_t m = lo; m < hi; ++m) {
            factor_point(s, p, m, scale, bins, vals);
            mean_vec_solve(s.mv.data(), s.A.data(), K);
            for (int64_t j = 0; j < K; ++j) mean_vec[m * K + j] = s.mv[j];
            sd[m] = s.A[K * s.n + K];
        }
    });
}

// ---- src/api.jl:113-141 + src/cpu_native.jl:86-112 (fused per-batch apply) ------------------
template <typename T>
void refine_meanvec_std(const Prob& p, T* mean_vec, T* sd);

template <typename T>
void refine(const Prob& p, T* values, const T* xi_ref) {
    const T* bins = (const T*)p.bins; const T* vals = (const T*)p.vals; const T scale = T(p.scale);
    const int64_t K = p.K, n0 = p.n0;
    if (p.aniso) {
        // src/api.jl:143-168: materialise mean_vec/std, then per batch acc = sum mv*v; v = acc + std*xi
        const int64_t M = p.N - n0;
        std::vector<T> mv(M * K > 0 ? M * K : 1), sd(M > 0 ? M : 1);
        refine_meanvec_std(p, mv.data(), sd.data());
        for (int64_t b = 1; b < p.n_offsets; ++b) {
            const int64_t m_lo = p.offsets[b - 1] - n0;
            const int64_t len = p.offsets[b] - p.offsets[b - 1];
            if (len <= 0) continue;
            threaded_points(len, p.nthreads, [&](int64_t lo, int64_t hi) {
                for (int64_t t = lo; t < hi; ++t) {
                    const int64_t m = m_lo + t;
                    T acc = T(0);
                    for (int64_t j = 0; j < K; ++j) acc += mv[m * K + j] * values[p.neighbors[m * K + j]];
                    values[n0 + m] = acc + sd[m] * xi_ref[m];
                }
            });
        }
        return;
    }
    for (int64_t b = 1; b < p.n_offsets; ++b) {
        const int64_t m_lo = p.offsets[b - 1] - n0;
        const int64_t len = p.offsets[b] - p.offsets[b - 1];
        if (len <= 0) continue;
        threaded_points(len, p.nthreads, [&](int64_t lo, int64_t hi) {
            Scratch<T> s(K, p.D);
            for (int64_t t = lo; t < hi; ++t) {
                const int64_t m = m_lo + t;
                factor_point(s, p, m, scale, bins, vals);
                mean_vec_solve(s.mv.data(), s.A.data(), K);
                T acc = s.A[K * s.n + K] * xi_ref[m];
                for (int64_t j = 0; j < K; ++j) acc += s.mv[j] * values[p.neighbors[m * K + j]];
                values[n0 + m] = acc;
            }
        });
    }
}

// ---- src/dense.jl:15-40 ---------------------------------------------------------------------
// Full symmetric n x n matrix, row-major (symmetric, so the layout is immaterial).
template <typename T>
void assemble_dense_cov(const Prob& p, int64_t n, T* Kd) {
    const T* bins = (const T*)p.bins; const T* vals = (const T*)p.vals; const T scale = T(p.scale);
    const int64_t D = p.D;
    if (p.aniso) {  // src/aniso.jl:222-247
        const T diagv = aniso_lookup(T(0), T(0), p);
        for (int64_t j = 0; j < n; ++j) {
            Kd[j * n + j] = diagv;
            for (int64_t i = j + 1; i < n; ++i) {
                const T v = aniso_pair(p.coords + i * D, p.coords + j * D, D, scale, p);
                Kd[i * n + j] = v;
                Kd[j * n + i] = v;
            }
        }
        return;
    }
    for (int64_t j = 0; j < n; ++j) {
        Kd[j * n + j] = cov_lookup(T(0), bins, vals, p.nbins);
        for (int64_t i = j + 1; i < n; ++i) {
            int64_t sq = sqdist(p.coords + i * D, p.coords + j * D, D);
            T r = std::sqrt(T(sq)) * scale;
            T v = cov_lookup(r, bins, vals, p.nbins);
            Kd[i * n + j] = v;
            Kd[j * n + i] = v;
        }
    }
}

// Unblocked lower Cholesky of the full matrix (LAPACK potrf semantics: fails on a
// non-positive or NaN pivot). Returns false on failure. L is written to the lower triangle of
// `L` (row-major), upper triangle zeroed.
template <typename T>
bool potrf_lower(const T* Kd, int64_t n, T* L) {
    for (int64_t i = 0; i < n * n; ++i) L[i] = T(0);
    for (int64_t i = 0; i < n; ++i)
        for (int64_t j = 0; j <= i; ++j) L[i * n + j] = Kd[i * n + j];
    for (int64_t j = 0; j < n; ++j) {
        T s = L[j * n + j];
        for (int64_t p = 0; p < j; ++p) s = std::fma(-L[j * n + p], L[j * n + p], s);
        if (!(s > T(0))) return false;
        T d = std::sqrt(s);
        L[j * n + j] = d;
        // Rows are independent within a column; each keeps its own fma chain in p order. Four
        // rows per iteration only interleave four independent chains.
        const int64_t r0 = j + 1, nr = n - r0, nq = (nr + 3) / 4;
#pragma omp parallel for schedule(static) if (nr > 256)
        for (int64_t q = 0; q < nq; ++q) {
            const int64_t i = r0 + 4 * q;
            const T* lj = L + j * n;
            if (i + 3 < n) {
                T* a = L + i * n; T* b = a + n; T* c = b + n; T* e = c + n;
                T t0 = a[j], t1 = b[j], t2 = c[j], t3 = e[j];
                for (int64_t p = 0; p < j; ++p) {
                    const T lp = lj[p];
                    t0 = std::fma(-a[p], lp, t0);
                    t1 = std::fma(-b[p], lp, t1);
                    t2 = std::fma(-c[p], lp, t2);
                    t3 = std::fma(-e[p], lp, t3);
                }
                a[j] = t0 / d; b[j] = t1 / d; c[j] = t2 / d; e[j] = t3 / d;
            } else {
                for (int64_t ii = i; ii < n; ++ii) {
                    T t = L[ii * n + j];
                    for (int64_t p = 0; p < j; ++p) t = std::fma(-L[ii * n + p], lj[p], t);
                    L[ii * n + j] = t / d;
                }
            }
        }
    }
    return true;
}

// ---- src/dense.jl:46-67 (jitter retry) ------------------------------------------------------
template <typename T>
bool dense_chol_L(const T* Kd, int64_t n, T* L) {
    if (potrf_lower(Kd, n, L)) return true;
    T dmean = T(0);
    for (int64_t i = 0; i < n; ++i) dmean += Kd[i * n + i];
    dmean = dmean / T(n > 1 ? n : 1);
    std::vector<T> Kj(Kd, Kd + n * n);
    T e = T(1e-9);
    while (e <= T(1e-2)) {
        for (int64_t i = 0; i < n; ++i) Kj[i * n + i] = Kd[i * n + i] + e * dmean;
        if (potrf_lower(Kj.data(), n, L)) return true;
        e *= T(10);
    }
    return false;
}

template <typename T>
bool dense_factor(const Prob& p, std::vector<T>& L) {
    const int64_t n = p.n0;
    std::vector<T> Kd(n * n);
    assemble_dense_cov(p, n, Kd.data());
    L.assign(n * n, T(0));
    return dense_chol_L(Kd.data(), n, L.data());
}

// L * x (dense.jl:118), forward substitution L \ v (dense.jl:134), L^T * v (grad.jl:457).
template <typename T>
void trmv_lower(const T* L, int64_t n, const T* x, T* y) {
    for (int64_t i = 0; i < n; ++i) {
        T acc = T(0);
        for (int64_t j = 0; j <= i; ++j) acc = std::fma(L[i * n + j], x[j], acc);
        y[i] = acc;
    }
}
template <typename T>
void trsv_lower(const T* L, int64_t n, const T* b, T* x) {
    for (int64_t i = 0; i < n; ++i) {
        T s = b[i];
        for (int64_t j = 0; j < i; ++j) s = std::fma(-L[i * n + j], x[j], s);
        x[i] = s / L[i * n + i];
    }
}
template <typename T>
void trmv_lower_t(const T* L, int64_t n, const T* x, T* y) {
    for (int64_t i = 0; i < n; ++i) {
        T acc = T(0);
        for (int64_t j = i; j < n; ++j) acc = std::fma(L[j * n + i], x[j], acc);
        y[i] = acc;
    }
}
template <typename T>
void trsv_lower_t(const T* L, int64_t n, const T* b, T* x) {
    for (int64_t i = n - 1; i >= 0; --i) {
        T s = b[i];
        for (int64_t j = i + 1; j < n; ++j) s = std::fma(-L[j * n + i], x[j], s);
        x[i] = s / L[i * n + i];
    }
}

// Scatter a dense lower-triangle cotangent G[a][b] (a >= b) into dv through lookup weights.
template <typename T>
void dense_scatter(const Prob& p, int64_t n, const T* G, T* dv) {
    const T* bins = (const T*)p.bins; const T scale = T(p.scale);
    const int64_t D = p.D;
    for (int64_t b = 0; b < n; ++b)
        for (int64_t a = b; a < n; ++a) {
            int64_t sq = sqdist(p.coords + a * D, p.coords + b * D, D);
            T r = std::sqrt(T(sq)) * scale;
            int64_t lo; T wlo, whi;
            cov_lookup_weights(r, bins, p.nbins, lo, wlo, whi);
            T g = G[a * n + b];
            dv[lo] += g * wlo;
            dv[lo + 1] += g * whi;
        }
}

// dense_scatter with a double cotangent and double accumulation (radii and weights in T, as
// the reference computes them).
template <typename T>
void dense_scatter64(const Prob& p, int64_t n, const double* G, double* dv) {
    const T* bins = (const T*)p.bins; const T scale = T(p.scale);
    const int64_t D = p.D;
    for (int64_t b = 0; b < n; ++b)
        for (int64_t a = b; a < n; ++a) {
            int64_t sq = sqdist(p.coords + a * D, p.coords + b * D, D);
            T r = std::sqrt(T(sq)) * scale;
            int64_t lo; T wlo, whi;
            cov_lookup_weights(r, bins, p.nbins, lo, wlo, whi);
            const double g = G[a * n + b];
            dv[lo] += g * (double)wlo;
            dv[lo + 1] += g * (double)whi;
        }
}

// The dense logdet and inverse-loss cotangents of src/dense.jl:153-183 / 229-252 in double,
// from the T factor (the acc64 mode).
template <typename T>
void dense_logdet_grad_vals64(const Prob& p, const std::vector<T>& L, double* dv) {
    const int64_t n = p.n0;
    std::vector<double> Ld(L.begin(), L.end()), Linv(n * n, 0.0), e(n), col(n), G(n * n, 0.0);
    for (int64_t c = 0; c < n; ++c) {
        for (int64_t i = 0; i < n; ++i) e[i] = i == c ? 1.0 : 0.0;
        trsv_lower(Ld.data(), n, e.data(), col.data());
        for (int64_t i = 0; i < n; ++i) Linv[i * n + c] = col[i];
    }
    for (int64_t b = 0; b < n; ++b)
        for (int64_t a = b; a < n; ++a) {
            double kinv = 0.0;
            for (int64_t kk = 0; kk < n; ++kk) kinv += Linv[kk * n + a] * Linv[kk * n + b];
            G[a * n + b] = a == b ? 0.5 * kinv : kinv;
        }
    dense_scatter64<T>(p, n, G.data(), dv);
}
template <typename T>
void dense_inv_loss_grad_vals64(const Prob& p, const std::vector<T>& L, const T* y, double* dv,
                                double* xi_out) {
    const int64_t n = p.n0;
    std::vector<double> Ld(L.begin(), L.end()), yd(y, y + n), alpha(n), G(n * n, 0.0);
    trsv_lower(Ld.data(), n, yd.data(), xi_out);
    trsv_lower_t(Ld.data(), n, xi_out, alpha.data());
    for (int64_t b = 0; b < n; ++b)
        for (int64_t a = b; a < n; ++a)
            G[a * n + b] = a == b ? -0.5 * alpha[a] * alpha[a] : -alpha[a] * alpha[b];
    dense_scatter64<T>(p, n, G.data(), dv);
}

// ---- src/dense.jl:153-183 -------------------------------------------------------------------
template <typename T>
void dense_logdet_grad_vals(const Prob& p, const std::vector<T>& L, T* dv) {
    const int64_t n = p.n0;
    // Linv = inv(LowerTriangular(L)) column by column.
    std::vector<T> Linv(n * n, T(0)), e(n), col(n);
    for (int64_t c = 0; c < n; ++c) {
        for (int64_t i = 0; i < n; ++i) e[i] = T(i == c ? 1 : 0);
        trsv_lower(L.data(), n, e.data(), col.data());
        for (int64_t i = 0; i < n; ++i) Linv[i * n + c] = col[i];
    }
    std::vector<T> G(n * n, T(0));
    for (int64_t b = 0; b < n; ++b)
        for (int64_t a = b; a < n; ++a) {
            T kinv = T(0);
            for (int64_t kk = 0; kk < n; ++kk) kinv += Linv[kk * n + a] * Linv[kk * n + b];
            G[a * n + b] = a == b ? T(0.5) * kinv : kinv;
        }
    dense_scatter(p, n, G.data(), dv);
}

// ---- src/dense.jl:229-252 -------------------------------------------------------------------
template <typename T>
void dense_inv_loss_grad_vals(const Prob& p, const std::vector<T>& L, const T* y, T* dv, T* xi_out) {
    const int64_t n = p.n0;
    std::vector<T> alpha(n);
    trsv_lower(L.data(), n, y, xi_out);
    trsv_lower_t(L.data(), n, xi_out, alpha.data());
    std::vector<T> G(n * n, T(0));
    for (int64_t b = 0; b < n; ++b)
        for (int64_t a = b; a < n; ++a)
            G[a * n + b] = a == b ? -T(0.5) * alpha[a] * alpha[a] : -alpha[a] * alpha[b];
    dense_scatter(p, n, G.data(), dv);
}

// ---- src/orchestrate.jl:19-42 ---------------------------------------------------------------
template <typename T>
int generate(const Prob& p, const T* xi, T* out) {
    const int64_t N = p.N, n0 = p.n0;
    std::vector<T> xo(N), v(N, T(0)), L;
    for (int64_t i = 0; i < N; ++i) xo[i] = p.indices ? xi[p.indices[i]] : xi[i];
    if (!dense_factor(p, L)) return 6;
    trmv_lower(L.data(), n0, xo.data(), v.data());
    refine(p, v.data(), xo.data() + n0);
    for (int64_t i = 0; i < N; ++i) {
        if (p.indices) out[p.indices[i]] = v[i]; else out[i] = v[i];
    }
    return 0;
}

// ---- src/orchestrate.jl:53-81 ---------------------------------------------------------------
template <typename T>
int generate_inv(const Prob& p, const T* values, T* xi_out) {
    const int64_t N = p.N, n0 = p.n0;
    std::vector<T> vo(N), xi(N, T(0)), L;
    for (int64_t i = 0; i < N; ++i) vo[i] = p.indices ? values[p.indices[i]] : values[i];
    refine_inv(p, vo.data(), xi.data() + n0);
    if (!dense_factor(p, L)) return 6;
    trsv_lower(L.data(), n0, vo.data(), xi.data());
    for (int64_t i = 0; i < N; ++i) {
        if (p.indices) xi_out[p.indices[i]] = xi[i]; else xi_out[i] = xi[i];
    }
    return 0;
}

// ---- src/orchestrate.jl:89-97 (+ dense.jl:142-147) ------------------------------------------
template <typename T>
int generate_logdet(const Prob& p, double* out) {
    std::vector<T> L;
    if (!dense_factor(p, L)) return 6;
    T ld_dense = T(0);
    for (int64_t i = 0; i < p.n0; ++i) ld_dense += std::log(L[i * p.n0 + i]);
    const int64_t M = p.N - p.n0;
    std::vector<T> terms(M > 0 ? M : 1);
    refine_logdet_terms(p, terms.data());
    T ld_ref = T(0);
    for (int64_t m = 0; m < M; ++m) ld_ref += terms[m];
    *out = (double)(ld_dense + ld_ref);
    return 0;
}

// ---- src/grad.jl:32-87 (privatized per-task histograms, summed in task order) ----------------
template <typename T>
void refine_logdet_grad_vals(const Prob& p, T* dvals, double* logdet) {
    const T* bins = (const T*)p.bins; const T* vals = (const T*)p.vals; const T scale = T(p.scale);
    const int64_t M = p.N - p.n0, K = p.K, nb = p.nbins;
    int nch = (int)std::max<int64_t>(1, std::min<int64_t>(p.nthreads, M));
    std::vector<std::vector<T>> dvs(nch, std::vector<T>(p.acc64 ? 0 : nb, T(0)));
    std::vector<std::vector<double>> dvs64(nch, std::vector<double>(p.acc64 ? nb : 0, 0.0));
    std::vector<T> lds(nch, T(0));
    if (M > 0) {
        int64_t chunk = (M + nch - 1) / nch;
#pragma omp parallel for num_threads(p.nthreads) schedule(static, 1)
        for (int c = 0; c < nch; ++c) {
            Scratch<T> s(K, p.D);
            int64_t lo = c * chunk, hi = std::min<int64_t>(lo + chunk, M);
            for (int64_t m = lo; m < hi; ++m) {
                factor_point(s, p, m, scale, bins, vals);
                T ldt = std::log(s.A[K * s.n + K]);
                zero_lbar(s.Lbar.data(), s.n);
                s.Lbar[K * s.n + K] = T(1) / s.A[K * s.n + K];  // linalg.jl:140-146, seed 1
                chol_pullback_impl<T, false>(s.Abar.data(), s.Lbar.data(), s.A.data(), s.n);
                if (p.acc64) scatter_abar(dvs64[c].data(), s, scale, bins, nb, p.D);
                else scatter_abar(dvs[c].data(), s, scale, bins, nb, p.D);
                lds[c] += ldt;
            }
        }
    }
    T ld = T(0);
    for (int64_t i = 0; i < nb; ++i) dvals[i] = T(0);
    for (int c = 0; c < nch; ++c) {
        ld += lds[c];
        if (!p.acc64)
            for (int64_t i = 0; i < nb; ++i) dvals[i] += dvs[c][i];
    }
    if (p.acc64)
        for (int64_t i = 0; i < nb; ++i) {
            double t = 0.0;
            for (int c = 0; c < nch; ++c) t += dvs64[c][i];
            dvals[i] = (T)t;
        }
    if (logdet) *logdet = (double)ld;
}

// ---- src/grad.jl:680-715 (CPU branch) = generate_logdet_grad_vals (grad.jl:149-154) ---------
template <typename T>
int generate_logdet_grad_vals(const Prob& p, T* dvals, double* logdet) {
    double ld_ref = 0;
    refine_logdet_grad_vals(p, dvals, &ld_ref);
    std::vector<T> L;
    if (!dense_factor(p, L)) return 6;
    if (p.acc64) {
        std::vector<double> dd(p.nbins, 0.0);
        dense_logdet_grad_vals64(p, L, dd.data());
        for (int64_t i = 0; i < p.nbins; ++i) dvals[i] = (T)(dd[i] + (double)dvals[i]);
    } else {
        std::vector<T> dd(p.nbins, T(0));
        dense_logdet_grad_vals(p, L, dd.data());
        for (int64_t i = 0; i < p.nbins; ++i) dvals[i] = dd[i] + dvals[i];
    }
    T ld_dense = T(0);
    for (int64_t i = 0; i < p.n0; ++i) ld_dense += std::log(L[i * p.n0 + i]);
    if (logdet) *logdet = (double)(ld_dense + (T)ld_ref);
    return 0;
}

// ---- src/grad.jl:533-626 (refine_inv_loss_grad_vals, CPU) -----------------------------------
// Per-point backward of 0.5*xi_m^2 (src/kernels_adjoint.jl:183-211; the same seeds in
// src/grad.jl:280-300): factor, seed the factor cotangents, Cholesky pullback into s.Abar.
// Returns xi_m.
template <typename T>
T inv_loss_point_pullback(Scratch<T>& s, const Prob& p, int64_t m, const T* values, T scale,
                          const T* bins, const T* vals) {
    const int64_t K = p.K, n0 = p.n0, n = s.n;
    factor_point(s, p, m, scale, bins, vals);
    mean_vec_solve(s.mv.data(), s.A.data(), K);
    const T sd = s.A[K * n + K];
    T mean_val = T(0);
    for (int64_t j = 0; j < K; ++j) mean_val += s.mv[j] * values[p.neighbors[m * K + j]];
    const T xi_m = (values[n0 + m] - mean_val) / sd;
    zero_lbar(s.Lbar.data(), n);
    s.Lbar[K * n + K] = -xi_m * xi_m / sd;
    for (int64_t j = 0; j < K; ++j) s.zbar[j] = -xi_m * values[p.neighbors[m * K + j]] / sd;
    for (int64_t i = 0; i < K; ++i) {
        T t = s.zbar[i];
        for (int64_t q = 0; q < i; ++q) t -= s.A[i * n + q] * s.zbar[q];
        s.zbar[i] = t / s.A[i * n + i];
    }
    for (int64_t j = 0; j < K; ++j) {
        s.Lbar[K * n + j] += s.zbar[j];
        for (int64_t i = 0; i <= j; ++i) s.Lbar[j * n + i] -= s.zbar[i] * s.mv[j];
    }
    chol_pullback_impl<T, false>(s.Abar.data(), s.Lbar.data(), s.A.data(), n);
    return xi_m;
}

template <typename T>
void refine_inv_loss_grad_vals(const Prob& p, const T* values, T* dvals, double* loss) {
    const T* bins = (const T*)p.bins; const T* vals = (const T*)p.vals; const T scale = T(p.scale);
    const int64_t M = p.N - p.n0, K = p.K, nb = p.nbins;
    int nch = (int)std::max<int64_t>(1, std::min<int64_t>(p.nthreads, M));
    std::vector<std::vector<T>> dvs(nch, std::vector<T>(p.acc64 ? 0 : nb, T(0)));
    std::vector<std::vector<double>> dvs64(nch, std::vector<double>(p.acc64 ? nb : 0, 0.0));
    std::vector<T> ls(nch, T(0));
    if (M > 0) {
        int64_t chunk = (M + nch - 1) / nch;
#pragma omp parallel for num_threads(p.nthreads) schedule(static, 1)
        for (int c = 0; c < nch; ++c) {
            Scratch<T> s(K, p.D);
            int64_t lo = c * chunk, hi = std::min<int64_t>(lo + chunk, M);
            for (int64_t m = lo; m < hi; ++m) {
                const T xi_m = inv_loss_point_pullback(s, p, m, values, scale, bins, vals);
                if (p.acc64) scatter_abar(dvs64[c].data(), s, scale, bins, nb, p.D);
                else scatter_abar(dvs[c].data(), s, scale, bins, nb, p.D);
                ls[c] += xi_m * xi_m / T(2);
            }
        }
    }
    T l = T(0);
    for (int64_t i = 0; i < nb; ++i) dvals[i] = T(0);
    for (int c = 0; c < nch; ++c) {
        l += ls[c];
        if (!p.acc64)
            for (int64_t i = 0; i < nb; ++i) dvals[i] += dvs[c][i];
    }
    if (p.acc64)
        for (int64_t i = 0; i < nb; ++i) {
            double t = 0.0;
            for (int c = 0; c < nch; ++c) t += dvs64[c][i];
            dvals[i] = (T)t;
        }
    if (loss) *loss = (double)l;
}

// ---- src/grad.jl:514-529 --------------------------------------------------------------------
template <typename T>
int generate_inv_loss_grad_vals(const Prob& p, const T* data, T* dvals, double* loss) {
    const int64_t N = p.N, n0 = p.n0;
    std::vector<T> d(N);
    for (int64_t i = 0; i < N; ++i) d[i] = p.indices ? data[p.indices[i]] : data[i];
    std::vector<T> L;
    if (!dense_factor(p, L)) return 6;
    double ref_loss = 0;
    if (p.acc64) {
        std::vector<double> xid(n0), gd(p.nbins, 0.0);
        dense_inv_loss_grad_vals64(p, L, d.data(), gd.data(), xid.data());
        double dense_loss = 0.0;
        for (int64_t i = 0; i < n0; ++i) dense_loss += xid[i] * xid[i];
        refine_inv_loss_grad_vals(p, d.data(), dvals, &ref_loss);
        for (int64_t i = 0; i < p.nbins; ++i) dvals[i] = (T)((double)dvals[i] + gd[i]);
        if (loss) *loss = dense_loss / 2.0 + ref_loss;
        return 0;
    }
    std::vector<T> xid(n0), gd(p.nbins, T(0));
    dense_inv_loss_grad_vals(p, L, d.data(), gd.data(), xid.data());
    T dense_loss = T(0);
    for (int64_t i = 0; i < n0; ++i) dense_loss += xid[i] * xid[i];
    dense_loss = dense_loss / T(2);
    refine_inv_loss_grad_vals(p, d.data(), dvals, &ref_loss);
    for (int64_t i = 0; i < p.nbins; ++i) dvals[i] = dvals[i] + gd[i];
    if (loss) *loss = (double)(dense_loss + (T)ref_loss);
    return 0;
}

// ---- src/grad.jl:392-464 (CPU path: meanvec pass, serial reverse sweep, dense L^T) -----------
template <typename T>
int generate_grad_xi(const Prob& p, const T* vbar, T* xbar) {
    const int64_t N = p.N, n0 = p.n0, K = p.K, M = N - n0;
    std::vector<T> mv(M * K > 0 ? M * K : 1), sd(M > 0 ? M : 1);
    refine_meanvec_std(p, mv.data(), sd.data());
    std::vector<T> vb(N), xg(N, T(0));
    for (int64_t i = 0; i < N; ++i) vb[i] = p.indices ? vbar[p.indices[i]] : vbar[i];
    for (int64_t b = p.n_offsets - 1; b >= 1; --b) {
        const int64_t lo = p.offsets[b - 1], hi = p.offsets[b];
        for (int64_t q = hi - 1; q >= lo; --q) {
            const int64_t m = q - n0;
            xg[q] = sd[m] * vb[q];
            for (int64_t j = 0; j < K; ++j) {
                int64_t nbj = p.neighbors[m * K + j];
                if (nbj < 0) continue;
                vb[nbj] += mv[m * K + j] * vb[q];
            }
        }
    }
    std::vector<T> L;
    if (!dense_factor(p, L)) return 6;
    trmv_lower_t(L.data(), n0, vb.data(), xg.data());
    for (int64_t i = 0; i < N; ++i) {
        if (p.indices) xbar[p.indices[i]] = xg[i]; else xbar[i] = xg[i];
    }
    return 0;
}

// ---- src/grad_generate_vals.jl:111-212 (CPU path) -------------------------------------------
template <typename T>
int generate_grad_vals(const Prob& p, const T* xi, const T* vbar, T* dvals) {
    const T* bins = (const T*)p.bins; const T* vals = (const T*)p.vals; const T scale = T(p.scale);
    const int64_t N = p.N, n0 = p.n0, K = p.K, M = N - n0, nb = p.nbins, D = p.D;
    std::vector<T> mv(M * K > 0 ? M * K : 1), sd(M > 0 ? M : 1);
    refine_meanvec_std(p, mv.data(), sd.data());
    std::vector<T> xih(N), vb(N), v(N, T(0)), L;
    for (int64_t i = 0; i < N; ++i) xih[i] = p.indices ? xi[p.indices[i]] : xi[i];
    if (!dense_factor(p, L)) return 6;
    trmv_lower(L.data(), n0, xih.data(), v.data());
    // Serial forward (grad_generate_vals.jl:149-161): sum mv*v first, add std*xi last.
    for (int64_t b = 1; b < p.n_offsets; ++b)
        for (int64_t q = p.offsets[b - 1]; q < p.offsets[b]; ++q) {
            const int64_t m = q - n0;
            T acc = T(0);
            for (int64_t j = 0; j < K; ++j) {
                int64_t nbj = p.neighbors[m * K + j];
                if (nbj >= 0) acc += mv[m * K + j] * v[nbj];
            }
            v[q] = acc + sd[m] * xih[q];
        }
    for (int64_t i = 0; i < N; ++i) vb[i] = p.indices ? vbar[p.indices[i]] : vbar[i];
    for (int64_t i = 0; i < nb; ++i) dvals[i] = T(0);
    std::vector<double> dv64(p.acc64 ? nb : 0, 0.0);
    auto add = [&](int64_t bin, T g) {
        if (p.acc64) dv64[bin] += (double)g;
        else dvals[bin] += g;
    };
    Scratch<T> s(K, D);
    const int64_t n = s.n;
    const T pivfloor_c = T(1.5) * std::sqrt(eps_of<T>());
    // Reverse sweep with the per-point pullback (grad_generate_vals.jl:44-103, 175-186).
    for (int64_t b = p.n_offsets - 1; b >= 1; --b)
        for (int64_t q = p.offsets[b] - 1; q >= p.offsets[b - 1]; --q) {
            const int64_t m = q - n0;
            const T vbp = vb[q];
            const T stdbar = vbp * xih[q];
            factor_point(s, p, m, scale, bins, vals);
            mean_vec_solve(s.mv.data(), s.A.data(), K);
            const T pivfloor = pivfloor_c * s.A[0];
            zero_lbar(s.Lbar.data(), n);
            s.Lbar[K * n + K] = stdbar;
            for (int64_t j = 0; j < K; ++j) s.zbar[j] = vbp * v[p.neighbors[m * K + j]];
            for (int64_t i = 0; i < K; ++i) {
                if (s.A[i * n + i] > pivfloor) {
                    T t = s.zbar[i];
                    for (int64_t r = 0; r < i; ++r) t -= s.A[i * n + r] * s.zbar[r];
                    s.zbar[i] = t / s.A[i * n + i];
                } else {
                    s.zbar[i] = T(0);
                }
            }
            for (int64_t j = 0; j < K; ++j) {
                s.Lbar[K * n + j] += s.zbar[j];
                for (int64_t i = 0; i <= j; ++i) s.Lbar[j * n + i] -= s.zbar[i] * s.mv[j];
            }
            chol_pullback_impl<T, false>(s.Abar.data(), s.Lbar.data(), s.A.data(), n);
            if (p.acc64) scatter_abar(dv64.data(), s, scale, bins, nb, D);
            else scatter_abar(dvals, s, scale, bins, nb, D);
            for (int64_t j = 0; j < K; ++j) {
                int64_t nbj = p.neighbors[m * K + j];
                if (nbj >= 0) vb[nbj] += mv[m * K + j] * vbp;
            }
        }
    // Dense backward (grad_generate_vals.jl:188-211); with acc64 in double from the T factor.
    if (p.acc64) {
        std::vector<double> Ld(L.begin(), L.end()), Lb(n0 * n0, 0.0), Kb(n0 * n0, 0.0);
        for (int64_t j = 0; j < n0; ++j)
            for (int64_t i = j; i < n0; ++i) Lb[i * n0 + j] = (double)vb[i] * (double)xih[j];
        chol_pullback_impl<double, true>(Kb.data(), Lb.data(), Ld.data(), n0);
        for (int64_t j = 0; j < n0; ++j)
            for (int64_t i = j + 1; i < n0; ++i) Kb[j * n0 + i] = 0.0;  // lower triangle only
        for (int64_t j = 0; j < n0; ++j) {
            dv64[0] += Kb[j * n0 + j];
            for (int64_t i = j + 1; i < n0; ++i) {
                int64_t sq = sqdist(p.coords + i * D, p.coords + j * D, D);
                T r = std::sqrt(T(sq)) * scale;
                int64_t lo; T wlo, whi;
                cov_lookup_weights(r, bins, nb, lo, wlo, whi);
                const double g = Kb[i * n0 + j];
                dv64[lo] += g * (double)wlo;
                dv64[lo + 1] += g * (double)whi;
            }
        }
        for (int64_t i = 0; i < nb; ++i) dvals[i] = (T)dv64[i];
        return 0;
    }
    std::vector<T> Lbar_d(n0 * n0, T(0)), Kbar_d(n0 * n0, T(0));
    for (int64_t j = 0; j < n0; ++j)
        for (int64_t i = j; i < n0; ++i) Lbar_d[i * n0 + j] = vb[i] * xih[j];
    chol_pullback_impl<T, true>(Kbar_d.data(), Lbar_d.data(), L.data(), n0);
    for (int64_t j = 0; j < n0; ++j) {
        add(0, Kbar_d[j * n0 + j]);
        for (int64_t i = j + 1; i < n0; ++i) {
            int64_t sq = sqdist(p.coords + i * D, p.coords + j * D, D);
            T r = std::sqrt(T(sq)) * scale;
            int64_t lo; T wlo, whi;
            cov_lookup_weights(r, bins, nb, lo, wlo, whi);
            T g = Kbar_d[i * n0 + j];
            add(lo, g * wlo);
            add(lo + 1, g * whi);
        }
    }
    if (p.acc64)
        for (int64_t i = 0; i < nb; ++i) dvals[i] = (T)dv64[i];
    return 0;
}

// ================================ point-position gradients ====================================
// ---- src/interp.jl:43-60: d cov / d r, the bracketing segment's slope (0 outside the table) --
template <typename T>
inline T cov_lookup_dr(T r, const T* bins, const T* vals, int64_t n) {
    if (r <= bins[0] || r >= bins[n - 1]) return T(0);
    const int64_t lo = search_lo(r, bins, n);
    return (vals[lo + 1] - vals[lo]) / (bins[lo + 1] - bins[lo]);
}

// Off-diagonal cotangent g of the pair (ga, gb) at lattice coordinates (ca, cb) through
// k'(r) dr/dx into both points (src/grad.jl:205-225): coincident pairs and pairs outside the
// table's range contribute nothing. dp is point-major (D per point), tree order.
template <typename T, typename A>
inline void pair_to_points(A* dp, int64_t ga, int64_t gb, const uint32_t* ca, const uint32_t* cb,
                           int64_t D, T g, T scale, const T* bins, const T* vals, int64_t nb) {
    const int64_t sq = sqdist(ca, cb, D);
    if (sq == 0) return;
    const T r = std::sqrt(T(sq)) * scale;
    const T dcov = cov_lookup_dr(r, bins, vals, nb);
    if (dcov == T(0)) return;
    const T factor = g * dcov / r;
    for (int64_t dd = 0; dd < D; ++dd) {
        const T diff = scale * (T((int64_t)ca[dd]) - T((int64_t)cb[dd]));
        const T c = factor * diff;
        dp[ga * D + dd] += (A)c;
        dp[gb * D + dd] -= (A)c;
    }
}

// Abar of one refined point m into its k+1 points.
template <typename T, typename A>
inline void scatter_points(A* dp, const Scratch<T>& s, const Prob& p, int64_t m, T scale,
                           const T* bins, const T* vals) {
    const int64_t n = s.n, K = p.K, D = p.D;
    for (int64_t a = 1; a < n; ++a) {
        const int64_t ga = a < K ? p.neighbors[m * K + a] : p.n0 + m;
        for (int64_t b = 0; b < a; ++b) {
            const int64_t gb = b < K ? p.neighbors[m * K + b] : p.n0 + m;
            pair_to_points(dp, ga, gb, s.jc.data() + a * D, s.jc.data() + b * D, D,
                           s.Abar[a * n + b], scale, bins, vals, p.nbins);
        }
    }
}

// Serial over the refined points in order, as the reference's host loops; dp (N x D) is summed
// in T, or in double with acc64.
template <typename T, typename F>
void refine_points_loop(const Prob& p, T* dp, F&& seed_pullback) {
    const T* bins = (const T*)p.bins; const T* vals = (const T*)p.vals; const T scale = T(p.scale);
    const int64_t M = p.N - p.n0, N = p.N, D = p.D;
    std::vector<double> dp64(p.acc64 ? N * D : 0, 0.0);
    for (int64_t i = 0; i < N * D; ++i) dp[i] = T(0);
    Scratch<T> s(p.K, p.D);
    for (int64_t m = 0; m < M; ++m) {
        seed_pullback(s, m, scale, bins, vals);
        if (p.acc64) scatter_points(dp64.data(), s, p, m, scale, bins, vals);
        else scatter_points(dp, s, p, m, scale, bins, vals);
    }
    if (p.acc64)
        for (int64_t i = 0; i < N * D; ++i) dp[i] = (T)dp64[i];
}

// ---- src/grad.jl:168-226 --------------------------------------------------------------------
template <typename T>
void refine_logdet_grad_points(const Prob& p, T* dp, double* logdet) {
    double ld = 0.0;
    const int64_t K = p.K;
    refine_points_loop(p, dp, [&](Scratch<T>& s, int64_t m, T scale, const T* bins, const T* vals) {
        factor_point(s, p, m, scale, bins, vals);
        const T sd = s.A[K * s.n + K];
        ld += (double)std::log(sd);
        zero_lbar(s.Lbar.data(), s.n);
        s.Lbar[K * s.n + K] = T(1) / sd;  // linalg.jl:140-146, seed 1
        chol_pullback_impl<T, false>(s.Abar.data(), s.Lbar.data(), s.A.data(), s.n);
    });
    if (logdet) *logdet = ld;
}

// ---- src/grad.jl:239-319 --------------------------------------------------------------------
template <typename T>
void refine_inv_loss_grad_points(const Prob& p, const T* values, T* dp, double* loss) {
    double l = 0.0;
    refine_points_loop(p, dp, [&](Scratch<T>& s, int64_t m, T scale, const T* bins, const T* vals) {
        const T xi_m = inv_loss_point_pullback(s, p, m, values, scale, bins, vals);
        l += (double)(xi_m * xi_m / T(2));
    });
    if (loss) *loss = l;
}

// Dense off-diagonal cotangents G[a][b] (a > b) into the first n0 points (src/dense.jl:185-222,
// 268-300).
template <typename T>
void dense_points_scatter(const Prob& p, const std::vector<T>& G, T* dp) {
    const T* bins = (const T*)p.bins; const T* vals = (const T*)p.vals; const T scale = T(p.scale);
    const int64_t n = p.n0, D = p.D;
    std::vector<double> dp64(p.acc64 ? n * D : 0, 0.0);
    for (int64_t b = 0; b < n; ++b)
        for (int64_t a = b + 1; a < n; ++a) {
            if (p.acc64)
                pair_to_points(dp64.data(), a, b, p.coords + a * D, p.coords + b * D, D,
                               G[a * n + b], scale, bins, vals, p.nbins);
            else
                pair_to_points(dp, a, b, p.coords + a * D, p.coords + b * D, D, G[a * n + b],
                               scale, bins, vals, p.nbins);
        }
    if (p.acc64)
        for (int64_t i = 0; i < n * D; ++i) dp[i] += (T)dp64[i];
}

// ---- src/dense.jl:185-222: cotangent K^-1[a][b] ----------------------------------------------
template <typename T>
void dense_logdet_grad_points(const Prob& p, const std::vector<T>& L, T* dp) {
    const int64_t n = p.n0;
    std::vector<T> Linv(n * n, T(0)), e(n), col(n), G(n * n, T(0));
    for (int64_t c = 0; c < n; ++c) {
        for (int64_t i = 0; i < n; ++i) e[i] = T(i == c ? 1 : 0);
        trsv_lower(L.data(), n, e.data(), col.data());
        for (int64_t i = 0; i < n; ++i) Linv[i * n + c] = col[i];
    }
    for (int64_t b = 0; b < n; ++b)
        for (int64_t a = b + 1; a < n; ++a) {
            T kinv = T(0);
            for (int64_t kk = 0; kk < n; ++kk) kinv += Linv[kk * n + a] * Linv[kk * n + b];
            G[a * n + b] = kinv;
        }
    dense_points_scatter(p, G, dp);
}

// ---- src/dense.jl:268-300: cotangent -alpha_a alpha_b, alpha = K^-1 y -------------------------
template <typename T>
void dense_inv_loss_grad_points(const Prob& p, const std::vector<T>& L, const T* y, T* dp,
                                double* loss) {
    const int64_t n = p.n0;
    std::vector<T> xi(n), alpha(n), G(n * n, T(0));
    trsv_lower(L.data(), n, y, xi.data());
    trsv_lower_t(L.data(), n, xi.data(), alpha.data());
    for (int64_t b = 0; b < n; ++b)
        for (int64_t a = b + 1; a < n; ++a) G[a * n + b] = -alpha[a] * alpha[b];
    dense_points_scatter(p, G, dp);
    double l = 0.0;
    for (int64_t i = 0; i < n; ++i) l += 0.5 * (double)xi[i] * (double)xi[i];
    if (loss) *loss = l;
}

// ---- src/grad.jl:228-236 --------------------------------------------------------------------
template <typename T>
int generate_logdet_grad_points(const Prob& p, T* dp, double* logdet) {
    double ld_ref = 0.0;
    refine_logdet_grad_points(p, dp, &ld_ref);
    std::vector<T> L;
    if (!dense_factor(p, L)) return 6;
    dense_logdet_grad_points(p, L, dp);
    double ld_dense = 0.0;
    for (int64_t i = 0; i < p.n0; ++i) ld_dense += std::log((double)L[i * p.n0 + i]);
    if (logdet) *logdet = ld_dense + ld_ref;
    return 0;
}

// ---- src/grad.jl:321-336: data in the original order ----------------------------------------
template <typename T>
int generate_inv_loss_grad_points(const Prob& p, const T* data, T* dp, double* loss) {
    const int64_t N = p.N;
    std::vector<T> d(N);
    for (int64_t i = 0; i < N; ++i) d[i] = p.indices ? data[p.indices[i]] : data[i];
    double l_ref = 0.0, l_dense = 0.0;
    refine_inv_loss_grad_points(p, d.data(), dp, &l_ref);
    std::vector<T> L;
    if (!dense_factor(p, L)) return 6;
    dense_inv_loss_grad_points(p, L, d.data(), dp, &l_dense);
    if (loss) *loss = l_ref + l_dense;
    return 0;
}

}  // namespace

// ================================= C ABI for the tests ========================================
extern "C" {

typedef Prob ggp_oracle_problem;

int oracle_refine_logdet_terms_f32(const ggp_oracle_problem* p, float* t) { refine_logdet_terms<float>(*p, t); return 0; }
int oracle_refine_logdet_terms_f64(const ggp_oracle_problem* p, double* t) { refine_logdet_terms<double>(*p, t); return 0; }
int oracle_refine_inv_f32(const ggp_oracle_problem* p, const float* v, float* xi) { refine_inv<float>(*p, v, xi); return 0; }
int oracle_refine_inv_f64(const ggp_oracle_problem* p, const double* v, double* xi) { refine_inv<double>(*p, v, xi); return 0; }
int oracle_refine_meanvec_std_f32(const ggp_oracle_problem* p, float* mv, float* sd) { refine_meanvec_std<float>(*p, mv, sd); return 0; }
int oracle_refine_meanvec_std_f64(const ggp_oracle_problem* p, double* mv, double* sd) { refine_meanvec_std<double>(*p, mv, sd); return 0; }
int oracle_refine_f32(const ggp_oracle_problem* p, float* v, const float* xr) { refine<float>(*p, v, xr); return 0; }
int oracle_refine_f64(const ggp_oracle_problem* p, double* v, const double* xr) { refine<double>(*p, v, xr); return 0; }
int oracle_generate_f32(const ggp_oracle_problem* p, const float* xi, float* out) { return generate<float>(*p, xi, out); }
int oracle_generate_f64(const ggp_oracle_problem* p, const double* xi, double* out) { return generate<double>(*p, xi, out); }
int oracle_generate_inv_f32(const ggp_oracle_problem* p, const float* v, float* xi) { return generate_inv<float>(*p, v, xi); }
int oracle_generate_inv_f64(const ggp_oracle_problem* p, const double* v, double* xi) { return generate_inv<double>(*p, v, xi); }
int oracle_generate_logdet_f32(const ggp_oracle_problem* p, double* o) { return generate_logdet<float>(*p, o); }
int oracle_generate_logdet_f64(const ggp_oracle_problem* p, double* o) { return generate_logdet<double>(*p, o); }
int oracle_refine_logdet_grad_vals_f32(const ggp_oracle_problem* p, float* dv, double* ld) { refine_logdet_grad_vals<float>(*p, dv, ld); return 0; }
int oracle_refine_logdet_grad_vals_f64(const ggp_oracle_problem* p, double* dv, double* ld) { refine_logdet_grad_vals<double>(*p, dv, ld); return 0; }
int oracle_generate_logdet_grad_vals_f32(const ggp_oracle_problem* p, float* dv, double* ld) { return generate_logdet_grad_vals<float>(*p, dv, ld); }
int oracle_generate_logdet_grad_vals_f64(const ggp_oracle_problem* p, double* dv, double* ld) { return generate_logdet_grad_vals<double>(*p, dv, ld); }
int oracle_refine_inv_loss_grad_vals_f32(const ggp_oracle_problem* p, const float* v, float* dv, double* l) { refine_inv_loss_grad_vals<float>(*p, v, dv, l); return 0; }
int oracle_refine_inv_loss_grad_vals_f64(const ggp_oracle_problem* p, const double* v, double* dv, double* l) { refine_inv_loss_grad_vals<double>(*p, v, dv, l); return 0; }
int oracle_generate_inv_loss_grad_vals_f32(const ggp_oracle_problem* p, const float* d, float* dv, double* l) { return generate_inv_loss_grad_vals<float>(*p, d, dv, l); }
int oracle_generate_inv_loss_grad_vals_f64(const ggp_oracle_problem* p, const double* d, double* dv, double* l) { return generate_inv_loss_grad_vals<double>(*p, d, dv, l); }
int oracle_generate_grad_xi_f32(const ggp_oracle_problem* p, const float* vb, float* xb) { return generate_grad_xi<float>(*p, vb, xb); }
int oracle_generate_grad_xi_f64(const ggp_oracle_problem* p, const double* vb, double* xb) { return generate_grad_xi<double>(*p, vb, xb); }
int oracle_generate_grad_vals_f32(const ggp_oracle_problem* p, const float* xi, const float* vb, float* dv) { return generate_grad_vals<float>(*p, xi, vb, dv); }
int oracle_generate_grad_vals_f64(const ggp_oracle_problem* p, const double* xi, const double* vb, double* dv) { return generate_grad_vals<double>(*p, xi, vb, dv); }

// Point-position gradients exist for the tabulated isotropic covariance only (the reference
// differentiates cov_lookup in r); an anisotropic problem returns 7.
int oracle_refine_logdet_grad_points_f32(const ggp_oracle_problem* p, float* dp, double* ld) { if (p->aniso) return 7; refine_logdet_grad_points<float>(*p, dp, ld); return 0; }
int oracle_refine_logdet_grad_points_f64(const ggp_oracle_problem* p, double* dp, double* ld) { if (p->aniso) return 7; refine_logdet_grad_points<double>(*p, dp, ld); return 0; }
int oracle_generate_logdet_grad_points_f32(const ggp_oracle_problem* p, float* dp, double* ld) { if (p->aniso) return 7; return generate_logdet_grad_points<float>(*p, dp, ld); }
int oracle_generate_logdet_grad_points_f64(const ggp_oracle_problem* p, double* dp, double* ld) { if (p->aniso) return 7; return generate_logdet_grad_points<double>(*p, dp, ld); }
int oracle_refine_inv_loss_grad_points_f32(const ggp_oracle_problem* p, const float* v, float* dp, double* l) { if (p->aniso) return 7; refine_inv_loss_grad_points<float>(*p, v, dp, l); return 0; }
int oracle_refine_inv_loss_grad_points_f64(const ggp_oracle_problem* p, const double* v, double* dp, double* l) { if (p->aniso) return 7; refine_inv_loss_grad_points<double>(*p, v, dp, l); return 0; }
int oracle_generate_inv_loss_grad_points_f32(const ggp_oracle_problem* p, const float* d, float* dp, double* l) { if (p->aniso) return 7; return generate_inv_loss_grad_points<float>(*p, d, dp, l); }
int oracle_generate_inv_loss_grad_points_f64(const ggp_oracle_problem* p, const double* d, double* dp, double* l) { if (p->aniso) return 7; return generate_inv_loss_grad_points<double>(*p, d, dp, l); }

// Primitive-level entry points for the unit tests (single point / single matrix).
double oracle_cov_lookup_f64(double r, const double* bins, const double* vals, int64_t n) { return cov_lookup<double>(r, bins, vals, n); }
float oracle_cov_lookup_f32(float r, const float* bins, const float* vals, int64_t n) { return cov_lookup<float>(r, bins, vals, n); }
void oracle_cov_lookup_weights_f64(double r, const double* bins, int64_t n, int64_t* lo, double* wlo, double* whi) { cov_lookup_weights<double>(r, bins, n, *lo, *wlo, *whi); }
void oracle_chol_lower_f64(double* A, int64_t n) { chol_lower<double>(A, n); }
void oracle_chol_lower_f32(float* A, int64_t n) { chol_lower<float>(A, n); }
void oracle_mean_vec_solve_f64(double* x, const double* L, int64_t K) { mean_vec_solve<double>(x, L, K); }
void oracle_chol_pullback_f64(double* Abar, double* Lbar, const double* L, int64_t n) { chol_pullback_impl<double, false>(Abar, Lbar, L, n); }
void oracle_chol_pullback_dyn_f64(double* Abar, double* Lbar, const double* L, int64_t n) { chol_pullback_impl<double, true>(Abar, Lbar, L, n); }
int oracle_dense_factor_f64(const ggp_oracle_problem* p, double* L) { std::vector<double> l; bool ok = dense_factor<double>(*p, l); std::memcpy(L, l.data(), l.size() * sizeof(double)); return ok ? 0 : 6; }
int oracle_dense_factor_f32(const ggp_oracle_problem* p, float* L) { std::vector<float> l; bool ok = dense_factor<float>(*p, l); std::memcpy(L, l.data(), l.size() * sizeof(float)); return ok ? 0 : 6; }
int oracle_max_threads(void) { return omp_get_max_threads(); }

}  // extern "C"
