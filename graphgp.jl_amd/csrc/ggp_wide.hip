// ggp_wide.hip — launchers of the group-per-point kernels (any k <= 31), compiled once per
// (element type, dimension, part): -DGGP_T=<float|double> -DGGP_D=<2|3|4> -DGGP_PART=<0|1|2>
// (0: the factor pass; 1: the pullback with the table in LDS; 2: the pullback with the table in
// global memory), so the heavy instantiations build in parallel.
#include "ggp_wide.h"

#if !defined(GGP_T) || !defined(GGP_D)
#error "compile with -DGGP_T=<float|double> -DGGP_D=<2|3|4>"
#endif

namespace ggp {

static inline unsigned grid_wide(int64_t M, unsigned nblk) {
    const int64_t need = (M + kWidePts - 1) / kWidePts;
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>((int64_t)nblk, need));
}

#if GGP_PART == 0
template <typename T, int D>
void WideD<T, D>::factor(const Graph& g, const Table<T>& tb, int mode, T* mv, T* sd, T* terms,
                      double* partial, const T* values, T* xi_out, unsigned nblk,
                      hipStream_t st) {
    const bool aniso = tb.aniso.grid != nullptr;
    const size_t lds = aniso ? (size_t)tb.aniso.lds
                             : tb.global ? 0 : tab_bytes<T>(tb.P.nb, tb.P.ucells);
    const T scale = (T)g.scale;
    const int K = (int)g.K;
    // TERMS writes one partial per launched workgroup: keep the grid at nblk so the host's
    // reduction over nblk partials sees every slot written.
    const unsigned grid = (mode & F_TERMS) ? nblk : grid_wide(g.M, nblk);
    if (!aniso && tb.global) {  // one instantiation, the mode at run time
        hipLaunchKernelGGL((k_factor_w<T, D, -1, false, true>), dim3(grid), dim3(kWideBlock), 0,
                           st, g.coords, g.nbr, g.M, g.n0, K, scale, tb.tab, tb.acc, tb.params,
                           mv, sd, terms, partial, values, xi_out, tb.aniso, g.nbr64, mode);
        return;
    }
#define GGP_FACTOR_W(MODEV)                                                                    \
    do {                                                                                       \
        if (aniso)                                                                             \
            hipLaunchKernelGGL((k_factor_w<T, D, MODEV, true, false>), dim3(grid),              \
                               dim3(kWideBlock), lds, st, g.coords, g.nbr, g.M, g.n0, K, scale, \
                               tb.tab, tb.acc, tb.params, mv, sd, terms, partial, values,       \
                               xi_out, tb.aniso, g.nbr64, 0);                                   \
        else                                                                                   \
            hipLaunchKernelGGL((k_factor_w<T, D, MODEV, false, false>), dim3(grid),             \
                               dim3(kWideBlock), lds, st, g.coords, g.nbr, g.M, g.n0, K, scale, \
                               tb.tab, tb.acc, tb.params, mv, sd, terms, partial, values,       \
                               xi_out, tb.aniso, g.nbr64, 0);                                   \
    } while (0)
    switch (mode) {
        case F_MV: GGP_FACTOR_W(F_MV); break;
        case F_TERMS: GGP_FACTOR_W(F_TERMS); break;
        case F_INV: GGP_FACTOR_W(F_INV); break;
        default: break;
    }
#undef GGP_FACTOR_W
}
template void WideD<GGP_T, GGP_D>::factor(const Graph&, const Table<GGP_T>&, int, GGP_T*, GGP_T*,
                                          GGP_T*, double*, const GGP_T*, GGP_T*, unsigned,
                                          hipStream_t);

#elif GGP_PART == 1
template <typename T, int D>
void WideD<T, D>::pullback(const Graph& g, const Table<T>& tb, int mode, const T* v, const T* xi,
                        const T* vb, double* hist_partial, double* scalar_partial,
                        unsigned nblk, hipStream_t st) {
    if (tb.global) {
        WideG<T, D>::pullback(g, tb, mode, v, xi, vb, hist_partial, scalar_partial, nblk, st);
        return;
    }
    const size_t lds = tab_bytes<T>(tb.P.nb, tb.P.ucells) +
                       ((mode & P_PTS) ? 0 : (size_t)tb.P.nb * sizeof(double));
    const T scale = (T)g.scale;
    const int K = (int)g.K;
    // every one of the nblk histogram rows is written, so the grid stays at nblk
#define GGP_PULL_W(MODEV)                                                                      \
    hipLaunchKernelGGL((k_pullback_w<T, D, MODEV, false>), dim3(nblk), dim3(kWideBlock), lds,   \
                       st, g.coords, g.nbr, g.M, g.n0, K, scale, tb.tab, tb.acc, tb.params, v,  \
                       xi, vb, hist_partial, scalar_partial, 0)
    switch (mode) {
        case P_LOGDET: GGP_PULL_W(P_LOGDET); break;
        case P_INVLOSS: GGP_PULL_W(P_INVLOSS); break;
        case P_GENVALS: GGP_PULL_W(P_GENVALS); break;
        case P_LOGDET | P_PTS: GGP_PULL_W(P_LOGDET | P_PTS); break;
        case P_INVLOSS | P_PTS: GGP_PULL_W(P_INVLOSS | P_PTS); break;
        default: break;
    }
#undef GGP_PULL_W
}
template void WideD<GGP_T, GGP_D>::pullback(const Graph&, const Table<GGP_T>&, int,
                                            const GGP_T*, const GGP_T*, const GGP_T*, double*,
                                            double*, unsigned, hipStream_t);

#elif GGP_PART == 2
// The table in global memory: one instantiation with the mode at run time; the histogram rows
// accumulate with atomics, so they start at zero.
template <typename T, int D>
void WideG<T, D>::pullback(const Graph& g, const Table<T>& tb, int mode, const T* v, const T* xi,
                           const T* vb, double* hist_partial, double* scalar_partial,
                           unsigned nblk, hipStream_t st) {
    if (!(mode & P_PTS)) launch_fill<double>(hist_partial, 0.0, (int64_t)nblk * tb.P.nb, st);
    hipLaunchKernelGGL((k_pullback_w<T, D, -1, true>), dim3(nblk), dim3(kWideBlock), 0, st,
                       g.coords, g.nbr, g.M, g.n0, (int)g.K, (T)g.scale, tb.tab, tb.acc,
                       tb.params, v, xi, vb, hist_partial, scalar_partial, mode);
}
template struct WideG<GGP_T, GGP_D>;
#else
#error "compile with -DGGP_PART=<0|1|2>"
#endif

}  // namespace ggp
