// ggp_wide.hip — launchers of the wavefront-per-point kernels (any k <= 31), compiled once per
// (element type, dimension): -DGGP_T=<float|double> -DGGP_D=<2|3|4>.
#include "ggp_wide.h"

#if !defined(GGP_T) || !defined(GGP_D)
#error "compile with -DGGP_T=<float|double> -DGGP_D=<2|3|4>"
#endif

namespace ggp {

static inline unsigned grid_wide(int64_t M, unsigned nblk) {
    const int64_t need = (M + kWideWaves - 1) / kWideWaves;
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>((int64_t)nblk, need));
}

template <typename T, int D>
void WideD<T, D>::factor(const Graph& g, const Table<T>& tb, int mode, T* mv, T* sd, T* terms,
                      double* partial, const T* values, T* xi_out, unsigned nblk,
                      hipStream_t st) {
    const bool aniso = tb.aniso.grid != nullptr;
    const size_t lds = aniso ? 0 : tab_bytes<T>(tb.P.nb, tb.P.ucells);
    const T scale = (T)g.scale;
    const int K = (int)g.K;
    // TERMS writes one partial per launched workgroup: keep the grid at nblk so the host's
    // reduction over nblk partials sees every slot written.
    const unsigned grid = (mode & F_TERMS) ? nblk : grid_wide(g.M, nblk);
#define GGP_FACTOR_W(DD, MODEV)                                                                \
    do {                                                                                       \
        if (aniso)                                                                             \
            hipLaunchKernelGGL((k_factor_w<T, DD, MODEV, true>), dim3(grid), dim3(kWideBlock),  \
                               0, st, g.coords, g.nbr, g.M, g.n0, K, scale, tb.tab, tb.acc,     \
                               tb.params, mv, sd, terms, partial, values, xi_out, tb.aniso,     \
                               g.nbr64);                                                        \
        else                                                                                   \
            hipLaunchKernelGGL((k_factor_w<T, DD, MODEV, false>), dim3(grid), dim3(kWideBlock), \
                               lds, st, g.coords, g.nbr, g.M, g.n0, K, scale, tb.tab, tb.acc,   \
                               tb.params, mv, sd, terms, partial, values, xi_out, tb.aniso,     \
                               g.nbr64);                                                        \
    } while (0)
#define GGP_FACTOR_W_D(DD)                                                                     \
    switch (mode) {                                                                            \
        case F_MV: GGP_FACTOR_W(DD, F_MV); break;                                              \
        case F_TERMS: GGP_FACTOR_W(DD, F_TERMS); break;                                        \
        case F_INV: GGP_FACTOR_W(DD, F_INV); break;                                            \
        default: break;                                                                        \
    }
    GGP_FACTOR_W_D(D);
#undef GGP_FACTOR_W_D
#undef GGP_FACTOR_W
}

template <typename T, int D>
void WideD<T, D>::pullback(const Graph& g, const Table<T>& tb, int mode, const T* v, const T* xi,
                        const T* vb, double* hist_partial, double* scalar_partial,
                        unsigned nblk, hipStream_t st) {
    const size_t lds = tab_bytes<T>(tb.P.nb, tb.P.ucells) +
                       ((mode & P_PTS) ? 0 : (size_t)tb.P.nb * sizeof(double));
    const T scale = (T)g.scale;
    const int K = (int)g.K;
    // every one of the nblk histogram rows is written, so the grid stays at nblk
#define GGP_PULL_W(DD, MODEV)                                                                  \
    hipLaunchKernelGGL((k_pullback_w<T, DD, MODEV>), dim3(nblk), dim3(kWideBlock), lds, st,     \
                       g.coords, g.nbr, g.M, g.n0, K, scale, tb.tab, tb.acc, tb.params, v, xi,  \
                       vb, hist_partial, scalar_partial)
#define GGP_PULL_W_D(DD)                                                                       \
    switch (mode) {                                                                            \
        case P_LOGDET: GGP_PULL_W(DD, P_LOGDET); break;                                        \
        case P_INVLOSS: GGP_PULL_W(DD, P_INVLOSS); break;                                      \
        case P_GENVALS: GGP_PULL_W(DD, P_GENVALS); break;                                      \
        case P_LOGDET | P_PTS: GGP_PULL_W(DD, P_LOGDET | P_PTS); break;                        \
        case P_INVLOSS | P_PTS: GGP_PULL_W(DD, P_INVLOSS | P_PTS); break;                      \
        default: break;                                                                        \
    }
    GGP_PULL_W_D(D);
#undef GGP_PULL_W_D
#undef GGP_PULL_W
}

template struct WideD<GGP_T, GGP_D>;

}  // namespace ggp
