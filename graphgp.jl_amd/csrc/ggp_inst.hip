// ggp_inst.hip — one (element type, k) instantiation of the per-point kernels; the build
// compiles this file once per pair with -DGGP_T=<float|double> -DGGP_K=<k>.
#include "ggp_point_kernels.h"

#if !defined(GGP_T) || !defined(GGP_K)
#error "compile with -DGGP_T=<float|double> -DGGP_K=<k>"
#endif

template struct ggp::PointK<GGP_T, GGP_K>;
