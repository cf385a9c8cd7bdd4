/* graphgp_hip.h — C ABI of libgraphgp_hip, the MI355X (gfx950) implementation of GraphGP.jl's
 * fused per-point Vecchia refinement.
 *
 * Conventions (those of the reference's accelerator ABI, csrc/graphgp_capi.cu:70-119):
 *   - every function returns an int status, 0 = success; ggp_last_error() gives the message;
 *   - `stream` is a hipStream_t passed as void* (NULL = the default stream);
 *   - arrays passed to the ops are DEVICE pointers of the problem's element type (float for
 *     GGP_F32, double for GGP_F64) unless the name says _host;
 *   - indices into points are 0-based.
 * Status codes: 2 = k unsupported, 3 = D unsupported (as csrc/graphgp_capi.cu:53-68),
 *   4 = malformed graph (the invariants of check_graph, src/graph_build.jl:20-57),
 *   5 = HIP runtime error, 6 = dense first-layer covariance not positive definite even with
 *   1e-2 relative jitter (src/dense.jl:65-66), 7 = invalid argument, 8 = no covariance set.
 *
 * The problem handle stands for the reference's GraphGPProblem after to_backend
 * (src/types.jl:22-106): the handle owns device copies of the graph in the layout the kernels
 * want (neighbours as int32 structure-of-arrays, a reverse neighbour list, the level table) and
 * never retains caller buffers. One handle must not be used from two host threads at once;
 * different handles are independent.
 *
 * All ops take and return arrays in the ORIGINAL point order, as src/orchestrate.jl does
 * (xi[indices] gathered on input, out[indices] = values scattered on output); the refine_* ops
 * work in tree order, as src/api.jl does. Every op returns after its work on `stream` is done.
 */
#ifndef GRAPHGP_HIP_H
#define GRAPHGP_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ggp_graph ggp_graph;

enum { GGP_F32 = 0, GGP_F64 = 1 };

enum {
    GGP_OK = 0,
    GGP_ERR_K = 2,
    GGP_ERR_D = 3,
    GGP_ERR_GRAPH = 4,
    GGP_ERR_HIP = 5,
    GGP_ERR_NOT_PD = 6,
    GGP_ERR_ARG = 7,
    GGP_ERR_NO_COV = 8
};

/* Message for the last non-zero status returned on this host thread. */
const char* ggp_last_error(void);

/* Supported neighbour counts k and dimensions D: 1 <= k <= 31, D in {2, 3, 4}. k in {4, 8, 10,
 * 16} run on register-block kernels (a lane per point), every other k on group-per-point
 * kernels; the results are the same IEEE operations either way (csrc/graphgp_capi.cu:52-68
 * dispatches k to compiled bounds up to 64). Returns 0, GGP_ERR_K or GGP_ERR_D. */
int ggp_supported(int64_t k, int32_t D);

/* Problem construction = GraphGPProblem(coords, neighbors, offsets, n0, scale, bins, vals,
 * indices) followed by to_backend (src/types.jl:32-56, 99-106). Host inputs:
 *   coords_host    N*D uint32, point-major (the reference's (D,N) column-major lattice coords)
 *   neighbors_host M*k int64, point-major (the reference's (K,M) column-major), 0-based,
 *                  M = N - n0; every neighbour must lie in an earlier depth level
 *   offsets_host   n_offsets int64, 0-based exclusive level ends, offsets[0] = n0,
 *                  offsets[n_offsets-1] = N (the reference's `offsets`)
 *   indices_host   N int64 or NULL; indices[tree_pos] = original_pos (the reference's `indices`)
 *   scale          physical length of one lattice step (the reference's `scale`)
 * The graph is validated as check_graph does (status 4 on a violation). */
int ggp_graph_create(ggp_graph** out, const uint32_t* coords_host, const int64_t* neighbors_host,
                     const int64_t* offsets_host, int64_t n_offsets, const int64_t* indices_host,
                     int64_t n0, int64_t k, int64_t N, int32_t D, double scale, int32_t dtype);
int ggp_graph_destroy(ggp_graph* h);

/* Problem shape: N, n0, k, D, number of depth levels (excluding the dense level), dtype. */
int ggp_graph_shape(const ggp_graph* h, int64_t* N, int64_t* n0, int64_t* k, int32_t* D,
                    int64_t* n_levels, int32_t* dtype);

/* Isotropic covariance table (bins, vals): the reference's prob.bins / prob.vals
 * (src/types.jl:28-29; built by make_cov_bins / rbf_kernel / matern_kernel, src/extras.jl).
 * Host arrays of the problem's element type; bins strictly increasing with bins[0] >= 0.
 * Replacing the table is the analogue of _set_vals (src/chainrules.jl:18-21). */
int ggp_set_cov_iso(ggp_graph* h, const void* bins_host, const void* vals_host, int64_t nbins);

/* Anisotropic covariance K(d_spatial, d_z) (AnisoCov, src/types.jl:15-20; src/aniso.jl): a
 * bilinear table grid (n_s x n_z, row-major: grid[i*n_z + j] = K(spatial_bins[i], z_bins[j]))
 * over the spatial distance of the first D-1 coordinates and |dz| * scale / alpha of the last.
 * Host arrays of the problem's element type, axes strictly increasing. Replaces any isotropic
 * table. As in the reference, anisotropic problems are forward-only: generate, generate_inv,
 * generate_logdet, refine_* and generate_grad_xi (the transpose of the forward map) run; the
 * d/dvals ops return GGP_ERR_ARG. */
int ggp_set_cov_aniso(ggp_graph* h, const void* spatial_bins_host, int64_t n_s,
                      const void* z_bins_host, int64_t n_z, const void* grid_host, double alpha);

/* ---- forward ops -------------------------------------------------------------------------- */

/* generate (src/orchestrate.jl:19-42): out = G(xi), both length N, original order. */
int ggp_generate(ggp_graph* h, const void* xi, void* out, void* stream);

/* generate_inv (src/orchestrate.jl:53-81): xi = G^-1(values), both length N, original order. */
int ggp_generate_inv(ggp_graph* h, const void* values, void* xi, void* stream);

/* generate_logdet (src/orchestrate.jl:89-97): dense + refinement log-determinant. */
int ggp_generate_logdet(ggp_graph* h, double* logdet_host, void* stream);

/* refine_logdet_terms (src/api.jl:30-57): terms[m] = log std_m, length M, tree order.
 * refine_logdet (src/api.jl:24-27): the sum of those terms (accumulated in double). */
int ggp_refine_logdet_terms(ggp_graph* h, void* terms, void* stream);
int ggp_refine_logdet(ggp_graph* h, double* out_host, void* stream);

/* refine_inv (src/api.jl:66-103): xi_ref[m] for the M refined points from values_tree (N). */
int ggp_refine_inv(ggp_graph* h, const void* values_tree, void* xi_ref, void* stream);

/* refine! (src/api.jl:113-141): values_tree (N, first n0 preset) is completed in place from
 * xi_ref (M). */
int ggp_refine(ggp_graph* h, void* values_tree, const void* xi_ref, void* stream);

/* ---- adjoints ----------------------------------------------------------------------------- */

/* generate_grad_xi (src/grad.jl:392-506): xbar = G^T vbar, both length N, original order. */
int ggp_generate_grad_xi(ggp_graph* h, const void* vbar, void* xbar, void* stream);

/* generate_grad_vals (src/grad_generate_vals.jl:111-282): d_vals (nbins) = d<vbar, G(xi)>/dvals.
 * xi and vbar are length N, original order. */
int ggp_generate_grad_vals(ggp_graph* h, const void* xi, const void* vbar, void* d_vals,
                           void* stream);

/* refine_logdet_grad_vals (src/grad.jl:96-119): d_vals = d(refine_logdet)/dvals; the logdet
 * itself is written to *logdet_host when non-NULL (the fused form, src/grad.jl:680-715). */
int ggp_refine_logdet_grad_vals(ggp_graph* h, void* d_vals, double* logdet_host, void* stream);

/* generate_logdet_grad_vals (src/grad.jl:149-154) = generate_logdet_and_grad_vals
 * (src/grad.jl:680-715): dense + refinement. */
int ggp_generate_logdet_grad_vals(ggp_graph* h, void* d_vals, double* logdet_host, void* stream);

/* refine_inv_loss_grad_vals (src/grad.jl:626-671): loss = 0.5*||refine_inv(values_tree)||^2 and
 * its gradient w.r.t. vals. */
int ggp_refine_inv_loss_grad_vals(ggp_graph* h, const void* values_tree, void* d_vals,
                                  double* loss_host, void* stream);

/* generate_inv_loss_grad_vals (src/grad.jl:514-529): 0.5*||generate_inv(data)||^2 and its
 * gradient w.r.t. vals; data is length N, original order. */
int ggp_generate_inv_loss_grad_vals(ggp_graph* h, const void* data, void* d_vals,
                                    double* loss_host, void* stream);

/* ---- gradients w.r.t. the point positions x = scale * coords ------------------------------
 * d_points is N x D, tree order, point-major: the memory layout of the reference's (D, N)
 * matrix. Each off-diagonal covariance cotangent reaches the two points through k'(r) dr/dx
 * (the table's segment slope, 0 outside it); the lattice is straight-through. Isotropic table
 * only (an anisotropic table returns GGP_ERR_ARG). The scalar (logdet or loss) goes to
 * *_host when non-NULL. */

/* refine_logdet_grad_points (src/grad.jl:168-226). */
int ggp_refine_logdet_grad_points(ggp_graph* h, void* d_points, double* logdet_host,
                                  void* stream);

/* generate_logdet_grad_points (src/grad.jl:242-247; dense part src/dense.jl:188-222). */
int ggp_generate_logdet_grad_points(ggp_graph* h, void* d_points, double* logdet_host,
                                    void* stream);

/* refine_inv_loss_grad_points (src/grad.jl:259-319): values_tree is length N, tree order. */
int ggp_refine_inv_loss_grad_points(ggp_graph* h, const void* values_tree, void* d_points,
                                    double* loss_host, void* stream);

/* generate_inv_loss_grad_points (src/grad.jl:368-377; dense part src/dense.jl:271-300): data
 * is length N, original order. */
int ggp_generate_inv_loss_grad_points(ggp_graph* h, const void* data, void* d_points,
                                      double* loss_host, void* stream);

/* ---- stateless entry points with the reference's accelerator signatures --------------------
 * gpcuda_refine_logdet_f32 / gpcuda_refine_inv_f32 (csrc/graphgp_capi.cu:70-94, bound by
 * refine_logdet_custom / refine_inv_custom, ext/GraphGPCUDAExt.jl:38-63): the order-independent
 * per-point ops over all M = n_points - n0 refined points in one launch, on the caller's device
 * arrays, with no problem handle. The one change of signature: the reference passes float
 * positions (scale * coords, csrc/graphgp_capi.cu:10-13), which do not reproduce the lattice
 * lookup (src/linalg.jl:19-24); these take the integer lattice `coords` and `scale` instead.
 *   coords     device, n_points * ndim uint32, point-major, tree order (the reference's (D, N)
 *              column-major prob.coords)
 *   neighbors  device, (n_points - n0) * k int64, point-major, 0-based (prob.neighbors .- 1);
 *              each index must precede its point (an index that does not is read as the point
 *              itself, so no access leaves the arrays, and that point's result is meaningless)
 *   cov_bins / cov_vals  device, n_cov entries (prob.bins / prob.vals), bins strictly
 *              increasing with bins[0] = 0; not validated on the host
 *   out        device, 1 entry: sum over the refined points of log std (refine_logdet)
 *   values / xi  device, n_points / (n_points - n0) entries: refine_inv, tree order
 * Asynchronous on `stream` (a hipStream_t; NULL = default stream), as the reference's; the
 * scratch they need (the prepared table and partial sums, a few tens of KiB) is allocated and
 * released stream-ordered on that stream. Returns 0, 2 (k outside 1..31), 3 (ndim not 2, 3 or
 * 4), 7 (other argument) or 5 (HIP error). */
int gphip_refine_logdet_f32(const uint32_t* coords, float scale, const int64_t* neighbors,
                            const float* cov_bins, const float* cov_vals, float* out, int64_t n0,
                            int64_t k, int64_t n_points, int64_t n_cov, int64_t ndim,
                            void* stream);
int gphip_refine_inv_f32(const uint32_t* coords, float scale, const int64_t* neighbors,
                         const float* cov_bins, const float* cov_vals, const float* values,
                         float* xi, int64_t n0, int64_t k, int64_t n_points, int64_t n_cov,
                         int64_t ndim, void* stream);
/* No counterpart in the reference: gphip_refine_logdet_f32 for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Same arguments and result; the scratch is a fixed 64 KiB device array of the
 * library (one per device, held until the process ends) instead of a stream-ordered allocation,
 * and no allocating routine is called. Limit: n_cov <= 2048 (status 7 beyond). Every call on a
 * device shares that array, so calls that overlap on one device (different streams or host
 * threads) race and must be serialized by the caller. */
int gphip_refine_logdet_f32_noalloc(const uint32_t* coords, float scale,
                                    const int64_t* neighbors, const float* cov_bins,
                                    const float* cov_vals, float* out, int64_t n0, int64_t k,
                                    int64_t n_points, int64_t n_cov, int64_t ndim, void* stream);
/* The same in Float64 (no counterpart in the reference's ABI, which is Float32 only). */
int gphip_refine_logdet_f64(const uint32_t* coords, double scale, const int64_t* neighbors,
                            const double* cov_bins, const double* cov_vals, double* out,
                            int64_t n0, int64_t k, int64_t n_points, int64_t n_cov,
                            int64_t ndim, void* stream);
int gphip_refine_inv_f64(const uint32_t* coords, double scale, const int64_t* neighbors,
                         const double* cov_bins, const double* cov_vals, const double* values,
                         double* xi, int64_t n0, int64_t k, int64_t n_points, int64_t n_cov,
                         int64_t ndim, void* stream);

/* ---- graph build on the device ----------------------------------------------------------
 * build_graph (src/graph_build.jl:254-288) on the GPU; replaces gpcuda_build_graph_f32
 * (csrc/graphgp_capi.cu:100-117, driven by build_graph_cuda, ext/GraphGPCUDAExt.jl:66-105).
 * Unlike that build (float points, a differently tie-broken tree), this one follows the host
 * build_graph step for step in double, so it returns the same graph as ggp_build_graph.
 *   points        device, N*D doubles, point-major, original order
 *   coords        device, N*D uint32 lattice coordinates, tree order
 *   neighbors     device, (N-n0)*k int64, 0-based tree positions
 *   indices       device, N int64, indices[tree_pos] = original_pos
 *   offsets_host  host, room for offsets_cap level ends (N-n0+1 always suffices);
 *                 *n_offsets receives the count, *scale the lattice step
 * 1 <= k <= 32, k <= n0 < N < 2^31, D in 1..4. Synchronous on `stream`; scratch memory is
 * allocated and released inside the call. Returns 0, GGP_ERR_ARG, GGP_ERR_D or GGP_ERR_HIP. */
int ggp_build_graph_device(const double* points, int64_t N, int32_t D, int64_t n0, int64_t k,
                           int32_t lattice_bits, uint32_t* coords, int64_t* neighbors,
                           int64_t* indices, int64_t* offsets_host, int64_t offsets_cap,
                           int64_t* n_offsets, double* scale, void* stream);

/* ---- measurement ------------------------------------------------------------------------- */
/* No counterpart in the reference (its benchmarks time whole calls, bench/compare/run_julia.jl:50-58).
 * `enable` is a bit mask over "factor" (1), "pullback" (2), "sweep_fwd" (4), "sweep_rev" (8),
 * "dense" (16: assembly + Cholesky of the dense block), "op" (32, the whole op) and "potrf"
 * (64: the dense Cholesky launch alone); 0 turns timing off, 127 times everything. Each
 * enabled timer brackets its kernels with HIP events on the stream they run on (every event
 * pair adds a few microseconds to the op); ggp_kernel_timer_read returns the summed
 * milliseconds and the number of timed launches for one name. Enabling resets the sums. */
int ggp_kernel_timers(ggp_graph* h, int32_t enable);
int ggp_kernel_timer_read(const ggp_graph* h, const char* name, double* total_ms, int64_t* count);

/* No counterpart in the reference. Self-check of the f32 square roots: the one the per-point
 * kernels use for pair radii (a correctly rounded sqrt without range scaling, on 0 and
 * [1e-30, 2^64]) and the range-reduced one of the dense factor's pivots (every float; NaN
 * results compared as NaN). Compares them bit for bit with sqrtf on the current device over the
 * `count` float bit patterns starting at `first_bits` and stores the number of differences.
 * Synchronous. */
int ggp_selftest_sqrt_f32(uint32_t first_bits, uint32_t count, uint64_t* mismatches);

/* No counterpart in the reference. Self-check of the division the per-point Cholesky,
 * mean_vec and the dense tile solves use: t / d from one reciprocal per divisor with a one-fma
 * remainder correction, compared bit for bit with the IEEE division on the current device.
 * GGP_F32: every divisor bit pattern in [first, first + count), whose reciprocal (v_rcp_f32 and
 * one Newton step) is also compared with 1/d (on [2^-126, 2^126), zeros and infinities; NaN
 * for NaN); GGP_F64: `count` random divisors in [2^-60, 2^60) drawn from `seed`. Each divisor
 * gets per_divisor numerators (zero, then random ones over 2^-100 .. 2^100 in f32 or
 * 2^-900 .. 2^900 in f64). Stores the number of differences. Synchronous. */
int ggp_selftest_div(int32_t dtype, uint64_t first, uint64_t count, uint32_t per_divisor,
                     uint64_t seed, uint64_t* mismatches);

#ifdef __cplusplus
}
#endif

#endif /* GRAPHGP_HIP_H */
