/* graphgp_graph.h — host-side construction of the refinement graph (libggp_graph.so).
 *
 * The reference builds the graph on the CPU with build_graph (src/graph_build.jl:254-288):
 * the heap-order k-d tree of src/tree_special.jl, the stackless preceding k-nearest-neighbour
 * query, depth relaxation, reordering by depth and 21-bit lattice quantization. This library
 * is the same pipeline in C++ (OpenMP); its output feeds ggp_graph_create.
 */
#ifndef GRAPHGP_GRAPH_H
#define GRAPHGP_GRAPH_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Opaque result of a build; free with ggp_built_graph_free. */
typedef struct ggp_built_graph ggp_built_graph;

/* build_graph(points, n0, k; lattice_bits) (src/graph_build.jl:254-288).
 *   points    N*D doubles, point-major (row i = point i), original order
 *   n0, k     initial dense-block size and neighbour count (k <= n0 < N)
 *   nthreads  OpenMP threads (0 = default)
 * Returns 0 on success, 7 on invalid arguments. */
int ggp_build_graph(const double* points, int64_t N, int32_t D, int64_t n0, int64_t k,
                    int32_t lattice_bits, int32_t nthreads, ggp_built_graph** out);

/* Sizes of a built graph: N, n0 (number of depth-0 points), k, D, number of offsets. */
int ggp_built_graph_shape(const ggp_built_graph* g, int64_t* N, int64_t* n0, int64_t* k,
                          int32_t* D, int64_t* n_offsets);

/* Copies the build into caller buffers (any may be NULL):
 *   coords     N*D uint32 lattice coords, tree order, point-major
 *   neighbors  (N-n0)*k int64, 0-based, point-major
 *   offsets    n_offsets int64, 0-based exclusive level ends, offsets[0] = n0
 *   indices    N int64, indices[tree_pos] = original_pos
 *   scale      lattice step (physical units) */
int ggp_built_graph_copy(const ggp_built_graph* g, uint32_t* coords, int64_t* neighbors,
                         int64_t* offsets, int64_t* indices, double* scale);

void ggp_built_graph_free(ggp_built_graph* g);

#ifdef __cplusplus
}
#endif

#endif /* GRAPHGP_GRAPH_H */
