"""build_graph on the host (src/graph_build.jl:254-288) through libggp_graph.so."""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _native as nat
from .problem import GraphGPProblem


def build_graph_arrays(points, n0, k, lattice_bits=21, nthreads=0):
    """Returns (coords (N,D) uint32, neighbors (M,K) int64, offsets, n0, scale, indices)."""
    pts = np.ascontiguousarray(points, dtype=np.float64)
    N, D = pts.shape
    lib = nat.graphlib()
    h = C.c_void_p()
    rc = lib.ggp_build_graph(pts.ctypes.data, N, D, int(n0), int(k), int(lattice_bits),
                             int(nthreads), C.byref(h))
    if rc != 0:
        raise ValueError(f"ggp_build_graph returned {rc}: need k <= n0 < N and 1 <= bits <= 30")
    try:
        n, nn0, kk, dd, no = C.c_int64(), C.c_int64(), C.c_int64(), C.c_int32(), C.c_int64()
        lib.ggp_built_graph_shape(h, C.byref(n), C.byref(nn0), C.byref(kk), C.byref(dd), C.byref(no))
        coords = np.zeros((N, D), np.uint32)
        nbr = np.zeros((N - nn0.value, k), np.int64)
        offs = np.zeros(no.value, np.int64)
        idx = np.zeros(N, np.int64)
        scale = C.c_double()
        lib.ggp_built_graph_copy(h, coords.ctypes.data, nbr.ctypes.data, offs.ctypes.data,
                                 idx.ctypes.data, C.byref(scale))
    finally:
        lib.ggp_built_graph_free(h)
    return coords, nbr, offs, nn0.value, scale.value, idx


def build_graph(points, n0, k, bins, vals, lattice_bits=21, nthreads=0) -> GraphGPProblem:
    """GraphGPProblem built from float points (src/graph_build.jl:254-288)."""
    coords, nbr, offs, nn0, scale, idx = build_graph_arrays(points, n0, k, lattice_bits, nthreads)
    return GraphGPProblem(coords, nbr, offs, nn0, scale, bins, vals, indices=idx)
