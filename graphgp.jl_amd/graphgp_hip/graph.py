"""build_graph on the host (src/graph_build.jl:254-288) through libggp_graph.so, and the graph
interchange format.

The interchange format is the reference's own .npz schema (test/loadref.jl:17-26,
bench/compare/dump_graph.py:60-70): coords (N, D) uint32 in tree order, neighbors (M, K)
0-based, offsets (0-based exclusive level ends, offsets[0] = n0), n0, scale, and the covariance
table as cov_bins32/cov_vals32 or cov_bins64/cov_vals64; this package adds indices (tree
position -> original position) when the problem has a permutation, and aniso_* keys for an
anisotropic covariance. A file written by save_graph loads with the reference's load_problem,
and the reference's fixtures load with load_graph. build_graph(..., cache=path) uses such a file
as a build cache (the reference's save_graph is Julia serialization only,
ext/GraphGPMPIExt.jl:176-190).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import _native as nat
from .problem import AnisoCov, GraphGPProblem


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


def build_graph_device_arrays(points, n0, k, lattice_bits=21, as_numpy=True):
    """The graph built on the GPU (ggp_build_graph_device; the role of build_graph_cuda,
    ext/GraphGPCUDAExt.jl:66-105). Same result as build_graph_arrays. points: (N, D) numpy or a
    torch tensor on the GPU. Returns (coords, neighbors, offsets, n0, scale, indices); the
    arrays stay torch GPU tensors when as_numpy is False (offsets are always numpy)."""
    import torch
    if isinstance(points, torch.Tensor):
        pts = points.to(device="cuda", dtype=torch.float64).contiguous()
    else:
        pts = torch.from_numpy(np.ascontiguousarray(points, dtype=np.float64)).to("cuda")
    N, D = pts.shape
    M = N - int(n0)
    coords = torch.empty((N, D), dtype=torch.int32, device="cuda")  # uint32 bits
    nbr = torch.empty((max(M, 1), int(k)), dtype=torch.int64, device="cuda")
    idx = torch.empty(N, dtype=torch.int64, device="cuda")
    offs = np.zeros(max(M, 0) + 1, np.int64)
    n_off, scale = C.c_int64(), C.c_double()
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    nat.call("ggp_build_graph_device", C.c_void_p(pts.data_ptr()), N, D, int(n0), int(k),
             int(lattice_bits), C.c_void_p(coords.data_ptr()), C.c_void_p(nbr.data_ptr()),
             C.c_void_p(idx.data_ptr()), offs.ctypes.data, len(offs), C.byref(n_off),
             C.byref(scale), stream)
    offs = offs[: n_off.value].copy()
    nbr = nbr[:M]
    if as_numpy:
        return (coords.cpu().numpy().view(np.uint32), nbr.cpu().numpy(), offs, int(n0),
                scale.value, idx.cpu().numpy())
    return coords, nbr, offs, int(n0), scale.value, idx


def build_graph(points, n0, k, bins, vals, lattice_bits=21, nthreads=0,
                cache=None, backend="cpu") -> GraphGPProblem:
    """GraphGPProblem built from float points (src/graph_build.jl:254-288).

    backend: "cpu" (the host builder) or "hip" (the same graph built on the GPU).
    cache: path of an interchange .npz. If it exists and holds a graph of the same N, D, n0 and
    k, that graph is used (with the given bins/vals); otherwise the graph is built and saved
    there."""
    pts = np.asarray(points)
    if cache is not None and os.path.exists(cache):
        with np.load(cache, allow_pickle=False) as z:
            if (z["coords"].shape == pts.shape and int(z["n0"]) == int(n0)
                    and z["neighbors"].shape[1:] == (int(k),)):
                idx = z["indices"] if "indices" in z.files else None
                return GraphGPProblem(z["coords"], z["neighbors"], z["offsets"], int(z["n0"]),
                                      float(z["scale"]), bins, vals, indices=idx)
    if backend in ("hip", "gpu", "cuda"):
        coords, nbr, offs, nn0, scale, idx = build_graph_device_arrays(pts, n0, k, lattice_bits)
    elif backend == "cpu":
        coords, nbr, offs, nn0, scale, idx = build_graph_arrays(pts, n0, k, lattice_bits,
                                                                nthreads)
    else:
        raise ValueError(f"unknown backend {backend!r}")
    prob = GraphGPProblem(coords, nbr, offs, nn0, scale, bins, vals, indices=idx)
    if cache is not None:
        save_graph(prob, cache)
    return prob


def save_graph(prob: GraphGPProblem, path) -> None:
    """Write prob in the interchange schema (uncompressed .npz: loads at memory speed)."""
    s = "64" if prob.dtype == np.float64 else "32"
    arrays = dict(coords=prob.coords, neighbors=prob.neighbors, offsets=prob.offsets,
                  n0=np.int64(prob.n0), scale=np.float64(prob.scale))
    if prob.cov is None:
        arrays["cov_bins" + s] = prob.bins
        arrays["cov_vals" + s] = prob.vals
    else:
        arrays.update(aniso_spatial_bins=prob.cov.spatial_bins, aniso_z_bins=prob.cov.z_bins,
                      aniso_grid=prob.cov.grid, aniso_alpha=np.float64(prob.cov.alpha))
    if prob.indices is not None:
        arrays["indices"] = prob.indices
    tmp = str(path) + ".tmp.npz"
    np.savez(tmp, **arrays)
    os.replace(tmp, path)


def load_graph(path, dtype=None) -> GraphGPProblem:
    """Read a graph in the interchange schema (the reference's fixtures included). dtype picks
    the covariance table when both precisions are stored (default: Float64 if present)."""
    with np.load(path, allow_pickle=False) as z:
        files = set(z.files)
        idx = z["indices"] if "indices" in files else None
        common = (z["coords"], z["neighbors"], z["offsets"], int(z["n0"]), float(z["scale"]))
        if "aniso_grid" in files:
            dt = np.dtype(dtype or z["aniso_grid"].dtype)
            cov = AnisoCov(z["aniso_spatial_bins"].astype(dt), z["aniso_z_bins"].astype(dt),
                           z["aniso_grid"].astype(dt), float(z["aniso_alpha"]))
            return GraphGPProblem(*common, indices=idx, cov=cov)
        if dtype is None:
            s = "64" if "cov_bins64" in files else "32"
        else:
            s = "64" if np.dtype(dtype) == np.float64 else "32"
            if "cov_bins" + s not in files:  # convert the stored precision
                other = "32" if s == "64" else "64"
                return GraphGPProblem(*common, z["cov_bins" + other].astype(dtype),
                                      z["cov_vals" + other].astype(dtype), indices=idx)
        return GraphGPProblem(*common, z["cov_bins" + s], z["cov_vals" + s], indices=idx)
