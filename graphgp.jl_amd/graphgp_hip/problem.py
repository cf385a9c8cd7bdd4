"""GraphGPProblem and the refinement ops, mirroring GraphGP.jl's public API on the HIP library.

Reference interface (file:line in the reference):
  GraphGPProblem / to_backend ....... src/types.jl:22-106
  generate / generate_inv / _logdet .. src/orchestrate.jl:19-97
  refine_logdet(_terms) / refine_inv / refine! ... src/api.jl:24-169
  generate_grad_xi .................. src/grad.jl:392-506
  generate_grad_vals ................ src/grad_generate_vals.jl:111-282
  refine_logdet_grad_vals ........... src/grad.jl:96-119
  generate_logdet_grad_vals ......... src/grad.jl:149-154 (+ the fused form :680-715)
  refine/generate_inv_loss_grad_vals  src/grad.jl:514-671
  refine/generate_logdet_grad_points  src/grad.jl:168-247 (dense part src/dense.jl:188-222)
  refine/generate_inv_loss_grad_points src/grad.jl:259-377 (dense part src/dense.jl:271-300)
  check_graph ....................... src/graph_build.jl:20-57

Conventions are those of the JAX fixtures the reference's tests read (test/loadref.jl): numpy
arrays, 0-based indices, coords (N, D) uint32 in tree order (memory layout of the reference's
(D, N) column-major), neighbors (M, K), offsets 0-based exclusive level ends with
offsets[0] = n0, indices[tree_pos] = original_pos.

A host GraphGPProblem only holds arrays; `to_backend(prob)` creates the device problem
(HipProblem) that the ops run on. Every op needs a HipProblem: there is no CPU path. Op inputs
may be torch tensors on the GPU (used in place, results returned as tensors on the GPU) or
numpy arrays (copied to the GPU; results returned as numpy).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _native as nat


class AnisoCov:
    """Anisotropic covariance K(d_spatial, d_z) on a bilinear table (src/types.jl:15-20):
    spatial_bins (ns,), z_bins (nz,), grid (ns, nz), alpha."""

    def __init__(self, spatial_bins, z_bins, grid, alpha):
        self.spatial_bins = np.asarray(spatial_bins)
        self.z_bins = np.asarray(z_bins)
        self.grid = np.asarray(grid)
        self.alpha = float(alpha)
        if self.grid.shape != (len(self.spatial_bins), len(self.z_bins)):
            raise ValueError("grid must be (length(spatial_bins), length(z_bins))")


def build_anisotropic_covariance(spatial_bins, z_bins, grid, alpha, jitter=0.0, dtype=None):
    """AnisoCov with grid[0, 0] inflated by (1 + jitter) (src/aniso.jl:22-37)."""
    dt = np.dtype(dtype or np.asarray(grid).dtype)
    g = np.array(grid, dtype=dt)
    g[0, 0] = g[0, 0] * (dt.type(1) + dt.type(jitter))
    return AnisoCov(np.asarray(spatial_bins, dtype=dt), np.asarray(z_bins, dtype=dt), g,
                    float(alpha))


class GraphGPProblem:
    """Host container: graph + discretized covariance (src/types.jl:22-58). With `cov` set (an
    AnisoCov) the anisotropic covariance replaces (bins, vals), as in the reference."""

    def __init__(self, coords, neighbors, offsets, n0, scale, bins=None, vals=None, indices=None,
                 cov=None):
        if cov is not None and vals is None:
            bins, vals = cov.spatial_bins, cov.z_bins   # placeholders, as src/types.jl:75-80
        self.cov = cov
        self.coords = np.ascontiguousarray(coords, dtype=np.uint32)
        self.neighbors = np.ascontiguousarray(neighbors, dtype=np.int64)
        self.offsets = np.ascontiguousarray(offsets, dtype=np.int64)
        self.n0 = int(n0)
        vals = np.asarray(vals)
        self.dtype = np.dtype(np.float32 if vals.dtype == np.float32 else np.float64)
        self.bins = np.ascontiguousarray(bins, dtype=self.dtype)
        self.vals = np.ascontiguousarray(vals, dtype=self.dtype)
        self.scale = float(self.dtype.type(scale))
        self.indices = None if indices is None else np.ascontiguousarray(indices, dtype=np.int64)
        if self.coords.ndim != 2:
            raise ValueError("coords must be (N, D)")
        if self.neighbors.ndim != 2 or self.neighbors.shape[0] != self.N - self.n0:
            raise ValueError("neighbors must be (N - n0, K)")

    N = property(lambda self: self.coords.shape[0])
    D = property(lambda self: self.coords.shape[1])
    K = property(lambda self: self.neighbors.shape[1])
    M = property(lambda self: self.neighbors.shape[0])
    nbins = property(lambda self: len(self.bins))


# npoints / nneighbors / nrefined / ndims_space / nbins (src/types.jl:83-87)
def npoints(p):
    return p.N


def nneighbors(p):
    return p.K


def nrefined(p):
    return p.M


def ndims_space(p):
    return p.D


def nbins(p):
    return p.nbins


def check_graph(prob: GraphGPProblem) -> None:
    """Raise ValueError on the first violated invariant (src/graph_build.jl:20-57)."""
    N, M, n0, offs = prob.N, prob.M, prob.n0, prob.offsets
    if len(offs) == 0:
        raise ValueError("offsets is empty")
    if offs[0] != n0:
        raise ValueError(f"offsets[0] ({offs[0]}) must equal n0 ({n0})")
    if n0 != N - M:
        raise ValueError(f"n0 ({n0}) must equal npoints - nrefined ({N - M})")
    if np.any(np.diff(offs) < 0):
        raise ValueError("offsets must be non-decreasing")
    if offs[-1] > N:
        raise ValueError(f"offsets[end] ({offs[-1]}) must be <= npoints ({N})")
    if M == 0:
        return
    mx = prob.neighbors.max(axis=1)
    p = n0 + np.arange(M)
    bad = np.nonzero(mx >= p)[0]
    if len(bad):
        raise ValueError(f"point at position {p[bad[0]]} has neighbor {mx[bad[0]]} that does not "
                         "precede it (not topological)")
    b = np.searchsorted(offs, p, side="right")
    prev_end = np.where(b >= 1, offs[np.clip(b - 1, 0, len(offs) - 1)], 0)
    inlev = b < len(offs)
    bad = np.nonzero(inlev & (mx >= prev_end))[0]
    if len(bad):
        raise ValueError(f"point at position {p[bad[0]]} has a neighbor ({mx[bad[0]]}) in its own "
                         "batch; neighbors must be in earlier batches")


# ---------------------------------------------------------------------------------------------
def _torch():
    import torch
    return torch


class HipProblem:
    """A GraphGPProblem moved to the GPU: owns a ggp_graph handle (include/graphgp_hip.h)."""

    def __init__(self, prob: GraphGPProblem):
        self.host = prob
        self.N, self.n0, self.K, self.D, self.M = prob.N, prob.n0, prob.K, prob.D, prob.M
        self.dtype = prob.dtype
        self._h = C.c_void_p()
        self.table_version = 0  # bumped by every set_vals / set_aniso
        self._table = None
        idx = prob.indices
        nat.call("ggp_graph_create", C.byref(self._h), prob.coords.ctypes.data,
                 prob.neighbors.ctypes.data if prob.M else None, prob.offsets.ctypes.data,
                 len(prob.offsets), None if idx is None else idx.ctypes.data, prob.n0, prob.K,
                 prob.N, prob.D, prob.scale,
                 nat.GGP_F32 if self.dtype == np.float32 else nat.GGP_F64)
        if prob.cov is not None:
            self.set_aniso(prob.cov)
        else:
            self.set_vals(prob.vals, prob.bins)

    def set_aniso(self, cov):
        """Use the anisotropic covariance (forward-only, as in the reference)."""
        sb = np.ascontiguousarray(cov.spatial_bins, dtype=self.dtype)
        zb = np.ascontiguousarray(cov.z_bins, dtype=self.dtype)
        g = np.ascontiguousarray(cov.grid, dtype=self.dtype)
        self._aniso_arrays = (sb, zb, g)
        self.bins = self.vals = None
        nat.call("ggp_set_cov_aniso", self._h, sb.ctypes.data, len(sb), zb.ctypes.data, len(zb),
                 g.ctypes.data, float(cov.alpha))
        self.table_version += 1
        self._table = ("aniso", cov)
        return self

    def set_vals(self, vals, bins=None):
        """Replace the covariance table (the analogue of _set_vals, src/chainrules.jl:18-21)."""
        bins = self.host.bins if bins is None else np.ascontiguousarray(bins, dtype=self.dtype)
        vals = _to_host(vals, self.dtype).copy()
        self.bins, self.vals = bins, vals
        nat.call("ggp_set_cov_iso", self._h, bins.ctypes.data, vals.ctypes.data, len(bins))
        self.table_version += 1
        self._table = ("iso", bins, vals)
        return self

    def table_snapshot(self):
        """The covariance table in use now, for use_table(): a pullback closes over the problem
        its forward ran on (src/chainrules.jl:32-37), whatever tables are set in between."""
        return (self.table_version, self._table)

    def use_table(self, snap):
        """Put back the table of table_snapshot() if another one has been set since."""
        version, table = snap
        if version != self.table_version:
            if table[0] == "aniso":
                self.set_aniso(table[1])
            else:
                self.set_vals(table[2], table[1])
        return self

    @property
    def handle(self):
        return self._h

    @property
    def n_levels(self):
        return len(self.host.offsets) - 1

    def close(self):
        if self._h:
            nat.hip().ggp_graph_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def to_backend(prob: GraphGPProblem, backend: str = "hip") -> HipProblem:
    """Move a host problem to the GPU (src/types.jl:99-106)."""
    if backend not in ("hip", "gpu", "cuda"):
        raise ValueError("the only backend of this library is the HIP GPU backend")
    return HipProblem(prob)


def _to_host(x, dtype):
    if hasattr(x, "detach"):
        x = x.detach().cpu().numpy()
    return np.ascontiguousarray(x, dtype=dtype)


def _nb(prob):
    """Length of the d/dvals output. An anisotropic problem has no table to differentiate; the
    library rejects its d/dvals calls, so a one-element buffer stands in for the output."""
    return 1 if prob.bins is None else len(prob.bins)


def _require(prob):
    if not isinstance(prob, HipProblem):
        raise TypeError("ops run on the GPU problem: call to_backend(prob) first "
                        "(the reference's CPU path is not part of this library)")


def _dev(x, n, dtype):
    """(device tensor, input_was_numpy)."""
    torch = _torch()
    tdt = torch.float32 if dtype == np.float32 else torch.float64
    if isinstance(x, torch.Tensor):
        if not x.is_cuda:
            raise ValueError("torch inputs must live on the GPU")
        if x.dtype != tdt or not x.is_contiguous():
            x = x.to(dtype=tdt).contiguous()
        if x.numel() != n:
            raise ValueError(f"expected {n} elements, got {x.numel()}")
        return x, False
    a = np.ascontiguousarray(x, dtype=dtype).reshape(-1)
    if a.size != n:
        raise ValueError(f"expected {n} elements, got {a.size}")
    return torch.from_numpy(a).to("cuda"), True


def _empty(n, dtype):
    torch = _torch()
    return torch.empty(max(n, 1), dtype=torch.float32 if dtype == np.float32 else torch.float64,
                       device="cuda")


def _stream():
    torch = _torch()
    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)  # ~0.1 us against ~3 us
    if raw is not None:
        return C.c_void_p(raw(torch.cuda.current_device()))
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _out(t, n, as_numpy):
    if t.numel() != n:
        t = t[:n]
    return t.cpu().numpy() if as_numpy else t


def _ptr(t):
    return C.c_void_p(t.data_ptr())


# ---- forward ops -------------------------------------------------------------------------------
def generate(prob, xi):
    """Field in original order from unit-normal xi in original order (src/orchestrate.jl:19-42)."""
    _require(prob)
    x, np_in = _dev(xi, prob.N, prob.dtype)
    out = _empty(prob.N, prob.dtype)
    nat.call("ggp_generate", prob.handle, _ptr(x), _ptr(out), _stream())
    return _out(out, prob.N, np_in)


def generate_inv(prob, values):
    """xi in original order from a field in original order (src/orchestrate.jl:53-81)."""
    _require(prob)
    v, np_in = _dev(values, prob.N, prob.dtype)
    out = _empty(prob.N, prob.dtype)
    nat.call("ggp_generate_inv", prob.handle, _ptr(v), _ptr(out), _stream())
    return _out(out, prob.N, np_in)


def generate_logdet(prob) -> float:
    """Dense + refinement log-determinant (src/orchestrate.jl:89-97)."""
    _require(prob)
    out = C.c_double()
    nat.call("ggp_generate_logdet", prob.handle, C.byref(out), _stream())
    return out.value


def refine_logdet(prob) -> float:
    """Sum of log std over refined points (src/api.jl:24-27)."""
    _require(prob)
    out = C.c_double()
    nat.call("ggp_refine_logdet", prob.handle, C.byref(out), _stream())
    return out.value


def refine_logdet_terms(prob, as_numpy=True):
    """Per-point log std, tree order (src/api.jl:30-57)."""
    _require(prob)
    out = _empty(prob.M, prob.dtype)
    nat.call("ggp_refine_logdet_terms", prob.handle, _ptr(out), _stream())
    return _out(out, prob.M, as_numpy)


def refine_inv(prob, values_tree):
    """xi of the refined points from tree-order values (src/api.jl:66-103)."""
    _require(prob)
    v, np_in = _dev(values_tree, prob.N, prob.dtype)
    out = _empty(prob.M, prob.dtype)
    nat.call("ggp_refine_inv", prob.handle, _ptr(v), _ptr(out), _stream())
    return _out(out, prob.M, np_in)


def refine(prob, initial_values, xi_ref):
    """Forward refinement from the first n0 values (src/api.jl:113-182)."""
    _require(prob)
    torch = _torch()
    iv, np_in = _dev(initial_values, prob.n0, prob.dtype)
    xr, _ = _dev(xi_ref, prob.M, prob.dtype) if prob.M else (_empty(1, prob.dtype), False)
    v = torch.zeros(prob.N, dtype=iv.dtype, device="cuda")
    v[: prob.n0] = iv
    nat.call("ggp_refine", prob.handle, _ptr(v), _ptr(xr), _stream())
    return _out(v, prob.N, np_in)


# ---- adjoints ----------------------------------------------------------------------------------
def generate_grad_xi(prob, vbar):
    """G^T vbar, original order in and out (src/grad.jl:392-506)."""
    _require(prob)
    vb, np_in = _dev(vbar, prob.N, prob.dtype)
    out = _empty(prob.N, prob.dtype)
    nat.call("ggp_generate_grad_xi", prob.handle, _ptr(vb), _ptr(out), _stream())
    return _out(out, prob.N, np_in)


def generate_grad_vals(prob, xi, vbar):
    """d<vbar, generate(xi)>/dvals (src/grad_generate_vals.jl:111-282)."""
    _require(prob)
    x, np_in = _dev(xi, prob.N, prob.dtype)
    vb, _ = _dev(vbar, prob.N, prob.dtype)
    out = _empty(_nb(prob), prob.dtype)
    nat.call("ggp_generate_grad_vals", prob.handle, _ptr(x), _ptr(vb), _ptr(out), _stream())
    return _out(out, _nb(prob), np_in)


def refine_logdet_grad_vals(prob, as_numpy=True):
    """d(refine_logdet)/dvals (src/grad.jl:96-119)."""
    _require(prob)
    out = _empty(_nb(prob), prob.dtype)
    nat.call("ggp_refine_logdet_grad_vals", prob.handle, _ptr(out), None, _stream())
    return _out(out, _nb(prob), as_numpy)


def generate_logdet_and_grad_vals(prob, as_numpy=True):
    """(generate_logdet, its d/dvals) in one pass (src/grad.jl:680-715)."""
    _require(prob)
    out = _empty(_nb(prob), prob.dtype)
    ld = C.c_double()
    nat.call("ggp_generate_logdet_grad_vals", prob.handle, _ptr(out), C.byref(ld), _stream())
    return ld.value, _out(out, _nb(prob), as_numpy)


def generate_logdet_grad_vals(prob, as_numpy=True):
    """d(generate_logdet)/dvals (src/grad.jl:149-154)."""
    return generate_logdet_and_grad_vals(prob, as_numpy)[1]


def refine_inv_loss_grad_vals(prob, values_tree):
    """(0.5*||refine_inv(values)||^2, its d/dvals) (src/grad.jl:626-671)."""
    _require(prob)
    v, np_in = _dev(values_tree, prob.N, prob.dtype)
    out = _empty(_nb(prob), prob.dtype)
    loss = C.c_double()
    nat.call("ggp_refine_inv_loss_grad_vals", prob.handle, _ptr(v), _ptr(out), C.byref(loss),
             _stream())
    return loss.value, _out(out, _nb(prob), np_in)


def generate_inv_loss_grad_vals(prob, data):
    """(0.5*||generate_inv(data)||^2, its d/dvals), data in original order (src/grad.jl:514-529)."""
    _require(prob)
    d, np_in = _dev(data, prob.N, prob.dtype)
    out = _empty(_nb(prob), prob.dtype)
    loss = C.c_double()
    nat.call("ggp_generate_inv_loss_grad_vals", prob.handle, _ptr(d), _ptr(out), C.byref(loss),
             _stream())
    return loss.value, _out(out, _nb(prob), np_in)


# ---- gradients w.r.t. the point positions -------------------------------------------------------
# Results are (N, D) in tree order: the memory layout of the reference's (D, N) matrix. They are
# gradients w.r.t. the continuous positions x = scale * coords, the lattice straight-through.
def _points(prob, fn, vec, as_numpy):
    _require(prob)
    args, np_in = [], as_numpy
    if vec is not None:
        v, np_in = _dev(vec, prob.N, prob.dtype)
        args.append(_ptr(v))
    out = _empty(prob.N * prob.D, prob.dtype)
    s = C.c_double()
    nat.call(fn, prob.handle, *args, _ptr(out), C.byref(s), _stream())
    t = out[: prob.N * prob.D].view(prob.N, prob.D)
    return s.value, (t.cpu().numpy() if np_in else t)


def refine_logdet_grad_points(prob, as_numpy=True):
    """d(refine_logdet)/dpoints (src/grad.jl:168-226)."""
    return _points(prob, "ggp_refine_logdet_grad_points", None, as_numpy)[1]


def generate_logdet_grad_points(prob, as_numpy=True):
    """d(generate_logdet)/dpoints, dense + refinement (src/grad.jl:242-247)."""
    return _points(prob, "ggp_generate_logdet_grad_points", None, as_numpy)[1]


def generate_logdet_and_grad_points(prob, as_numpy=True):
    """(generate_logdet, its d/dpoints) in one pass."""
    return _points(prob, "ggp_generate_logdet_grad_points", None, as_numpy)


def refine_inv_loss_grad_points(prob, values_tree):
    """(0.5*||refine_inv(values)||^2, its d/dpoints), values in tree order
    (src/grad.jl:259-319)."""
    return _points(prob, "ggp_refine_inv_loss_grad_points", values_tree, True)


def generate_inv_loss_grad_points(prob, data):
    """(0.5*||generate_inv(data)||^2, its d/dpoints), data in original order
    (src/grad.jl:368-377)."""
    return _points(prob, "ggp_generate_inv_loss_grad_points", data, True)
