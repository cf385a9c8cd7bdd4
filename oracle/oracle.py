"""ctypes wrapper over libggp_oracle.so — TEST INFRASTRUCTURE ONLY.

The oracle is the CPU restatement of GraphGP.jl's refinement path (see graphgp_oracle.cpp for the
per-function reference citations). Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this module; the product never does.

Problems are described with the same arrays the HIP library takes: coords (N, D) uint32 in tree
order, neighbors (M, K) int64 0-based, offsets int64 0-based exclusive ends (offsets[0] = n0),
optional indices (N,) int64 (indices[tree_pos] = original_pos), bins/vals (nbins,) float.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libggp_oracle.so")


class _Prob(C.Structure):
    _fields_ = [
        ("coords", C.c_void_p),
        ("neighbors", C.c_void_p),
        ("offsets", C.c_void_p),
        ("indices", C.c_void_p),
        ("n_offsets", C.c_int64),
        ("n0", C.c_int64),
        ("K", C.c_int64),
        ("N", C.c_int64),
        ("D", C.c_int64),
        ("nbins", C.c_int64),
        ("scale", C.c_double),
        ("bins", C.c_void_p),
        ("vals", C.c_void_p),
        ("nthreads", C.c_int),
        ("aniso", C.c_int),
        ("sbins", C.c_void_p),
        ("zbins", C.c_void_p),
        ("grid", C.c_void_p),
        ("ns", C.c_int64),
        ("nz", C.c_int64),
        ("alpha", C.c_double),
        ("acc64", C.c_int),
    ]


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (a few seconds)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "all"], check=True)
    return _LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = C.CDLL(_LIB_PATH)
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


class Problem:
    """A refinement problem held in numpy arrays, in the oracle's (and the HIP ABI's) layout."""

    def __init__(self, coords, neighbors, offsets, n0, scale, bins, vals, indices=None,
                 dtype=np.float64, nthreads=None, aniso=None, acc64=False):
        """aniso: optional (spatial_bins, z_bins, grid (ns, nz), alpha) — the anisotropic
        covariance, which then replaces (bins, vals) (src/aniso.jl). acc64: sum the d/dvals
        histograms in double (the reference sums in the element type)."""
        self.dtype = np.dtype(dtype)
        self.coords = np.ascontiguousarray(coords, dtype=np.uint32)
        self.neighbors = np.ascontiguousarray(neighbors, dtype=np.int64)
        self.offsets = np.ascontiguousarray(offsets, dtype=np.int64)
        self.indices = None if indices is None else np.ascontiguousarray(indices, dtype=np.int64)
        self.n0 = int(n0)
        self.scale = float(scale)
        self.bins = np.ascontiguousarray(bins, dtype=self.dtype)
        self.vals = np.ascontiguousarray(vals, dtype=self.dtype)
        self.N, self.D = self.coords.shape
        self.M = self.N - self.n0
        self.K = self.neighbors.shape[1] if self.neighbors.ndim == 2 else 0
        assert self.neighbors.shape[0] == self.M
        self.nthreads = int(nthreads or os.cpu_count() or 1)
        self.aniso = aniso
        self.acc64 = bool(acc64)
        if aniso is not None:
            sb, zb, grid, alpha = aniso
            self._sb = np.ascontiguousarray(sb, dtype=self.dtype)
            self._zb = np.ascontiguousarray(zb, dtype=self.dtype)
            self._grid = np.ascontiguousarray(grid, dtype=self.dtype)
            assert self._grid.shape == (len(self._sb), len(self._zb))
            an = (1, _ptr(self._sb), _ptr(self._zb), _ptr(self._grid), len(self._sb),
                  len(self._zb), float(alpha))
        else:
            an = (0, None, None, None, 0, 0, 0.0)
        self._s = _Prob(_ptr(self.coords), _ptr(self.neighbors), _ptr(self.offsets),
                        _ptr(self.indices), len(self.offsets), self.n0, self.K, self.N, self.D,
                        len(self.bins), self.scale, _ptr(self.bins), _ptr(self.vals),
                        self.nthreads, *an, int(self.acc64))

    # the struct keeps raw pointers: keep arrays alive via self
    def with_vals(self, vals):
        return Problem(self.coords, self.neighbors, self.offsets, self.n0, self.scale, self.bins,
                       vals, self.indices, self.dtype, self.nthreads, self.aniso, self.acc64)

    def with_dtype(self, dtype):
        return Problem(self.coords, self.neighbors, self.offsets, self.n0, self.scale,
                       self.bins.astype(dtype), self.vals.astype(dtype), self.indices, dtype,
                       self.nthreads, self.aniso, self.acc64)

    @property
    def _sfx(self):
        return "f32" if self.dtype == np.float32 else "f64"

    def _call(self, name, *args):
        fn = getattr(lib(), f"oracle_{name}_{self._sfx}")
        fn.restype = C.c_int
        rc = fn(C.byref(self._s), *args)
        if rc != 0:
            raise RuntimeError(f"oracle {name} returned {rc}")

    def _vec(self, x, n):
        x = np.ascontiguousarray(x, dtype=self.dtype)
        assert x.shape == (n,), (x.shape, n)
        return x

    # ---- forward ops ----
    def refine_logdet_terms(self):
        out = np.zeros(max(self.M, 1), self.dtype)
        self._call("refine_logdet_terms", _ptr(out))
        return out[: self.M]

    def refine_inv(self, values_tree):
        v = self._vec(values_tree, self.N)
        out = np.zeros(max(self.M, 1), self.dtype)
        self._call("refine_inv", _ptr(v), _ptr(out))
        return out[: self.M]

    def refine_meanvec_std(self):
        mv = np.zeros((max(self.M, 1), self.K), self.dtype)
        sd = np.zeros(max(self.M, 1), self.dtype)
        self._call("refine_meanvec_std", _ptr(mv), _ptr(sd))
        return mv[: self.M], sd[: self.M]

    def refine(self, initial_values, xi_ref):
        v = np.zeros(self.N, self.dtype)
        v[: self.n0] = initial_values
        xr = self._vec(xi_ref, self.M) if self.M else np.zeros(1, self.dtype)
        self._call("refine", _ptr(v), _ptr(xr))
        return v

    def generate(self, xi):
        out = np.zeros(self.N, self.dtype)
        self._call("generate", _ptr(self._vec(xi, self.N)), _ptr(out))
        return out

    def generate_inv(self, values):
        out = np.zeros(self.N, self.dtype)
        self._call("generate_inv", _ptr(self._vec(values, self.N)), _ptr(out))
        return out

    def generate_logdet(self):
        out = C.c_double()
        self._call("generate_logdet", C.byref(out))
        return out.value

    # ---- gradients ----
    def refine_logdet_grad_vals(self):
        dv = np.zeros(len(self.bins), self.dtype)
        ld = C.c_double()
        self._call("refine_logdet_grad_vals", _ptr(dv), C.byref(ld))
        return ld.value, dv

    def generate_logdet_grad_vals(self):
        dv = np.zeros(len(self.bins), self.dtype)
        ld = C.c_double()
        self._call("generate_logdet_grad_vals", _ptr(dv), C.byref(ld))
        return ld.value, dv

    def refine_inv_loss_grad_vals(self, values_tree):
        dv = np.zeros(len(self.bins), self.dtype)
        loss = C.c_double()
        self._call("refine_inv_loss_grad_vals", _ptr(self._vec(values_tree, self.N)), _ptr(dv),
                   C.byref(loss))
        return loss.value, dv

    def generate_inv_loss_grad_vals(self, data):
        dv = np.zeros(len(self.bins), self.dtype)
        loss = C.c_double()
        self._call("generate_inv_loss_grad_vals", _ptr(self._vec(data, self.N)), _ptr(dv),
                   C.byref(loss))
        return loss.value, dv

    def generate_grad_xi(self, vbar):
        out = np.zeros(self.N, self.dtype)
        self._call("generate_grad_xi", _ptr(self._vec(vbar, self.N)), _ptr(out))
        return out

    def generate_grad_vals(self, xi, vbar):
        dv = np.zeros(len(self.bins), self.dtype)
        self._call("generate_grad_vals", _ptr(self._vec(xi, self.N)),
                   _ptr(self._vec(vbar, self.N)), _ptr(dv))
        return dv

    # ---- point-position gradients, (N, D) in tree order: the memory layout of the reference's
    # (D, N) Julia matrix ----
    def _pts(self, name, *vec):
        dp = np.zeros((self.N, self.D), self.dtype)
        out = C.c_double()
        self._call(name, *[_ptr(self._vec(v, self.N)) for v in vec], _ptr(dp), C.byref(out))
        return out.value, dp

    def refine_logdet_grad_points(self):
        return self._pts("refine_logdet_grad_points")

    def generate_logdet_grad_points(self):
        return self._pts("generate_logdet_grad_points")

    def refine_inv_loss_grad_points(self, values_tree):
        return self._pts("refine_inv_loss_grad_points", values_tree)

    def generate_inv_loss_grad_points(self, data):
        return self._pts("generate_inv_loss_grad_points", data)

    def dense_factor(self):
        L = np.zeros((self.n0, self.n0), self.dtype)
        self._call("dense_factor", _ptr(L))
        return L


# ---- primitive-level helpers (f64) ----
def cov_lookup(r, bins, vals):
    f = lib().oracle_cov_lookup_f64
    f.restype = C.c_double
    f.argtypes = [C.c_double, C.c_void_p, C.c_void_p, C.c_int64]
    b = np.ascontiguousarray(bins, np.float64)
    v = np.ascontiguousarray(vals, np.float64)
    return f(float(r), _ptr(b), _ptr(v), len(b))


def cov_lookup_weights(r, bins):
    f = lib().oracle_cov_lookup_weights_f64
    f.restype = None
    b = np.ascontiguousarray(bins, np.float64)
    lo, wlo, whi = C.c_int64(), C.c_double(), C.c_double()
    f(C.c_double(float(r)), _ptr(b), C.c_int64(len(b)), C.byref(lo), C.byref(wlo), C.byref(whi))
    return lo.value, wlo.value, whi.value


def chol_lower(A, dtype=np.float64):
    A = np.array(A, dtype=dtype, order="C")
    fn = lib().oracle_chol_lower_f64 if dtype == np.float64 else lib().oracle_chol_lower_f32
    fn.restype = None
    fn(_ptr(A), C.c_int64(A.shape[0]))
    return np.tril(A)


def mean_vec_solve(L):
    L = np.ascontiguousarray(L, np.float64)
    K = L.shape[0] - 1
    x = np.zeros(K)
    f = lib().oracle_mean_vec_solve_f64
    f.restype = None
    f(_ptr(x), _ptr(L), C.c_int64(K))
    return x


def chol_pullback(Lbar, L, dyn=False):
    L = np.ascontiguousarray(L, np.float64)
    Lb = np.array(Lbar, np.float64, order="C")
    Ab = np.zeros_like(L)
    f = lib().oracle_chol_pullback_dyn_f64 if dyn else lib().oracle_chol_pullback_f64
    f.restype = None
    f(_ptr(Ab), _ptr(Lb), _ptr(L), C.c_int64(L.shape[0]))
    return np.tril(Ab)


def max_threads():
    return int(lib().oracle_max_threads())
