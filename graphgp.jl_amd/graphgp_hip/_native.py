"""ctypes bindings of libgraphgp_hip.so (include/graphgp_hip.h) and libggp_graph.so
(include/graphgp_graph.h), built in-tree next to this package.

Loading is explicit and loud: if the HIP library has not been built, `hip()` raises; there is
no CPU fallback anywhere in the package.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

_PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(_PKG)                       # graphgp.jl_amd/
CSRC = os.path.join(ROOT, "csrc")
HIP_LIB = os.path.join(ROOT, "libgraphgp_hip.so")
GRAPH_LIB = os.path.join(ROOT, "libggp_graph.so")

GGP_F32, GGP_F64 = 0, 1
STATUS = {
    0: "ok", 2: "k unsupported", 3: "D unsupported", 4: "malformed graph", 5: "HIP error",
    6: "dense covariance not positive definite", 7: "invalid argument", 8: "no covariance set",
}


class GraphGPError(RuntimeError):
    def __init__(self, fn, code, msg):
        super().__init__(f"{fn} returned {code} ({STATUS.get(code, '?')}): {msg}")
        self.code = code


def build(jobs: int = 8) -> None:
    """Compile both libraries for gfx950 (hipcc) / the host (g++)."""
    subprocess.run(["make", "-C", CSRC, f"-j{jobs}", "all"], check=True)


_P = C.c_void_p
_I64 = C.c_int64
_I32 = C.c_int32
_DP = C.POINTER(C.c_double)

_HIP_SIGS = {
    "ggp_last_error": (C.c_char_p, []),
    "ggp_supported": (C.c_int, [_I64, _I32]),
    "ggp_graph_create": (C.c_int, [C.POINTER(_P), _P, _P, _P, _I64, _P, _I64, _I64, _I64, _I32,
                                   C.c_double, _I32]),
    "ggp_graph_destroy": (C.c_int, [_P]),
    "ggp_graph_shape": (C.c_int, [_P, C.POINTER(_I64), C.POINTER(_I64), C.POINTER(_I64),
                                  C.POINTER(_I32), C.POINTER(_I64), C.POINTER(_I32)]),
    "ggp_set_cov_iso": (C.c_int, [_P, _P, _P, _I64]),
    "ggp_set_cov_aniso": (C.c_int, [_P, _P, _I64, _P, _I64, _P, C.c_double]),
    "ggp_kernel_timers": (C.c_int, [_P, _I32]),
    "ggp_kernel_timer_read": (C.c_int, [_P, C.c_char_p, _DP, C.POINTER(_I64)]),
    "ggp_selftest_sqrt_f32": (C.c_int, [C.c_uint32, C.c_uint32, C.POINTER(C.c_uint64)]),
    "ggp_selftest_div": (C.c_int, [C.c_int32, C.c_uint64, C.c_uint64, C.c_uint32, C.c_uint64,
                                   C.POINTER(C.c_uint64)]),
    "ggp_generate": (C.c_int, [_P, _P, _P, _P]),
    "ggp_generate_inv": (C.c_int, [_P, _P, _P, _P]),
    "ggp_generate_logdet": (C.c_int, [_P, _DP, _P]),
    "ggp_refine_logdet_terms": (C.c_int, [_P, _P, _P]),
    "ggp_refine_logdet": (C.c_int, [_P, _DP, _P]),
    "ggp_refine_inv": (C.c_int, [_P, _P, _P, _P]),
    "ggp_refine": (C.c_int, [_P, _P, _P, _P]),
    "ggp_generate_grad_xi": (C.c_int, [_P, _P, _P, _P]),
    "ggp_generate_grad_vals": (C.c_int, [_P, _P, _P, _P, _P]),
    "ggp_refine_logdet_grad_vals": (C.c_int, [_P, _P, _DP, _P]),
    "ggp_generate_logdet_grad_vals": (C.c_int, [_P, _P, _DP, _P]),
    "ggp_refine_inv_loss_grad_vals": (C.c_int, [_P, _P, _P, _DP, _P]),
    "ggp_generate_inv_loss_grad_vals": (C.c_int, [_P, _P, _P, _DP, _P]),
    "ggp_refine_logdet_grad_points": (C.c_int, [_P, _P, _DP, _P]),
    "ggp_generate_logdet_grad_points": (C.c_int, [_P, _P, _DP, _P]),
    "ggp_refine_inv_loss_grad_points": (C.c_int, [_P, _P, _P, _DP, _P]),
    "ggp_generate_inv_loss_grad_points": (C.c_int, [_P, _P, _P, _DP, _P]),
    "ggp_build_graph_device": (C.c_int, [_P, _I64, _I32, _I64, _I64, _I32, _P, _P, _P, _P, _I64,
                                         C.POINTER(_I64), _DP, _P]),
    # stateless entry points with the reference's accelerator signatures
    "gphip_refine_logdet_f32": (C.c_int, [_P, C.c_float, _P, _P, _P, _P, _I64, _I64, _I64, _I64,
                                          _I64, _P]),
    "gphip_refine_inv_f32": (C.c_int, [_P, C.c_float, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64,
                                       _I64, _P]),
    "gphip_refine_logdet_f32_noalloc": (C.c_int, [_P, C.c_float, _P, _P, _P, _P, _I64, _I64, _I64,
                                                  _I64, _I64, _P]),
    "gphip_refine_logdet_f64": (C.c_int, [_P, C.c_double, _P, _P, _P, _P, _I64, _I64, _I64, _I64,
                                          _I64, _P]),
    "gphip_refine_inv_f64": (C.c_int, [_P, C.c_double, _P, _P, _P, _P, _P, _I64, _I64, _I64,
                                       _I64, _I64, _P]),
}

_GRAPH_SIGS = {
    "ggp_build_graph": (C.c_int, [_P, _I64, _I32, _I64, _I64, _I32, _I32, C.POINTER(_P)]),
    "ggp_built_graph_shape": (C.c_int, [_P, C.POINTER(_I64), C.POINTER(_I64), C.POINTER(_I64),
                                        C.POINTER(_I32), C.POINTER(_I64)]),
    "ggp_built_graph_copy": (C.c_int, [_P, _P, _P, _P, _P, _DP]),
    "ggp_built_graph_free": (None, [_P]),
}

_hip = None
_graph = None


def _bind(path, sigs):
    lib = C.CDLL(path)
    for name, (res, args) in sigs.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


def hip():
    """The loaded HIP library; raises if it has not been built."""
    global _hip
    if _hip is None:
        if not os.path.exists(HIP_LIB):
            raise RuntimeError(
                f"libgraphgp_hip.so not found at {HIP_LIB}: build it first "
                "(python -c 'import __graft_entry__ as g; g.build()' or make -C graphgp.jl_amd/csrc)")
        _torch_runtime_first()
        _hip = _bind(HIP_LIB, _HIP_SIGS)
    return _hip


def _torch_runtime_first():
    """Load torch's HIP runtime before the library. Both provide libamdhip64.so.7; loaded
    first, torch's copy satisfies the library's dependency and the process has one runtime.
    Loaded the other way round the process ends up with two, and torch then sees no GPU."""
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def graphlib():
    global _graph
    if _graph is None:
        if not os.path.exists(GRAPH_LIB):
            raise RuntimeError(f"libggp_graph.so not found at {GRAPH_LIB}: build it first")
        _graph = _bind(GRAPH_LIB, _GRAPH_SIGS)
    return _graph


def check(fn: str, rc: int) -> None:
    if rc != 0:
        msg = hip().ggp_last_error()
        raise GraphGPError(fn, rc, msg.decode() if msg else "")


def call(name: str, *args) -> None:
    check(name, getattr(hip(), name)(*args))
