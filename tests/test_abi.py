"""The C-ABI boundary without a GPU: the library loads, exports every symbol declared in
include/*.h, and rejects bad problems with the documented status codes before touching the
device (check_graph, src/graph_build.jl:20-57; unsupported k / D, csrc/graphgp_capi.cu:53-68)."""
import ctypes as C
import os
import re

import numpy as np
import pytest

from conftest import ROOT, load_fixture

from graphgp_hip import _native as nat

HEADERS = [os.path.join(ROOT, "include", h) for h in ("graphgp_hip.h", "graphgp_graph.h")]


def declared(path):
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"\b((?:ggp|gphip)_[a-z_0-9]+)\s*\(", text)


@pytest.mark.parametrize("header", HEADERS, ids=os.path.basename)
def test_library_exports_every_declared_symbol(header):
    lib = C.CDLL(nat.HIP_LIB if "hip" in os.path.basename(header) else nat.GRAPH_LIB)
    names = declared(header)
    assert names
    for n in names:
        assert hasattr(lib, n), n


def _create(coords, nbr, offs, n0, k, D, scale=1e-6, dtype=0, idx=None):
    lib = nat.hip()
    h = C.c_void_p()
    rc = lib.ggp_graph_create(C.byref(h), coords.ctypes.data, nbr.ctypes.data if nbr.size else None,
                              offs.ctypes.data, len(offs),
                              None if idx is None else idx.ctypes.data, n0, k, len(coords), D,
                              scale, dtype)
    return rc, lib.ggp_last_error().decode()


def test_create_rejects_bad_inputs_before_any_device_call():
    z = load_fixture("small")
    coords = np.ascontiguousarray(z["coords"], np.uint32)
    nbr = np.ascontiguousarray(z["neighbors"], np.int64)
    offs = np.ascontiguousarray(z["offsets"], np.int64)
    n0 = int(z["n0"])
    assert _create(coords, nbr, offs, n0, 32, 3)[0] == 2         # k above 31 unsupported
    assert _create(coords, nbr, offs, n0, 0, 3)[0] == 2          # k = 0 unsupported
    assert _create(coords, nbr, offs, n0, 10, 5)[0] == 3         # D unsupported
    bad = offs.copy(); bad[0] += 1
    assert _create(coords, nbr, bad, n0, 10, 3)[0] == 4          # offsets[0] != n0
    nb2 = nbr.copy(); nb2[-1, 0] = len(coords) - 1
    rc, msg = _create(coords, nb2, offs, n0, 10, 3)
    assert rc == 4 and "level" in msg or "topological" in msg
    nb3 = nbr.copy(); nb3[5, 2] = -1
    assert _create(coords, nb3, offs, n0, 10, 3)[0] == 4         # unset neighbour
    idx = np.arange(len(coords), dtype=np.int64); idx[3] = idx[4]
    assert _create(coords, nbr, offs, n0, 10, 3, idx=idx)[0] == 4  # not a permutation
    assert _create(coords, nbr, offs, n0, 10, 3, scale=-1.0)[0] == 7
    assert _create(coords, nbr, offs, n0, 10, 3, dtype=9)[0] == 7
    assert nat.hip().ggp_supported(8, 3) == 0
    assert nat.hip().ggp_supported(9, 3) == 0
    assert nat.hip().ggp_supported(31, 4) == 0
    assert nat.hip().ggp_supported(32, 3) == 2
    assert nat.hip().ggp_supported(8, 5) == 3


def test_ops_require_a_device_problem():
    import graphgp_hip as G
    z = load_fixture("small")
    prob = G.GraphGPProblem(z["coords"], z["neighbors"], z["offsets"], int(z["n0"]),
                            float(z["scale"]), z["cov_bins32"], z["cov_vals32"])
    with pytest.raises(TypeError):
        G.generate(prob, np.zeros(prob.N, np.float32))


def test_stateless_entry_points_reject_bad_arguments_before_any_device_call():
    """gphip_refine_logdet_f32 / gphip_refine_inv_f32 return the reference's codes for an
    unsupported k (2) or ndim (3) (csrc/graphgp_capi.cu:53-68) and 7 for a null array, before
    any HIP call."""
    lib = nat.hip()
    f32 = C.c_float(1e-6)
    dummy = C.c_void_p(16)  # never dereferenced: every case below is rejected first
    for fn in (lib.gphip_refine_logdet_f32, lib.gphip_refine_logdet_f64):
        sc = f32 if fn is lib.gphip_refine_logdet_f32 else C.c_double(1e-6)
        assert fn(dummy, sc, dummy, dummy, dummy, dummy, 10, 32, 100, 50, 3, None) == 2
        assert fn(dummy, sc, dummy, dummy, dummy, dummy, 10, 0, 100, 50, 3, None) == 2
        assert fn(dummy, sc, dummy, dummy, dummy, dummy, 10, 8, 100, 50, 5, None) == 3
        assert fn(None, sc, dummy, dummy, dummy, dummy, 10, 8, 100, 50, 3, None) == 7
        assert fn(dummy, sc, dummy, dummy, dummy, dummy, 10, 8, 100, 1, 3, None) == 7
    assert lib.gphip_refine_inv_f32(dummy, f32, dummy, dummy, dummy, None, dummy, 10, 8, 100, 50,
                                    3, None) == 7
    assert lib.gphip_refine_inv_f32(dummy, f32, dummy, dummy, dummy, dummy, dummy, 10, 8, 100,
                                    50, 1, None) == 3
    assert b"ndim" in lib.ggp_last_error()
