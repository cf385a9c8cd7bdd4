"""The library's host code under AddressSanitizer and UndefinedBehaviorSanitizer, on the CPU.

tests/sanitize/Makefile builds pack_check with the host compiler and -fsanitize=address,undefined
from the sources of ggp_graph_create's validation and repacking (ggp_pack.cpp: the internal
Morton order, the int32 neighbour table, the reverse-neighbour lists and the sweep chunks) and
of the host graph builder (graph_build.cpp). pack_check runs them on graph files written here
(the reference's fixture graphs, edge shapes, rejected graphs, and graphs it builds itself from
random points) and checks the invariants of the packed layout; any sanitizer report or failed
invariant ends it with a non-zero status.
"""
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT, load_fixture

SAN = os.path.join(ROOT, "tests", "sanitize")
EXE = os.path.join(SAN, "pack_check")


@pytest.fixture(scope="module")
def pack_check():
    subprocess.run(["make", "-s", "-C", SAN], check=True)
    return EXE


def _run(exe, mode, path):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1", OMP_NUM_THREADS="4")
    r = subprocess.run([exe, mode, path], capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    return r.stdout.strip()


def _write_graph(path, coords, nbrs, offs, n0, idx=None):
    coords = np.ascontiguousarray(coords, np.uint32)
    nbrs = np.ascontiguousarray(nbrs, np.int64).reshape(-1)
    offs = np.ascontiguousarray(offs, np.int64)
    N, D = coords.shape
    k = nbrs.size // max(N - n0, 1) if N > n0 else 8
    hdr = np.array([N, D, n0, k, len(offs), idx is not None], np.int64)
    with open(path, "wb") as f:
        f.write(hdr.tobytes())
        f.write(coords.tobytes())
        f.write(nbrs.tobytes())
        f.write(offs.tobytes())
        if idx is not None:
            f.write(np.ascontiguousarray(idx, np.int64).tobytes())


@pytest.mark.parametrize("name", ["small", "medium", "generate_parity", "aniso_parity"])
def test_fixture_graphs(pack_check, tmp_path, name):
    z = load_fixture(name)
    p = str(tmp_path / "g.bin")
    idx = z["indices"] if "indices" in z.files else None
    _write_graph(p, z["coords"], z["neighbors"], z["offsets"], int(z["n0"]), idx)
    assert _run(pack_check, "graph", p) == "ok"


def test_edge_shapes_and_rejections(pack_check, tmp_path):
    z = load_fixture("small")
    c, nb, off, n0 = z["coords"], z["neighbors"], z["offsets"], int(z["n0"])
    p = str(tmp_path / "g.bin")
    # an empty level
    _write_graph(p, c, nb, np.concatenate([off[:2], off[1:2], off[2:]]), n0)
    assert _run(pack_check, "graph", p) == "ok"
    # points past the last level (the last level dropped from the offsets)
    _write_graph(p, c, nb, off[:-1], n0)
    assert _run(pack_check, "graph", p) == "ok"
    # the dense block only
    _write_graph(p, c[:n0], np.zeros((0, nb.shape[1]), np.int64), np.array([n0]), n0)
    assert _run(pack_check, "graph", p) == "ok"
    # a neighbour in its own level, and one out of range: status 4 (check_graph)
    bad = nb.copy()
    bad[-1, 0] = len(c) - 2
    _write_graph(p, c, bad, off, n0)
    assert _run(pack_check, "graph", p).startswith("rejected 4")
    bad[-1, 0] = len(c) + 5
    _write_graph(p, c, bad, off, n0)
    assert _run(pack_check, "graph", p).startswith("rejected 4")


@pytest.mark.parametrize("N,D,n0,k,seed", [(20000, 3, 200, 8, 1), (8000, 2, 100, 16, 2),
                                            (6000, 4, 64, 5, 3), (3000, 3, 40, 31, 4)])
def test_host_build_then_pack(pack_check, tmp_path, N, D, n0, k, seed):
    rng = np.random.default_rng(seed)
    pts = rng.random((N, D))
    pts[10:20] = pts[5]  # coincident points: lattice ties and zero distances
    p = str(tmp_path / "pts.bin")
    with open(p, "wb") as f:
        f.write(np.array([N, D, n0, k], np.int64).tobytes())
        f.write(np.ascontiguousarray(pts, np.float64).tobytes())
    assert _run(pack_check, "build", p).startswith("ok")
