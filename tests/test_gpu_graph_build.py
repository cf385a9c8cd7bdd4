"""The graph built on the GPU (ggp_build_graph_device) against the host builder, which itself
reproduces the reference's fixture graphs (tests/test_graph_and_tables.py): every output —
lattice coordinates, neighbours, level offsets, permutation and scale — must be identical,
including inputs full of ties (duplicate points, equal split coordinates) where only the
reference's tie-breaking decides the order."""
import sys
import time

import numpy as np
import pytest

from conftest import load_fixture

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def G():
    import graphgp_hip
    return graphgp_hip


def _points(kind, N, D, seed):
    rng = np.random.default_rng(seed)
    if kind == "uniform":
        return rng.random((N, D))
    if kind == "normal":
        return rng.standard_normal((N, D))
    if kind == "clustered":
        cent = rng.random((32, D))
        near = cent[rng.integers(0, 32, N)] + 0.01 * rng.standard_normal((N, D))
        return np.where((rng.random(N) < 0.8)[:, None], near, rng.random((N, D)))
    if kind == "ties":  # a coarse grid: many duplicate points and equal coordinates
        return rng.integers(0, 6, (N, D)).astype(np.float64) - 2.0
    raise ValueError(kind)


def _same(a, b):
    c1, n1, o1, z1, s1, i1 = a
    c2, n2, o2, z2, s2, i2 = b
    assert z1 == z2
    np.testing.assert_array_equal(o1, o2)
    np.testing.assert_array_equal(i1, i2)
    np.testing.assert_array_equal(n1, n2)
    np.testing.assert_array_equal(c1, c2)
    assert s1 == s2


CASES = [("uniform", 20000, 3, 100, 8), ("normal", 30000, 3, 64, 10),
         ("clustered", 40000, 3, 256, 16), ("ties", 5000, 3, 50, 8), ("ties", 3000, 2, 20, 6),
         ("uniform", 10000, 2, 40, 4), ("normal", 10000, 4, 100, 20), ("uniform", 4000, 1, 16, 5),
         ("uniform", 3000, 3, 32, 31), ("uniform", 3000, 3, 32, 32), ("uniform", 2, 2, 1, 1),
         ("normal", 1023, 3, 16, 8), ("normal", 1024, 3, 16, 8), ("normal", 1025, 3, 16, 8)]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}_N{c[1]}_D{c[2]}_n0{c[3]}_k{c[4]}")
def test_device_build_equals_host_build(gpu, case):
    kind, N, D, n0, k = case
    _say(f"case build {kind} N={N} D={D} n0={n0} k={k}")
    pts = _points(kind, N, D, seed=N + D + k)
    _same(G().build_graph_device_arrays(pts, n0, k), G().build_graph_arrays(pts, n0, k))


@pytest.mark.parametrize("name", ["generate_parity", "aniso_parity"])
def test_device_build_reproduces_fixture_graph(gpu, name):
    """The reference-built fixture graphs, rebuilt on the GPU from their points."""
    _say(f"case build fixture {name}")
    z = load_fixture(name)
    coords, nbr, offs, idx = z["coords"], z["neighbors"], z["offsets"], z["indices"]
    N, D = coords.shape
    pts = np.zeros((N, D))
    pts[idx] = coords.astype(np.float64) * float(z["scale"])
    c2, n2, o2, n0, s2, i2 = G().build_graph_device_arrays(pts, int(z["n0"]), nbr.shape[1])
    assert n0 == int(z["n0"])
    np.testing.assert_array_equal(o2, offs)
    np.testing.assert_array_equal(i2, idx)
    np.testing.assert_array_equal(n2, nbr)
    np.testing.assert_array_equal(c2, coords)


def test_device_build_one_million_points(gpu):
    """The 1M-point, k = 8 graph of the headline workload: identical to the host build; the
    problem built from it runs generate like the host-built one."""
    _say("case build 1M")
    pts = _points("uniform", 1_000_000, 3, seed=1)
    t0 = time.perf_counter()
    dev = G().build_graph_device_arrays(pts, 1000, 8)
    t1 = time.perf_counter()
    host = G().build_graph_arrays(pts, 1000, 8)
    t2 = time.perf_counter()
    _say(f"  device build {t1 - t0:.3f} s, host build {t2 - t1:.3f} s")
    _same(dev, host)


def test_device_build_rejects_bad_arguments(gpu):
    pts = _points("uniform", 100, 3, seed=0)
    for n0, k in ((10, 33), (4, 8), (100, 8), (10, 0)):
        with pytest.raises(G().GraphGPError):
            G().build_graph_device_arrays(pts, n0, k)
    with pytest.raises(G().GraphGPError):
        G().build_graph_device_arrays(np.zeros((100, 5)), 10, 4)
