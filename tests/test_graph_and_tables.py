"""Host-side inputs of the path: the graph builder (src/graph_build.jl, src/tree_special.jl),
check_graph, and the covariance tables / hyperparameter gradient (src/extras.jl)."""
import math

import numpy as np
import pytest

import graphgp_hip as G
from conftest import GOLDEN, load_fixture
import os


@pytest.mark.parametrize("name", ["generate_parity", "aniso_parity"])
def test_build_graph_reproduces_fixture_graph(name):
    """The fixture graphs were built by the reference pipeline; rebuilding from the lattice
    points (original order) gives the same neighbours, levels, permutation and lattice."""
    z = load_fixture(name)
    coords, nbr, offs, idx = z["coords"], z["neighbors"], z["offsets"], z["indices"]
    N, D = coords.shape
    pts = np.zeros((N, D))
    pts[idx] = coords.astype(np.float64) * float(z["scale"])
    c2, n2, o2, n0, s2, i2 = G.build_graph_arrays(pts, int(z["n0"]), nbr.shape[1])
    assert n0 == int(z["n0"])
    np.testing.assert_array_equal(o2, offs)
    np.testing.assert_array_equal(i2, idx)
    np.testing.assert_array_equal(n2, nbr)
    np.testing.assert_array_equal(c2, coords)
    assert s2 == pytest.approx(float(z["scale"]), rel=1e-15)


@pytest.mark.parametrize("name", ["small", "medium"])
def test_build_graph_on_tree_ordered_fixture_is_identity(name):
    z = load_fixture(name)
    c2, n2, o2, n0, s2, i2 = G.build_graph_arrays(z["coords"].astype(np.float64), int(z["n0"]),
                                                  z["neighbors"].shape[1])
    np.testing.assert_array_equal(i2, np.arange(len(i2)))
    np.testing.assert_array_equal(o2, z["offsets"])
    np.testing.assert_array_equal(n2, z["neighbors"])


def test_built_graph_invariants():
    rng = np.random.default_rng(0)
    pts = rng.random((5000, 3))
    bins, vals = G.rbf_kernel(1.0, 0.1, 1e-4, 2.0, 100)
    prob = G.build_graph(pts, 100, 8, bins, vals)
    G.check_graph(prob)
    assert prob.offsets[0] == prob.n0 and prob.offsets[-1] == prob.N
    assert sorted(prob.indices.tolist()) == list(range(prob.N))
    # every neighbour list is sorted by distance (src/tree_special.jl:322-328)
    x = prob.coords.astype(np.float64)
    for m in range(0, prob.M, 97):
        d = np.sum((x[prob.neighbors[m]] - x[prob.n0 + m]) ** 2, axis=1)
        assert np.all(np.diff(d) >= -1e-6 * d.max())


def test_check_graph_rejects_malformed():
    z = load_fixture("small")
    bins, vals = z["cov_bins64"], z["cov_vals64"]
    prob = G.GraphGPProblem(z["coords"], z["neighbors"], z["offsets"], int(z["n0"]),
                            float(z["scale"]), bins, vals)
    G.check_graph(prob)
    bad = z["offsets"].copy()
    bad[0] += 1
    with pytest.raises(ValueError):
        G.check_graph(G.GraphGPProblem(z["coords"], z["neighbors"], bad, int(z["n0"]),
                                       float(z["scale"]), bins, vals))
    nb = z["neighbors"].copy()
    nb[-1, 0] = len(z["coords"]) - 1     # a neighbour in its own (last) level
    with pytest.raises(ValueError):
        G.check_graph(G.GraphGPProblem(z["coords"], nb, z["offsets"], int(z["n0"]),
                                       float(z["scale"]), bins, vals))


# ---- tables (src/extras.jl) ---------------------------------------------------------------------
def test_rbf_table_matches_fixture_table():
    """small.npz was built with rbf_kernel(1, 0.3, 1e-4, 10, 1000; jitter=1e-3)
    (test/dump_reference.py:59-61, test/test_extras.jl:26-31)."""
    z = load_fixture("small")
    bins, vals = G.rbf_kernel(1.0, 0.3, 1e-4, 10.0, 1000, jitter=1e-3)
    np.testing.assert_allclose(bins, z["cov_bins64"], rtol=1e-14, atol=0)
    # the fixture table was evaluated by JAX; exp implementations differ by a few ulps in the tail
    np.testing.assert_allclose(vals, z["cov_vals64"], rtol=1e-10, atol=1e-300)


@pytest.mark.parametrize("p", [1, 2])
def test_matern_closed_forms(p):
    bins, vals = G.matern_kernel(p, 2.0, 0.3, 1e-4, 5.0, 300)
    s = math.sqrt(2 * p + 1) * bins / 0.3
    closed = 2.0 * np.exp(-s) * ((1 + s) if p == 1 else (1 + s + s * s / 3))
    np.testing.assert_allclose(vals, closed, rtol=1e-13)


def test_make_cov_bins():
    b = G.make_cov_bins(1e-4, 2.0, 1000)
    assert b[0] == 0.0 and len(b) == 1000
    np.testing.assert_allclose(b[1], 1e-4, rtol=1e-14)
    np.testing.assert_allclose(b[-1], 2.0, rtol=1e-14)
    assert np.all(np.diff(b) > 0)


def test_hyperparam_grad_analytic():
    g = np.random.default_rng(0).standard_normal(300)
    var, ell = 1.7, 0.4
    mk = lambda v, l: G.rbf_kernel(v, l, 1e-4, 3.0, 300, jitter=1e-5)
    got = G.hyperparam_grad(g, mk, [var, ell])
    bins, vals = mk(var, ell)
    dvar = vals / var
    dell = vals * bins ** 2 / ell ** 3
    np.testing.assert_allclose(got, [np.dot(dvar, g), np.dot(dell, g)], rtol=1e-12)
    mk2 = lambda v, l: G.matern_kernel(2, v, l, 1e-4, 3.0, 300)
    got2 = G.hyperparam_grad(g, mk2, [var, ell])
    h = 1e-6
    fd = [(np.dot(mk2(var + h, ell)[1], g) - np.dot(mk2(var - h, ell)[1], g)) / (2 * h),
          (np.dot(mk2(var, ell + h)[1], g) - np.dot(mk2(var, ell - h)[1], g)) / (2 * h)]
    np.testing.assert_allclose(got2, fd, rtol=1e-6)


def test_interchange_format_round_trip_and_reference_fixtures(tmp_path):
    """save_graph / load_graph use the reference's .npz schema (test/loadref.jl:17-26): a
    reference fixture loads to the same arrays the fixture loader builds, a saved graph reloads
    identically, and build_graph(cache=...) reuses the saved graph."""
    import graphgp_hip as G
    z = load_fixture("small")
    p64 = G.load_graph(os.path.join(GOLDEN, "small.npz"))
    assert p64.dtype == np.float64
    np.testing.assert_array_equal(p64.coords, z["coords"])
    np.testing.assert_array_equal(p64.neighbors, z["neighbors"])
    np.testing.assert_array_equal(p64.offsets, z["offsets"])
    np.testing.assert_array_equal(p64.vals, z["cov_vals64"])
    p32 = G.load_graph(os.path.join(GOLDEN, "small.npz"), dtype=np.float32)
    np.testing.assert_array_equal(p32.vals, z["cov_vals32"])
    out = tmp_path / "g.npz"
    G.save_graph(p32, out)
    q = G.load_graph(out)
    for a in ("coords", "neighbors", "offsets", "bins", "vals"):
        np.testing.assert_array_equal(getattr(q, a), getattr(p32, a))
    assert q.n0 == p32.n0 and q.scale == p32.scale and q.dtype == np.float32
    # the build cache
    rng = np.random.default_rng(4)
    pts = rng.random((3000, 3))
    bins, vals = G.rbf_kernel(1.0, 0.1, 1e-4, 2.0, 100)
    cache = tmp_path / "cache.npz"
    a = G.build_graph(pts, 100, 8, bins, vals, cache=str(cache))
    assert cache.exists()
    b = G.build_graph(pts, 100, 8, bins, vals, cache=str(cache))
    for f in ("coords", "neighbors", "offsets", "indices"):
        np.testing.assert_array_equal(getattr(a, f), getattr(b, f))
    # anisotropic covariance survives the round trip
    cov = G.AnisoCov(np.linspace(0, 1, 8), np.linspace(0, 0.1, 4), np.ones((8, 4)), 2.0)
    pa = G.GraphGPProblem(a.coords, a.neighbors, a.offsets, a.n0, a.scale, indices=a.indices,
                          cov=cov)
    G.save_graph(pa, tmp_path / "an.npz")
    qa = G.load_graph(tmp_path / "an.npz")
    np.testing.assert_array_equal(qa.cov.grid, cov.grid)
    assert qa.cov.alpha == 2.0
