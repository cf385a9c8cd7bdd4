"""GPU tests of the stateless entry points with the reference's accelerator signatures
(gphip_refine_logdet_f32 / gphip_refine_inv_f32 and their Float64 twins; the reference's
gpcuda_refine_logdet_f32 / gpcuda_refine_inv_f32, csrc/graphgp_capi.cu:70-94), called through
the C ABI on device arrays in the reference's layout (int64 point-major neighbours).

They run the handle path's factor kernels, so refine_inv is compared bit for bit with the oracle
and with ggp_refine_inv; refine_logdet (a sum of logs, device libm against host libm, summed in
another order) at 1e-5 (f32) / 1e-12 (f64) relative, as are the reference's fixtures.
"""
import ctypes as C
import sys

import numpy as np
import pytest

from conftest import load_fixture, relerr

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def G():
    import graphgp_hip
    return graphgp_hip


def O():
    import oracle
    return oracle


def lib():
    from graphgp_hip import _native as nat
    return nat.hip()


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def stateless(torch, prob, values):
    """(logdet, xi_ref) from the stateless entry points on the problem's arrays."""
    f64 = prob.dtype == np.float64
    tt = torch.float64 if f64 else torch.float32
    coords = _dev(torch, prob.coords)
    nbr = _dev(torch, prob.neighbors)
    bins, vals = _dev(torch, prob.bins), _dev(torch, prob.vals)
    out = torch.full((1,), float("nan"), dtype=tt, device="cuda")
    xi = torch.full((max(prob.M, 1),), float("nan"), dtype=tt, device="cuda")
    v = _dev(torch, values.astype(prob.dtype))
    sc = C.c_double(prob.scale) if f64 else C.c_float(prob.scale)
    L = lib()
    fl = L.gphip_refine_logdet_f64 if f64 else L.gphip_refine_logdet_f32
    fi = L.gphip_refine_inv_f64 if f64 else L.gphip_refine_inv_f32
    args = (prob.n0, prob.K, prob.N, len(prob.bins), prob.D, None)
    rc = fl(coords.data_ptr(), sc, nbr.data_ptr(), bins.data_ptr(), vals.data_ptr(),
            out.data_ptr(), *args)
    assert rc == 0, L.ggp_last_error()
    rc = fi(coords.data_ptr(), sc, nbr.data_ptr(), bins.data_ptr(), vals.data_ptr(),
            v.data_ptr(), xi.data_ptr(), *args)
    assert rc == 0, L.ggp_last_error()
    torch.cuda.synchronize()
    return float(out.cpu()[0]), xi.cpu().numpy()[:prob.M]


def _problem(N, D, n0, k, dtype, seed):
    rng = np.random.default_rng(seed)
    pts = rng.random((N, D))
    bins, vals = G().rbf_kernel(1.0, 0.1, 1e-4, 2.0, 500, jitter=1e-5)
    prob = G().build_graph(pts, n0, k, bins.astype(dtype), vals.astype(dtype))
    return prob, rng


SHAPES = [(4000, 3, 150, 8), (3000, 2, 100, 4), (3000, 4, 100, 10), (3000, 3, 200, 16),
          (2500, 3, 100, 5), (2000, 3, 128, 20), (1500, 3, 100, 30)]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"N{s[0]}_D{s[1]}_n0{s[2]}_k{s[3]}")
def test_stateless_vs_oracle_and_handle(gpu, shape, dtype):
    N, D, n0, k = shape
    _say(f"case stateless N={N} D={D} n0={n0} k={k} {np.dtype(dtype).name}")
    prob, rng = _problem(N, D, n0, k, dtype, seed=k + 3 * D)
    ref = O().Problem(prob.coords, prob.neighbors, prob.offsets, prob.n0, prob.scale, prob.bins,
                      prob.vals, indices=prob.indices, dtype=dtype)
    values = rng.standard_normal(N).astype(dtype)
    ld, xi = stateless(gpu, prob, values)
    xi_o = ref.refine_inv(values)
    np.testing.assert_array_equal(xi, xi_o)
    hp = G().to_backend(prob)
    np.testing.assert_array_equal(xi, G().refine_inv(hp, values))
    ld_o = float(np.sum(ref.refine_logdet_terms().astype(np.float64)))
    e = abs(ld - ld_o) / abs(ld_o)
    bar = 1e-5 if dtype == np.float32 else 1e-12
    _say(f"  refine_logdet: relative error {e:.3e} (bar {bar:.0e}); refine_inv bit-exact")
    assert e < bar


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_stateless_reference_fixture(gpu, dtype):
    """small.npz (test/reference, via test/test_refine.jl:1-30): refine_logdet and refine_inv
    at the reference's own tolerances."""
    _say(f"case stateless fixture {np.dtype(dtype).name}")
    z = load_fixture("small")
    s = "64" if dtype == np.float64 else "32"
    prob = G().GraphGPProblem(z["coords"], z["neighbors"], z["offsets"], int(z["n0"]),
                              float(z["scale"]), z["cov_bins" + s], z["cov_vals" + s])
    ld, xi = stateless(gpu, prob, z["values" + s])
    if dtype == np.float64:
        assert abs(ld - float(z["logdet64"])) <= 1e-6 * abs(float(z["logdet64"]))
        np.testing.assert_allclose(xi, z["xi64"], rtol=1e-6, atol=1e-8)
    else:
        assert abs(ld - float(z["logdet32"])) <= 2e-3 * abs(float(z["logdet32"]))
        assert relerr(xi, z["xi32"]) < 1e-2


def test_stateless_dense_only(gpu):
    """n_points = n0: no refined point; the logdet is 0 (csrc/graphgp_capi.cu:36-38)."""
    _say("case stateless dense-only")
    prob, rng = _problem(600, 3, 60, 8, np.float32, seed=1)
    p2 = G().GraphGPProblem(prob.coords[:60], np.zeros((0, 8), np.int64), np.array([60]), 60,
                            prob.scale, prob.bins, prob.vals)
    ld, xi = stateless(gpu, p2, rng.standard_normal(60))
    assert ld == 0.0 and xi.size == 0
