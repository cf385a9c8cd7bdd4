"""GPU parity of the point-position gradients (src/grad.jl:160-377, src/dense.jl:185-300,
src/chainrules.jl:84-122) through the C ABI, against the oracle and against central differences
of a continuous-position forward.

Tolerances (L2-relative): 1e-5 in Float32 and 1e-12 in Float64; the measured error of each
comparison is printed. Where the dense layer's K^-1 enters, the library forms it as L^-T L^-1 on
the matrix cores and the oracle by column solves (a different summation order). The refinement
sums each point's terms in double in another order than the oracle's pair loop; the oracle runs
with its double accumulator so that both are compared at the precision of the terms
themselves.
The reference's own GPU-vs-CPU check of these ops uses rtol 1e-3 (test/runtests.jl:143-157).
"""
import sys

import numpy as np
import pytest

from conftest import relerr

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


def _problem(N, D, n0, k, dtype, seed, length=0.4, n_bins=300, r_max=10.0, normal=True):
    rng = np.random.default_rng(seed)
    pts = rng.standard_normal((N, D)) if normal else rng.random((N, D))
    bins, vals = G().rbf_kernel(1.0, length, 1e-4, r_max, n_bins, jitter=1e-3)
    prob = G().build_graph(pts, n0, k, bins.astype(dtype), vals.astype(dtype))
    ref = O().Problem(prob.coords, prob.neighbors, prob.offsets, prob.n0, prob.scale, prob.bins,
                      prob.vals, indices=prob.indices, dtype=dtype, acc64=True)
    return prob, ref, rng


CASES = [  # (N, D, n0, k): the reference's GPU check (test/runtests.jl:143-157) first
    (4000, 3, 80, 10), (3000, 2, 100, 4), (3000, 3, 100, 8), (3000, 4, 120, 8),
    (2500, 3, 100, 16), (2000, 3, 16, 6), (2000, 3, 100, 20)]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("case", CASES, ids=lambda c: f"N{c[0]}_D{c[1]}_n0{c[2]}_k{c[3]}")
def test_point_gradients_vs_oracle(gpu, case, dtype):
    N, D, n0, k = case
    _say(f"case points N={N} D={D} n0={n0} k={k} {np.dtype(dtype).name}")
    prob, ref, rng = _problem(N, D, n0, k, dtype, seed=7 + k + D)
    hp = G().to_backend(prob)
    data = rng.standard_normal(N).astype(dtype)
    dord = data[prob.indices]
    f32 = dtype == np.float32
    t_ref = t_gen = 1e-5 if f32 else 1e-12

    def check(name, a, b, bar):
        e = relerr(a, b)
        _say(f"  {name}: L2-relative error {e:.3e} (bar {bar:.0e})")
        assert e < bar, (name, e)

    g = G().refine_logdet_grad_points(hp)
    ld_o, g_o = ref.refine_logdet_grad_points()
    assert g.shape == (N, D)
    check("refine_logdet_grad_points", g, g_o, t_ref)

    loss, gi = G().refine_inv_loss_grad_points(hp, dord)
    loss_o, gi_o = ref.refine_inv_loss_grad_points(dord)
    assert abs(loss - loss_o) <= t_ref * abs(loss_o)
    check("refine_inv_loss_grad_points", gi, gi_o, t_ref)

    ld, gg = G().generate_logdet_and_grad_points(hp)
    ld_o, gg_o = ref.generate_logdet_grad_points()
    assert abs(ld - ld_o) <= t_ref * abs(ld_o)
    check("generate_logdet_grad_points", gg, gg_o, t_gen)
    assert relerr(G().generate_logdet_grad_points(hp), gg) < t_ref  # atomics: order varies

    loss, gd = G().generate_inv_loss_grad_points(hp, data)
    loss_o, gd_o = ref.generate_inv_loss_grad_points(data)
    assert abs(loss - loss_o) <= t_ref * abs(loss_o)
    check("generate_inv_loss_grad_points", gd, gd_o, t_gen)
    # the refined rows carry no dense term
    assert relerr(gd[n0:], gi[n0:]) < t_ref


def _cov(P, Q, bins, vals):
    d = np.sqrt(np.sum((P[..., :, None, :] - Q[..., None, :, :]) ** 2, axis=-1))
    return np.interp(d, bins, vals)


def test_point_gradients_vs_continuous_finite_differences(gpu):
    """test/test_gradients.jl:78-128 on the GPU: N = 200, n0 = 16, k = 6, Float64."""
    _say("case points FD f64")
    prob, _, _ = _problem(200, 3, 16, 6, np.float64, seed=13, length=0.5, n_bins=400)
    hp = G().to_backend(prob)
    n0, k = prob.n0, prob.K
    idx = np.concatenate([prob.neighbors, (n0 + np.arange(prob.M))[:, None]], axis=1)

    def fwd(X):
        Ld = np.linalg.cholesky(_cov(X[:n0], X[:n0], prob.bins, prob.vals))
        P = X[idx]
        L = np.linalg.cholesky(_cov(P, P, prob.bins, prob.vals))
        return np.sum(np.log(np.diag(Ld))) + np.sum(np.log(L[:, k, k]))

    X = prob.scale * prob.coords.astype(np.float64)
    assert fwd(X) == pytest.approx(G().generate_logdet(hp), rel=1e-10)
    gp = G().generate_logdet_grad_points(hp)
    h = 1e-6
    for p, d in ((2, 0), (11, 1), (n0 + 4, 0), (n0 + 59, 2), (n0 + 149, 1)):
        Xp, Xm = X.copy(), X.copy()
        Xp[p, d] += h
        Xm[p, d] -= h
        assert gp[p, d] == pytest.approx((fwd(Xp) - fwd(Xm)) / (2 * h), rel=2e-3, abs=1e-6)


def test_points_rrules_compose(gpu):
    """test/test_gradients.jl:130-148: the torch rrules return the op gradients, alone and
    summed in one graph."""
    import torch
    from graphgp_hip import autograd as A
    _say("case points rrules")
    prob, _, rng = _problem(3000, 3, 100, 8, np.float64, seed=3)
    hp = G().to_backend(prob)
    data = torch.from_numpy(rng.standard_normal(prob.N)).cuda()
    X = torch.from_numpy(prob.scale * prob.coords.astype(np.float64)).cuda().requires_grad_()
    (gz,) = torch.autograd.grad(A.logdet_of_points(hp, X), X)
    g = G().generate_logdet_grad_points(hp)
    assert relerr(gz.cpu().numpy(), g) < 1e-12
    (gz2,) = torch.autograd.grad(A.inv_quadratic_loss_of_points(hp, X, data), X)
    _, g2 = G().generate_inv_loss_grad_points(hp, data)
    assert relerr(gz2.cpu().numpy(), g2.cpu().numpy()) < 1e-12
    tot = 2.0 * A.logdet_of_points(hp, X) + A.inv_quadratic_loss_of_points(hp, X, data)
    (gz3,) = torch.autograd.grad(tot, X)
    assert relerr(gz3.cpu().numpy(), 2.0 * g + g2.cpu().numpy()) < 1e-12


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_point_gradients_large_invariants(gpu, dtype):
    """200k points, k = 8, n0 = 1024 (too large for the oracle): every pair adds +c and -c, so
    the gradient sums to zero over the points; the refined rows of the generate_* gradient equal
    the refine_* ones."""
    _say(f"case points large {np.dtype(dtype).name}")
    prob, _, rng = _problem(200_000, 3, 1024, 8, dtype, seed=11, length=0.02, n_bins=500,
                            r_max=2.0, normal=False)
    hp = G().to_backend(prob)
    data = rng.standard_normal(prob.N).astype(dtype)
    tol = 1e-4 if dtype == np.float32 else 1e-11
    for g in (G().generate_logdet_grad_points(hp), G().generate_inv_loss_grad_points(hp, data)[1]):
        g = g.astype(np.float64)
        assert np.all(np.isfinite(g))
        assert np.max(np.abs(g.sum(axis=0))) <= tol * np.linalg.norm(g)
    gr = G().refine_logdet_grad_points(hp)
    gg = G().generate_logdet_grad_points(hp)
    n0 = prob.n0
    assert relerr(gg[n0:], gr[n0:]) < (1e-6 if dtype == np.float32 else 1e-14)


def test_point_gradients_reject_anisotropic_table(gpu):
    _say("case points aniso rejected")
    prob, _, _ = _problem(1500, 3, 64, 8, np.float32, seed=5)
    sb = np.linspace(0.0, 8.0, 32)
    zb = np.linspace(0.0, 4.0, 8)
    grid = np.exp(-sb[:, None]) * np.exp(-zb[None, :])
    cov = G().build_anisotropic_covariance(sb, zb, grid, 1.0, jitter=1e-3, dtype=np.float32)
    hp = G().to_backend(G().GraphGPProblem(prob.coords, prob.neighbors, prob.offsets, prob.n0,
                                           prob.scale, indices=prob.indices, cov=cov))
    with pytest.raises(G().GraphGPError):
        G().generate_logdet_grad_points(hp)
