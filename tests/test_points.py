"""Point-position gradients of the oracle (src/grad.jl:160-377, src/dense.jl:185-300), pinned
against central differences of a continuous-position forward written here in numpy — the
reference's own check (test/test_gradients.jl:78-215: the same sizes, tables, points and
tolerances). The forward treats X = scale * coords as free real positions, so it exercises
d cov / d r and d r / d x independently of the oracle's pair loop; a dropped term, a wrong sign
of the pair difference or a missing dense/refinement part fails it.
"""
import numpy as np
import pytest
from scipy.linalg import solve_triangular

import oracle as O


def _problem(seed, N, n0, k, n_bins):
    import graphgp_hip as Gh
    rng = np.random.default_rng(seed)
    pts = rng.standard_normal((N, 3))
    bins, vals = Gh.rbf_kernel(1.0, 0.5, 1e-4, 10.0, n_bins, jitter=1e-3)
    prob = Gh.build_graph(pts, n0, k, bins, vals)
    ref = O.Problem(prob.coords, prob.neighbors, prob.offsets, prob.n0, prob.scale, prob.bins,
                    prob.vals, indices=prob.indices)
    return prob, ref, rng


def _cov(P, Q, bins, vals):
    d = np.sqrt(np.sum((P[..., :, None, :] - Q[..., None, :, :]) ** 2, axis=-1))
    return np.interp(d, bins, vals)   # cov_lookup (pinned against np.interp in test_oracle)


def _refined_factors(X, prob):
    n0, k = prob.n0, prob.neighbors.shape[1]
    M = prob.N - n0
    idx = np.concatenate([prob.neighbors, (n0 + np.arange(M))[:, None]], axis=1)
    P = X[idx]
    return idx, np.linalg.cholesky(_cov(P, P, prob.bins, prob.vals)), k


def _logdet_fwd(X, prob):
    n0 = prob.n0
    Ld = np.linalg.cholesky(_cov(X[:n0], X[:n0], prob.bins, prob.vals))
    _, L, k = _refined_factors(X, prob)
    return np.sum(np.log(np.diag(Ld))) + np.sum(np.log(L[:, k, k]))


def _inv_loss_fwd(X, prob, dord):
    n0 = prob.n0
    Ld = np.linalg.cholesky(_cov(X[:n0], X[:n0], prob.bins, prob.vals))
    xid = solve_triangular(Ld, dord[:n0], lower=True)
    s = 0.5 * np.sum(xid ** 2)
    idx, L, k = _refined_factors(X, prob)
    for m in range(L.shape[0]):
        mv = solve_triangular(L[m, :k, :k].T, L[m, k, :k], lower=False)
        xim = (dord[n0 + m] - mv @ dord[idx[m, :k]]) / L[m, k, k]
        s += 0.5 * xim ** 2
    return s


_FD_POINTS = lambda n0: ((2, 0), (11, 1), (n0 + 4, 0), (n0 + 59, 2), (n0 + 149, 1))


def _fd(f, X, p, d, h=1e-6):
    Xp, Xm = X.copy(), X.copy()
    Xp[p, d] += h
    Xm[p, d] -= h
    return (f(Xp) - f(Xm)) / (2 * h)


def test_logdet_grad_points_vs_continuous_finite_differences():
    prob, ref, _ = _problem(13, 200, 16, 6, 400)
    X = prob.scale * prob.coords.astype(np.float64)
    assert _logdet_fwd(X, prob) == pytest.approx(ref.generate_logdet(), rel=1e-10)
    ld, gp = ref.generate_logdet_grad_points()
    assert gp.shape == (prob.N, 3)
    assert ld == pytest.approx(ref.generate_logdet(), rel=1e-12)
    for p, d in _FD_POINTS(prob.n0):
        fd = _fd(lambda Y: _logdet_fwd(Y, prob), X, p, d)
        assert gp[p, d] == pytest.approx(fd, rel=2e-3, abs=1e-6), (p, d)


def test_inv_loss_grad_points_vs_continuous_finite_differences():
    prob, ref, rng = _problem(21, 220, 16, 6, 300)
    data = rng.standard_normal(prob.N)
    dord = data[prob.indices]
    X = prob.scale * prob.coords.astype(np.float64)
    loss, gp = ref.generate_inv_loss_grad_points(data)
    assert loss == pytest.approx(_inv_loss_fwd(X, prob, dord), rel=1e-10)
    assert loss == pytest.approx(0.5 * np.sum(ref.generate_inv(data) ** 2), rel=1e-10)
    for p, d in _FD_POINTS(prob.n0):
        fd = _fd(lambda Y: _inv_loss_fwd(Y, prob, dord), X, p, d)
        assert gp[p, d] == pytest.approx(fd, rel=2e-3, abs=1e-6), (p, d)


def test_point_gradients_split_and_translation_invariance():
    """generate_* = refine_* + the dense part on the first n0 points only; each pair adds +c and
    -c, so the gradient sums to zero over the points (a rigid shift changes nothing)."""
    prob, ref, rng = _problem(5, 300, 24, 8, 300)
    data = rng.standard_normal(prob.N)
    dord = data[prob.indices]
    _, g = ref.generate_logdet_grad_points()
    _, gr = ref.refine_logdet_grad_points()
    _, gi = ref.generate_inv_loss_grad_points(data)
    _, gir = ref.refine_inv_loss_grad_points(dord)
    n0 = prob.n0
    np.testing.assert_array_equal(g[n0:], gr[n0:])
    np.testing.assert_array_equal(gi[n0:], gir[n0:])
    for a in (g, gr, gi, gir):
        assert np.all(np.isfinite(a))
        assert np.max(np.abs(a.sum(axis=0))) <= 1e-10 * np.max(np.abs(a)) * prob.N


def test_point_gradients_f32_track_f64():
    prob, ref, rng = _problem(6, 300, 24, 8, 300)
    data = rng.standard_normal(prob.N)
    r32 = ref.with_dtype(np.float32)
    for f64, f32 in ((ref.generate_logdet_grad_points(), r32.generate_logdet_grad_points()),
                     (ref.generate_inv_loss_grad_points(data),
                      r32.generate_inv_loss_grad_points(data.astype(np.float32)))):
        err = np.linalg.norm(f32[1] - f64[1]) / np.linalg.norm(f64[1])
        assert err < 1e-3, err


def test_point_gradients_reject_anisotropic_problem():
    prob, ref, _ = _problem(7, 120, 16, 4, 100)
    sb = np.linspace(0.0, 8.0, 32)
    zb = np.linspace(0.0, 4.0, 8)
    grid = np.exp(-sb[:, None]) * np.exp(-zb[None, :])
    an = O.Problem(prob.coords, prob.neighbors, prob.offsets, prob.n0, prob.scale, prob.bins,
                   prob.vals, indices=prob.indices, aniso=(sb, zb, grid, 1.0))
    with pytest.raises(RuntimeError, match="returned 7"):
        an.generate_logdet_grad_points()
