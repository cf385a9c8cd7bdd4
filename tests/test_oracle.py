"""Pins the oracle (CPU restatement of the reference, oracle/graphgp_oracle.cpp) before it is
trusted as the parity checker: against the reference's golden fixtures and against what the
mathematics fixes (numpy.interp, LAPACK Cholesky, finite differences, adjoint identities, the
dense Vecchia matrix on tiny problems). Each check is chosen so that a dropped term, a sign or
index error or a transposed operand in the restatement fails it.
"""
import numpy as np
import pytest

import oracle as O
from conftest import load_fixture, relerr


def fixture(name, dtype=np.float64):
    z = load_fixture(name)
    s = "64" if dtype == np.float64 else "32"
    bins = z["cov_bins" + s] if "cov_bins" + s in z.files else z["cov_bins64"].astype(dtype)
    vals = z["cov_vals" + s] if "cov_vals" + s in z.files else z["cov_vals64"].astype(dtype)
    idx = z["indices"] if "indices" in z.files else None
    return O.Problem(z["coords"], z["neighbors"], z["offsets"], int(z["n0"]), float(z["scale"]),
                     bins, vals, indices=idx, dtype=dtype), z


# ---- primitives (src/interp.jl, src/linalg.jl) --------------------------------------------------
def test_cov_lookup_matches_numpy_interp_and_edges():
    z = load_fixture("small")
    bins, vals = z["cov_bins64"], z["cov_vals64"]
    rng = np.random.default_rng(0)
    rs = np.concatenate([rng.uniform(0, bins[-1] * 1.2, 500), bins[:50], [0.0, bins[-1]]])
    got = np.array([O.cov_lookup(r, bins, vals) for r in rs])
    np.testing.assert_allclose(got, np.interp(rs, bins, vals), rtol=1e-12, atol=1e-15)
    # exact hits return the tabulated value; clamps at both ends (test/test_interp.jl:7-18)
    for i in (0, 1, 17, len(bins) - 1):
        assert O.cov_lookup(bins[i], bins, vals) == pytest.approx(vals[i], rel=1e-15)
    assert O.cov_lookup(bins[-1] * 3, bins, vals) == vals[-1]


def test_cov_lookup_weights_reconstruct_value():
    z = load_fixture("small")
    bins, vals = z["cov_bins64"], z["cov_vals64"]
    for r in np.random.default_rng(1).uniform(0, bins[-1] * 1.1, 200):
        lo, wlo, whi = O.cov_lookup_weights(r, bins)
        assert wlo * vals[lo] + whi * vals[lo + 1] == pytest.approx(np.interp(r, bins, vals),
                                                                     rel=1e-10, abs=1e-14)
        if 0 < r < bins[-1]:
            assert bins[lo] <= r < bins[lo + 1]


@pytest.mark.parametrize("n", [2, 5, 11])
def test_chol_lower_and_mean_vec_vs_lapack(n):
    rng = np.random.default_rng(n)
    X = rng.standard_normal((n, 2 * n))
    A = X @ X.T + 0.1 * np.eye(n)
    L = O.chol_lower(A)
    np.testing.assert_allclose(L, np.linalg.cholesky(A), rtol=1e-10, atol=1e-12)
    # mean_vec solves L[:K,:K]^T x = L[K,:K]
    x = O.mean_vec_solve(L)
    K = n - 1
    np.testing.assert_allclose(L[:K, :K].T @ x, L[K, :K], rtol=1e-10, atol=1e-12)


def test_chol_lower_clamps_indefinite_block():
    A = np.array([[1.0, 1.0, 0.2], [1.0, 1.0, 0.3], [0.2, 0.3, 1.0]])  # rank deficient
    L = O.chol_lower(A)
    assert np.all(np.isfinite(L))
    assert L[1, 1] == pytest.approx(np.sqrt(np.finfo(float).eps * 1.0))
    assert L[2, 1] == 0.0  # the degenerate column is zeroed (src/linalg.jl:59-68)
    x = O.mean_vec_solve(L)
    assert x[1] == 0.0      # zero weight for the degenerate neighbour (src/linalg.jl:96-99)


@pytest.mark.parametrize("dyn", [False, True])
def test_chol_pullback_vs_finite_differences_and_matrix_adjoint(dyn):
    n = 6
    rng = np.random.default_rng(3)
    X = rng.standard_normal((n, 2 * n))
    A = X @ X.T + 0.5 * np.eye(n)
    L = np.linalg.cholesky(A)
    Lbar = np.tril(rng.standard_normal((n, n)))
    Abar = O.chol_pullback(Lbar, L, dyn=dyn)

    def f(lower):
        S = np.tril(lower) + np.tril(lower, -1).T
        return float(np.sum(Lbar * np.linalg.cholesky(S)))

    h = 1e-6
    for i in range(n):
        for j in range(i + 1):
            E = np.zeros((n, n))
            E[i, j] = h
            fd = (f(A + E) - f(A - E)) / (2 * h)
            assert Abar[i, j] == pytest.approx(fd, rel=1e-5, abs=1e-7)
    # closed form: S = L^-T Phi(L^T Lbar) L^-1, Abar_ij = S_ij + S_ji (i>j), Abar_jj = S_jj
    P = np.tril(L.T @ Lbar)
    P[np.diag_indices(n)] *= 0.5
    Li = np.linalg.inv(L)
    S = Li.T @ P @ Li
    closed = np.tril(S + S.T)
    closed[np.diag_indices(n)] = np.diag(S)
    np.testing.assert_allclose(Abar, closed, rtol=1e-9, atol=1e-12)


# ---- refine ops vs the JAX fixtures (test/test_refine.jl) ----------------------------------------
@pytest.mark.parametrize("name", ["small", "medium"])
def test_refine_ops_f64_vs_fixture(name):
    p, z = fixture(name)
    assert p.refine_logdet_terms().sum() == pytest.approx(float(z["logdet64"]), rel=1e-12)
    assert relerr(p.refine_inv(z["values64"]), z["xi64"]) < 1e-12
    assert relerr(p.refine(z["initial_values64"], z["xi_ref64"]), z["refine_values64"]) < 1e-12


@pytest.mark.parametrize("name", ["small", "medium"])
def test_refine_ops_f32_vs_fixture(name):
    p, z = fixture(name, np.float32)
    ld = float(p.refine_logdet_terms().astype(np.float64).sum())
    assert ld == pytest.approx(float(z["logdet32"]), rel=2e-3)
    assert relerr(p.refine_inv(z["values32"]), z["xi32"]) < 1e-3
    assert relerr(p.refine(z["initial_values32"], z["xi_ref32"]), z["refine_values32"]) < 1e-3


def test_generate_parity_fixture():
    """Full generate / generate_inv with the dense layer and a non-identity permutation
    (test/python_parity_generate.jl: pass at <= 1e-12)."""
    p, z = fixture("generate_parity")
    f = p.generate(z["xi"])
    assert relerr(f, z["generate_field"]) < 1e-12
    assert relerr(p.generate_inv(z["values"]), z["generate_inv_xi"]) < 1e-12
    assert relerr(p.generate_inv(f), z["xi"]) < 1e-12


def test_gradients_vs_fixture():
    """test/test_gradients.jl:1-26: d_vals of logdet (rtol 1e-5 on nonzero bins) and of the
    inverse loss (loss rtol 1e-6, gradient rtol 1e-4)."""
    p, z = fixture("small")
    ld, g = p.refine_logdet_grad_vals()
    assert ld == pytest.approx(float(z["logdet64"]), rel=1e-12)
    nz = z["grad_logdet_vals64"] != 0
    np.testing.assert_allclose(g[nz], z["grad_logdet_vals64"][nz], rtol=1e-5, atol=1e-8)
    assert np.all(g[~nz] == 0)
    loss, gi = p.refine_inv_loss_grad_vals(z["values64"])
    assert loss == pytest.approx(float(z["inv_loss64"]), rel=1e-6)
    nz = z["grad_inv_loss_vals64"] != 0
    np.testing.assert_allclose(gi[nz], z["grad_inv_loss_vals64"][nz], rtol=1e-4, atol=1e-7)


# ---- tiny dense problems: the whole map G built explicitly ---------------------------------------
def tiny_problem(seed=0, N=120, n0=20, k=4, scale_len=0.4):
    import graphgp_hip as Gh
    rng = np.random.default_rng(seed)
    pts = rng.standard_normal((N, 3))
    bins, vals = Gh.rbf_kernel(1.0, scale_len, 1e-4, 10.0, 200, jitter=1e-3)
    prob = Gh.build_graph(pts, n0, k, bins, vals)
    return O.Problem(prob.coords, prob.neighbors, prob.offsets, prob.n0, prob.scale, prob.bins,
                     prob.vals, indices=prob.indices)


def test_generate_is_linear_and_grad_xi_is_its_transpose():
    p = tiny_problem()
    N = p.N
    Gm = np.stack([p.generate(np.eye(N)[i]) for i in range(N)], axis=1)
    rng = np.random.default_rng(5)
    xi = rng.standard_normal(N)
    vb = rng.standard_normal(N)
    np.testing.assert_allclose(p.generate(xi), Gm @ xi, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(p.generate_grad_xi(vb), Gm.T @ vb, rtol=1e-11, atol=1e-12)
    # generate_inv is the inverse map
    np.testing.assert_allclose(p.generate_inv(Gm @ xi), xi, rtol=1e-9, atol=1e-10)


def test_logdet_equals_half_logdet_of_vecchia_covariance():
    """generate_logdet = 0.5 log det(G G^T) = log|det G| for the explicit map G."""
    p = tiny_problem(seed=1)
    N = p.N
    Gm = np.stack([p.generate(np.eye(N)[i]) for i in range(N)], axis=1)
    sign, ld = np.linalg.slogdet(Gm)
    assert p.generate_logdet() == pytest.approx(ld, rel=1e-10)


def test_generate_grad_vals_vs_finite_differences():
    p = tiny_problem(seed=2)
    rng = np.random.default_rng(7)
    xi = rng.standard_normal(p.N)
    w = rng.standard_normal(p.N)
    dv = p.generate_grad_vals(xi, w)
    vals = p.vals.copy()
    h = 1e-6
    for i in (3, 10, 40, 80, 120):
        e = np.zeros_like(vals)
        e[i] = h
        fd = (np.dot(w, p.with_vals(vals + e).generate(xi)) -
              np.dot(w, p.with_vals(vals - e).generate(xi))) / (2 * h)
        assert dv[i] == pytest.approx(fd, rel=1e-5, abs=1e-8)


def test_logdet_and_inv_loss_grads_vs_finite_differences():
    p = tiny_problem(seed=3)
    data = p.generate(np.random.default_rng(8).standard_normal(p.N))
    ld, g = p.generate_logdet_grad_vals()
    loss, gi = p.generate_inv_loss_grad_vals(data)
    assert ld == pytest.approx(p.generate_logdet(), rel=1e-12)
    assert loss == pytest.approx(0.5 * np.sum(p.generate_inv(data) ** 2), rel=1e-10)
    vals = p.vals.copy()
    h = 1e-6
    for i in (2, 15, 60, 100):
        e = np.zeros_like(vals)
        e[i] = h
        pp, pm = p.with_vals(vals + e), p.with_vals(vals - e)
        fd = (pp.generate_logdet() - pm.generate_logdet()) / (2 * h)
        assert g[i] == pytest.approx(fd, rel=1e-5, abs=1e-8)
        fdi = (0.5 * np.sum(pp.generate_inv(data) ** 2) - 0.5 * np.sum(pm.generate_inv(data) ** 2)) / (2 * h)
        assert gi[i] == pytest.approx(fdi, rel=1e-5, abs=1e-6)


def test_dense_factor_matches_lapack_and_jitter_retry():
    p = tiny_problem(seed=4)
    L = p.dense_factor()
    from numpy.linalg import cholesky
    import graphgp_hip  # noqa: F401  (tables only)
    # rebuild K from the oracle's own factor and compare with numpy's factor of it
    K = L @ L.T
    np.testing.assert_allclose(cholesky(K), L, rtol=1e-9, atol=1e-12)
    # a duplicated dense point makes K singular: the retry adds jitter and still factors
    c = p.coords.copy()
    c[1] = c[0]
    q = O.Problem(c, p.neighbors, p.offsets, p.n0, p.scale, p.bins, p.vals.copy(), p.indices)
    q.vals[0] = q.vals[0] / (1 + 1e-3)   # remove the nugget
    Lq = q.dense_factor()
    assert np.all(np.isfinite(Lq)) and np.all(np.diag(Lq) > 0)


def test_f32_oracle_tracks_f64():
    p, z = fixture("small")
    p32, _ = fixture("small", np.float32)
    xi = np.random.default_rng(0).standard_normal(p.N)
    assert relerr(p32.generate(xi.astype(np.float32)), p.generate(xi)) < 1e-3


def test_double_histogram_mode_only_changes_the_summation():
    """acc64 sums the d/dvals histograms in double. In Float64 it must agree with the default to
    rounding; in Float32 it must sit closer to the Float64 answer than the Float32 sums do."""
    p, z = fixture("small")
    p64 = O.Problem(p.coords, p.neighbors, p.offsets, p.n0, p.scale, p.bins, p.vals,
                    indices=p.indices, acc64=True)
    _, g = p.refine_logdet_grad_vals()
    _, g64 = p64.refine_logdet_grad_vals()
    assert relerr(g64, g) < 1e-13
    xi = np.random.default_rng(1).standard_normal(p.N)
    vb = np.random.default_rng(2).standard_normal(p.N)
    assert relerr(p64.generate_grad_vals(xi, vb), p.generate_grad_vals(xi, vb)) < 1e-13
    p32, _ = fixture("small", np.float32)
    q32 = p32.with_vals(p32.vals)
    q32 = O.Problem(q32.coords, q32.neighbors, q32.offsets, q32.n0, q32.scale, q32.bins, q32.vals,
                    indices=q32.indices, dtype=np.float32, acc64=True)
    _, g32 = p32.refine_logdet_grad_vals()
    _, g32d = q32.refine_logdet_grad_vals()
    assert relerr(g32d, g) <= relerr(g32, g) * 1.01 + 1e-7


def test_double_mode_dense_cotangents():
    """acc64 also evaluates the dense-layer cotangents (the Cholesky adjoint of
    generate_grad_vals, K^-1 of the logdet gradient, alpha of the inverse loss) in double from
    the factor. In Float64 that is the default's arithmetic: the two modes agree to rounding. In
    Float32 the double evaluation must sit at least as close to the Float64 answer as the
    Float32 loops do (it removes their rounding, not the factor's)."""
    p, z = fixture("generate_parity")
    q = O.Problem(p.coords, p.neighbors, p.offsets, p.n0, p.scale, p.bins, p.vals,
                  indices=p.indices, acc64=True)
    rng = np.random.default_rng(3)
    xi, vb, d = (rng.standard_normal(p.N) for _ in range(3))
    assert relerr(q.generate_grad_vals(xi, vb), p.generate_grad_vals(xi, vb)) < 1e-13
    assert relerr(q.generate_logdet_grad_vals()[1], p.generate_logdet_grad_vals()[1]) < 1e-13
    l64, g64 = p.generate_inv_loss_grad_vals(d)
    lq, gq = q.generate_inv_loss_grad_vals(d)
    assert relerr(gq, g64) < 1e-13 and abs(lq - l64) <= 1e-13 * abs(l64)
    p32 = p.with_dtype(np.float32)
    q32 = O.Problem(p32.coords, p32.neighbors, p32.offsets, p32.n0, p32.scale, p32.bins,
                    p32.vals, indices=p32.indices, dtype=np.float32, acc64=True)
    x32, v32, d32 = xi.astype(np.float32), vb.astype(np.float32), d.astype(np.float32)
    want = p.generate_grad_vals(x32.astype(float), v32.astype(float))
    assert relerr(q32.generate_grad_vals(x32, v32), want) <= \
        relerr(p32.generate_grad_vals(x32, v32), want) * 1.05 + 1e-7
    want = p.generate_logdet_grad_vals()[1]
    assert relerr(q32.generate_logdet_grad_vals()[1], want) <= \
        relerr(p32.generate_logdet_grad_vals()[1], want) * 1.05 + 1e-7
    want = p.generate_inv_loss_grad_vals(d32.astype(float))[1]
    assert relerr(q32.generate_inv_loss_grad_vals(d32)[1], want) <= \
        relerr(p32.generate_inv_loss_grad_vals(d32)[1], want) * 1.05 + 1e-7
