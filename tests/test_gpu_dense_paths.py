"""The two schedules of the dense first-layer Cholesky (the persistent walker launch and the
blocked path of panel steps plus trailing updates, which large blocks take) against the oracle's
column-by-column factor.

Both schedules give every entry of the factor the unblocked left-looking fma chain in the same
order, so the dense part of generate (L xi, a product whose chain is also the oracle's) must
have the oracle's bits in Float32 and Float64, whichever schedule ran. GGP_POTRF_BLOCKED forces
the schedule, GGP_SYRK_BLOCK the blocked path's trailing-update block edge (64 or 128) and
GGP_POTRF_SUPER its super-panel width (4, 8 or 16 tile columns), all read at every call.
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


def _problem(N, n0, dtype, seed):
    rng = np.random.default_rng(seed)
    pts = rng.random((N, 3))
    bins, vals = G().rbf_kernel(1.0, 0.2, 1e-4, 2.0, 400, jitter=1e-4)
    prob = G().build_graph(pts, n0, 8, bins.astype(dtype), vals.astype(dtype))
    ref = O().Problem(prob.coords, prob.neighbors, prob.offsets, prob.n0, prob.scale, prob.bins,
                      prob.vals, indices=prob.indices, dtype=dtype)
    return prob, ref, rng


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("n0", [300, 1000, 1500])
def test_blocked_and_walker_factor_bit_exact(gpu, monkeypatch, n0, dtype):
    _say(f"case dense schedules n0={n0} {np.dtype(dtype).name}")
    prob, ref, rng = _problem(n0 + 500, n0, dtype, seed=n0)
    hp = G().to_backend(prob)
    xi = rng.standard_normal(prob.N).astype(dtype)
    want = ref.generate(xi)
    ld_want = ref.generate_logdet()
    out = {}
    for mode, blk, sup in (("0", "64", "4"), ("1", "64", "4"), ("1", "128", "4"),
                           ("1", "64", "8"), ("1", "128", "16")):
        monkeypatch.setenv("GGP_POTRF_BLOCKED", mode)
        monkeypatch.setenv("GGP_SYRK_BLOCK", blk)
        monkeypatch.setenv("GGP_POTRF_SUPER", sup)
        f = G().generate(hp, xi)
        ld = G().generate_logdet(hp)
        _say(f"  blocked={mode} block={blk} super={sup}: generate relerr {relerr(f, want):.3e}, "
             f"logdet {abs(ld - ld_want) / abs(ld_want):.3e}")
        np.testing.assert_array_equal(f, want)
        assert abs(ld - ld_want) <= (1e-12 if dtype == np.float64 else 1e-5) * abs(ld_want)
        out[mode + blk + sup] = f
    for key in ("1644", "11284", "1648", "112816"):
        np.testing.assert_array_equal(out["0644"], out[key])


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_trailing_update_blocks_agree_at_4160(gpu, monkeypatch, dtype):
    """At 4160 dense points (the blocked schedule by default) both trailing-update block edges
    and both super-panel widths give the same bits, the oracle's (the oracle's factor takes a few seconds at this
    size, so it is run once)."""
    _say(f"case trailing-update blocks n0=4160 {np.dtype(dtype).name}")
    prob, ref, rng = _problem(4800, 4160, dtype, seed=4160)
    hp = G().to_backend(prob)
    xi = rng.standard_normal(prob.N).astype(dtype)
    monkeypatch.delenv("GGP_POTRF_BLOCKED", raising=False)
    out = {}
    for blk, sup in (("64", "4"), ("128", "4"), ("128", "8"), ("64", "16")):
        monkeypatch.setenv("GGP_SYRK_BLOCK", blk)
        monkeypatch.setenv("GGP_POTRF_SUPER", sup)
        out[blk] = out[blk + sup] = G().generate(hp, xi)
    np.testing.assert_array_equal(out["644"], out["1284"])
    np.testing.assert_array_equal(out["644"], out["1288"])
    np.testing.assert_array_equal(out["644"], out["6416"])
    want = ref.generate(xi)
    _say(f"  generate relerr vs oracle {relerr(out['64'], want):.3e}")
    np.testing.assert_array_equal(out["64"], want)


def test_blocked_factor_not_positive_definite_retry(gpu, monkeypatch):
    """A covariance without jitter on coincident points fails the first factorization; the
    blocked schedule reports the pivot like the walker, and the jitter retry succeeds."""
    _say("case dense blocked retry")
    rng = np.random.default_rng(5)
    bins, vals = G().rbf_kernel(1.0, 0.2, 1e-4, 2.0, 400, jitter=0.0)
    base = G().build_graph(rng.random((900, 3)), 600, 8, bins, vals)
    coords = base.coords.copy()
    coords[5] = coords[3]
    coords[407] = coords[3]
    prob = G().GraphGPProblem(coords, base.neighbors, base.offsets, base.n0, base.scale,
                              base.bins, base.vals, indices=base.indices)
    hp = G().to_backend(prob)
    xi = rng.standard_normal(prob.N)
    res = {}
    for mode in ("0", "1"):
        monkeypatch.setenv("GGP_POTRF_BLOCKED", mode)
        res[mode] = G().generate(hp, xi)
        assert np.all(np.isfinite(res[mode]))
    np.testing.assert_array_equal(res["0"], res["1"])


def test_every_op_on_the_blocked_schedule(gpu, monkeypatch):
    """Every op that factors the dense block gives the walker schedule's results when the
    blocked schedule runs instead: the same factor bits, so equal fields and solves, and
    gradients equal up to the order of their f64 sums."""
    _say("case every op on the blocked schedule")
    prob, ref, rng = _problem(1500, 600, np.float64, seed=21)
    hp = G().to_backend(prob)
    xi = rng.standard_normal(prob.N)
    vbar = rng.standard_normal(prob.N)
    data = rng.standard_normal(prob.N)
    ops = {
        "generate": lambda: G().generate(hp, xi),
        "generate_inv": lambda: G().generate_inv(hp, data),
        "generate_logdet": lambda: np.array([G().generate_logdet(hp)]),
        "generate_grad_xi": lambda: G().generate_grad_xi(hp, vbar),
        "generate_grad_vals": lambda: G().generate_grad_vals(hp, xi, vbar),
        "generate_logdet_grad_vals": lambda: G().generate_logdet_grad_vals(hp),
        "generate_inv_loss_grad_vals": lambda: G().generate_inv_loss_grad_vals(hp, data),
        "generate_logdet_grad_points": lambda: G().generate_logdet_grad_points(hp),
    }
    def flat(r):
        parts = r if isinstance(r, (tuple, list)) else (r,)
        return np.concatenate([np.ravel(np.asarray(x, dtype=np.float64)) for x in parts])

    res = {}
    for mode in ("0", "1"):
        monkeypatch.setenv("GGP_POTRF_BLOCKED", mode)
        res[mode] = {k: flat(f()) for k, f in ops.items()}
    for k in ops:
        a, b = res["0"][k], res["1"][k]
        err = relerr(b, a)
        _say(f"  {k}: blocked vs walker relerr {err:.3e}")
        if k in ("generate", "generate_inv", "generate_grad_xi"):
            np.testing.assert_array_equal(a, b)
        else:
            assert err < 1e-12, k
