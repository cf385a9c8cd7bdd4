"""GPU tests of the reference's rrules (src/chainrules.jl:31-74, src/grad_generate_vals.jl:291-305)
as torch.autograd Functions over the HIP ops, alone and composed, against the oracle.

Each gradient the autograd graph returns is compared with the oracle's adjoint at 1e-5 (f32) /
1e-12 (f64) L2-relative; the measured error is printed. One case runs two generate_of_vals
forwards with different tables on the same problem and back-propagates through both: each
pullback must use the table of its own forward, as the reference's closures over prob2 do.
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


def A():
    import graphgp_hip.autograd as ag
    return ag


def O():
    import oracle
    return oracle


def _check(name, got, want, bar):
    e = relerr(np.asarray(got), np.asarray(want))
    _say(f"  {name}: L2-relative error {e:.3e} (bar {bar:.0e})")
    assert e < bar, (name, e)


def _setup(dtype, N=3000, D=3, n0=120, k=8, seed=5):
    rng = np.random.default_rng(seed)
    pts = rng.random((N, D))
    bins, vals = G().rbf_kernel(1.0, 0.1, 1e-4, 2.0, 400, jitter=1e-5)
    prob = G().build_graph(pts, n0, k, bins.astype(dtype), vals.astype(dtype))
    hp = G().to_backend(prob)
    return prob, hp, rng


def _oracle(prob, vals, dtype):
    return O().Problem(prob.coords, prob.neighbors, prob.offsets, prob.n0, prob.scale, prob.bins,
                       np.asarray(vals, dtype), indices=prob.indices, dtype=dtype)


DTYPES = [np.float32, np.float64]


def _bar(dtype):
    return 1e-5 if dtype == np.float32 else 1e-12


@pytest.mark.parametrize("dtype", DTYPES)
def test_generate_rrule(gpu, dtype):
    """rrule(generate): x̄ = generate_grad_xi(prob, ȳ) (src/chainrules.jl:51-58)."""
    torch = gpu
    _say(f"case rrule generate {np.dtype(dtype).name}")
    prob, hp, rng = _setup(dtype)
    ref = _oracle(prob, prob.vals, dtype)
    xi = torch.tensor(rng.standard_normal(prob.N).astype(dtype), device="cuda", requires_grad=True)
    w = rng.standard_normal(prob.N).astype(dtype)
    y = A().generate(hp, xi)
    _check("generate", y.detach().cpu().numpy(), ref.generate(xi.detach().cpu().numpy()), _bar(dtype))
    (y * torch.from_numpy(w).cuda()).sum().backward()
    _check("d/dxi", xi.grad.cpu().numpy(), ref.generate_grad_xi(w), _bar(dtype))


@pytest.mark.parametrize("dtype", DTYPES)
def test_logdet_and_inverse_loss_of_vals(gpu, dtype):
    """logdet_of_vals and inv_quadratic_loss_of_vals alone, then their sum (the marginal
    likelihood's two terms, src/chainrules.jl:1-12) through a hyperparameter map
    vals = variance * base, checked against the oracle's d/dvals by the chain rule."""
    torch = gpu
    _say(f"case rrule logdet/inv-loss of vals {np.dtype(dtype).name}")
    prob, hp, rng = _setup(dtype)
    data = rng.standard_normal(prob.N).astype(dtype)
    base = prob.vals.astype(np.float64)
    var = 1.3
    vals_np = (var * base).astype(dtype)
    ref = _oracle(prob, vals_np, dtype)
    ld_o, gl_o = ref.generate_logdet_grad_vals()
    loss_o, gi_o = ref.generate_inv_loss_grad_vals(data)

    v1 = torch.tensor(vals_np, requires_grad=True)
    ld = A().logdet_of_vals(hp, v1)
    ld.backward()
    ldv = float(ld.detach())
    _say(f"  logdet_of_vals: relative error {abs(ldv - ld_o) / abs(ld_o):.3e}")
    assert abs(ldv - ld_o) <= _bar(dtype) * abs(ld_o)
    _check("d logdet / d vals", v1.grad.numpy(), gl_o, _bar(dtype))

    v2 = torch.tensor(vals_np, requires_grad=True)
    loss = A().inv_quadratic_loss_of_vals(hp, v2, data)
    loss.backward()
    assert abs(float(loss.detach()) - loss_o) <= _bar(dtype) * abs(loss_o)
    _check("d inv-loss / d vals", v2.grad.numpy(), gi_o, _bar(dtype))

    # composed: theta = variance -> vals -> logdet + inverse loss
    th = torch.tensor(var, dtype=torch.float64, requires_grad=True)
    vals_t = (th * torch.from_numpy(base)).to(v1.dtype)
    total = A().logdet_of_vals(hp, vals_t) + A().inv_quadratic_loss_of_vals(hp, vals_t, data)
    total.backward()
    gl64, gi64 = gl_o.astype(np.float64), gi_o.astype(np.float64)
    want = float(np.sum(base * (gl64 + gi64)))
    # relative to the size of the summed terms: the two terms' d/dvals partly cancel
    e = abs(float(th.grad) - want) / float(np.sum(np.abs(base) * (np.abs(gl64) + np.abs(gi64))))
    _say(f"  d(logdet + inv-loss)/d variance: relative error {e:.3e}")
    assert e < (1e-5 if dtype == np.float32 else 1e-12)


@pytest.mark.parametrize("dtype", DTYPES)
def test_generate_of_vals_two_tables(gpu, dtype):
    """generate_of_vals (src/grad_generate_vals.jl:291-305) with two different tables in one
    graph: d/dvals of each call and the summed d/dxi match the oracle run on each table."""
    torch = gpu
    _say(f"case rrule generate_of_vals {np.dtype(dtype).name}")
    prob, hp, rng = _setup(dtype)
    vals1 = prob.vals.copy()
    vals2 = (0.7 * prob.vals.astype(np.float64)).astype(dtype)
    vals2[0] = vals1[0]  # keep the jittered diagonal: a table of the same family
    ref1, ref2 = _oracle(prob, vals1, dtype), _oracle(prob, vals2, dtype)
    xi_np = rng.standard_normal(prob.N).astype(dtype)
    w1 = rng.standard_normal(prob.N).astype(dtype)
    w2 = rng.standard_normal(prob.N).astype(dtype)
    xi = torch.tensor(xi_np, device="cuda", requires_grad=True)
    t1 = torch.tensor(vals1, requires_grad=True)
    t2 = torch.tensor(vals2, requires_grad=True)
    y1 = A().generate_of_vals(hp, t1, xi)
    y2 = A().generate_of_vals(hp, t2, xi)
    _check("generate_of_vals (table 1)", y1.detach().cpu().numpy(), ref1.generate(xi_np), _bar(dtype))
    _check("generate_of_vals (table 2)", y2.detach().cpu().numpy(), ref2.generate(xi_np), _bar(dtype))
    loss = (y1 * torch.from_numpy(w1).cuda()).sum() + (y2 * torch.from_numpy(w2).cuda()).sum()
    loss.backward()
    _check("d/dvals (table 1)", t1.grad.numpy(), ref1.generate_grad_vals(xi_np, w1), _bar(dtype))
    _check("d/dvals (table 2)", t2.grad.numpy(), ref2.generate_grad_vals(xi_np, w2), _bar(dtype))
    dxi = ref1.generate_grad_xi(w1).astype(np.float64) + ref2.generate_grad_xi(w2).astype(np.float64)
    _check("d/dxi (both calls)", xi.grad.cpu().numpy(), dxi, _bar(dtype))
    # the generate rrule after a table change also uses its own forward's table
    hp.set_vals(vals1)
    xj = torch.tensor(xi_np, device="cuda", requires_grad=True)
    y = A().generate(hp, xj)
    hp.set_vals(vals2)
    (y * torch.from_numpy(w1).cuda()).sum().backward()
    _check("generate rrule after set_vals", xj.grad.cpu().numpy(), ref1.generate_grad_xi(w1), _bar(dtype))
