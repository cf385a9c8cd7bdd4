"""Covariance tables and hyperparameter gradients — the host-side input generation of the
reference's src/extras.jl (make_cov_bins :14-17, rbf_kernel :26-38, matern_kernel :59-74,
hyperparam_grad :86-92). Tables are built in float64 and cast to the problem's precision by the
caller, as the reference does (`T.(vals)`).
"""
from __future__ import annotations

import math

import numpy as np


def make_cov_bins(r_min: float, r_max: float, n_bins: int) -> np.ndarray:
    """[0; 10 .^ range(log10 r_min, log10 r_max, n_bins-1)] (src/extras.jl:14-17)."""
    inner = 10.0 ** np.linspace(math.log10(float(r_min)), math.log10(float(r_max)), n_bins - 1)
    return np.concatenate([[0.0], inner])


def rbf_kernel(variance, scale, r_min, r_max, n_bins, jitter=0.0):
    """variance*exp(-(r/scale)^2/2) on make_cov_bins, vals[0] *= 1+jitter (src/extras.jl:26-38).

    variance/scale may be complex (complex-step differentiation in hyperparam_grad)."""
    bins = make_cov_bins(r_min, r_max, n_bins)
    vals = variance * np.exp(-0.5 * (bins / scale) ** 2)
    vals = np.array(vals, dtype=np.result_type(vals, float))
    vals[0] = vals[0] * (1 + jitter)
    return bins, vals


def _matern_coeffs(p: int) -> np.ndarray:
    # exp(loggamma(p+1) + loggamma(p+i+1) - loggamma(i+1) - loggamma(p-i+1) - loggamma(2p+1)),
    # i = 0..p (src/extras.jl:61-63), highest power first as jnp.polyval expects.
    lg = math.lgamma
    return np.array([math.exp(lg(p + 1.0) + lg(p + i + 1.0) - lg(i + 1.0) - lg(p - i + 1.0)
                              - lg(2 * p + 1.0)) for i in range(p + 1)])


def matern_kernel(p: int, variance, cutoff, r_min, r_max, n_bins, jitter=0.0):
    """Matern nu = p + 1/2 on make_cov_bins (src/extras.jl:59-74):
    variance * exp(-x) * polyval(coeffs, 2x) with x = sqrt(2p+1) r / cutoff."""
    bins = make_cov_bins(r_min, r_max, n_bins)
    coeffs = _matern_coeffs(int(p))
    x = math.sqrt(2 * p + 1) * bins / cutoff
    z = 2 * x
    acc = coeffs[0] + 0 * z
    for c in coeffs[1:]:
        acc = acc * z + c
    vals = variance * np.exp(-x) * acc
    vals = np.array(vals, dtype=np.result_type(vals, float))
    vals[0] = vals[0] * (1 + jitter)
    return bins, vals


def hyperparam_grad(grad_cov_vals, make_kernel, hyperparams) -> np.ndarray:
    """J(vals; hyperparams)^T grad_cov_vals (src/extras.jl:86-92).

    The reference takes the Jacobian with ForwardDiff (exact derivatives); here it is taken by
    complex-step differentiation, Im f(x + i h e_k) / h with h = 1e-30, which is exact to
    rounding for the analytic kernels above. make_kernel(*hyperparams) -> (bins, vals)."""
    hp = np.asarray(hyperparams, dtype=np.float64)
    g = np.asarray(grad_cov_vals, dtype=np.float64)
    h = 1e-30
    out = np.zeros(len(hp))
    for k in range(len(hp)):
        x = hp.astype(complex)
        x[k] += 1j * h
        _, vals = make_kernel(*x)
        out[k] = float(np.dot(np.imag(np.asarray(vals)) / h, g))
    return out
