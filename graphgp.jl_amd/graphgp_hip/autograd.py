"""The reference's ChainRules rrules (src/chainrules.jl, src/grad_generate_vals.jl:291-305) as
torch.autograd Functions over the HIP ops:

  generate(prob, xi)                       pullback: generate_grad_xi
  logdet_of_vals(prob, vals)               pullback: generate_logdet_grad_vals * ybar
  inv_quadratic_loss_of_vals(prob, vals, data)  pullback: generate_inv_loss_grad_vals * lbar
  generate_of_vals(prob, vals, xi)         pullback: (generate_grad_vals, generate_grad_xi)
  logdet_of_points(prob, points)           pullback: generate_logdet_grad_points * ybar
  inv_quadratic_loss_of_points(prob, points, data)  pullback: generate_inv_loss_grad_points * lbar

`points` is the (N, D) tensor of continuous positions in tree order (the reference's (D, N)
matrix); the forward values use the lattice coordinates and ignore it (straight-through,
src/chainrules.jl:84-122).

`vals` is a torch tensor (any device); setting it replaces the problem's table, as _set_vals
does. The reference's pullbacks close over the problem their forward ran on (prob2 =
_set_vals(prob, vals), src/chainrules.jl:32-37, src/grad_generate_vals.jl:294-305); here the
handle is shared, so each Function records the table of its forward and puts it back before its
pullback runs if another table was set in between. d/d(data) of the inverse loss is not
provided, as in the reference (@not_implemented).
"""
from __future__ import annotations

import numpy as np
import torch

from . import problem as P


def _set(prob, vals):
    prob.set_vals(vals.detach().cpu().numpy())


def _like(x, ref):
    return torch.as_tensor(x, dtype=ref.dtype, device=ref.device)


class _Generate(torch.autograd.Function):
    @staticmethod
    def forward(ctx, xi, prob):
        ctx.prob = prob
        ctx.table = prob.table_snapshot()
        return P.generate(prob, xi)

    @staticmethod
    def backward(ctx, ybar):
        ctx.prob.use_table(ctx.table)
        return P.generate_grad_xi(ctx.prob, ybar.contiguous()), None


class _LogdetOfVals(torch.autograd.Function):
    @staticmethod
    def forward(ctx, vals, prob):
        _set(prob, vals)
        ld, g = P.generate_logdet_and_grad_vals(prob)
        ctx.save_for_backward(_like(g, vals))
        return torch.tensor(ld, dtype=vals.dtype, device=vals.device)

    @staticmethod
    def backward(ctx, ybar):
        (g,) = ctx.saved_tensors
        return g * ybar, None


class _InvQuadOfVals(torch.autograd.Function):
    @staticmethod
    def forward(ctx, vals, prob, data):
        _set(prob, vals)
        loss, g = P.generate_inv_loss_grad_vals(prob, data)
        ctx.save_for_backward(_like(g, vals))
        return torch.tensor(loss, dtype=vals.dtype, device=vals.device)

    @staticmethod
    def backward(ctx, lbar):
        (g,) = ctx.saved_tensors
        return g * lbar, None, None


class _GenerateOfVals(torch.autograd.Function):
    @staticmethod
    def forward(ctx, vals, xi, prob):
        _set(prob, vals)
        ctx.prob = prob
        ctx.table = prob.table_snapshot()
        ctx.save_for_backward(xi)
        ctx.vals_meta = (vals.dtype, vals.device)
        return P.generate(prob, xi)

    @staticmethod
    def backward(ctx, ybar):
        (xi,) = ctx.saved_tensors
        ctx.prob.use_table(ctx.table)
        yb = ybar.contiguous()
        dvals = P.generate_grad_vals(ctx.prob, xi, yb)
        dxi = P.generate_grad_xi(ctx.prob, yb)
        dt, dev = ctx.vals_meta
        return torch.as_tensor(dvals, dtype=dt, device=dev), dxi, None


class _LogdetOfPoints(torch.autograd.Function):
    @staticmethod
    def forward(ctx, points, prob):
        ld, g = P.generate_logdet_and_grad_points(prob, as_numpy=False)
        ctx.save_for_backward(_like(g, points))
        return torch.tensor(ld, dtype=points.dtype, device=points.device)

    @staticmethod
    def backward(ctx, ybar):
        (g,) = ctx.saved_tensors
        return g * ybar, None


class _InvQuadOfPoints(torch.autograd.Function):
    @staticmethod
    def forward(ctx, points, prob, data):
        loss, g = P.generate_inv_loss_grad_points(prob, data)
        ctx.save_for_backward(_like(g, points))
        return torch.tensor(loss, dtype=points.dtype, device=points.device)

    @staticmethod
    def backward(ctx, lbar):
        (g,) = ctx.saved_tensors
        return g * lbar, None, None


def generate(prob, xi):
    return _Generate.apply(xi, prob)


def logdet_of_points(prob, points):
    return _LogdetOfPoints.apply(points, prob)


def inv_quadratic_loss_of_points(prob, points, data):
    return _InvQuadOfPoints.apply(points, prob, data)


def logdet_of_vals(prob, vals):
    return _LogdetOfVals.apply(vals, prob)


def inv_quadratic_loss_of_vals(prob, vals, data):
    return _InvQuadOfVals.apply(vals, prob, data)


def generate_of_vals(prob, vals, xi):
    return _GenerateOfVals.apply(vals, xi, prob)
