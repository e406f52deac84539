"""RMSNorm in one HIP kernel each way.

Drop-in for ``core/normalization.py`` (``RMSNorm(hidden_size, eps=1e-6)``, used
by core/transformer_layer.py:77,83 and core/models/gpt.py:22).  The reference's
forward is five eager passes over the activations (fp32 upcast, square, mean,
scale, downcast, weight multiply) and its autograd backward saves the fp32
copies.  Here:

* forward: one read of x, one write of y, plus the fp32 ``rstd`` per row;
  ``y = round_x(x * rstd) * weight`` with the same intermediate rounding to x's
  dtype as the reference (normalization.py:23) and the product in the promoted
  dtype (:24);
* backward: one read of x and dy, one write of dx, and a deterministic
  two-level reduction for the weight gradient.

The weight may have x's dtype (the model's bf16 parameters, once the optimizer
has moved them into its flat buffer) or fp32 (as created); any other pairing
is promoted the way torch promotes ``x.to(dtype) * weight``.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import _lib


def _rows_view(t: torch.Tensor) -> torch.Tensor:
    try:
        _lib._rows(t)
        return t
    except ValueError:
        return t.contiguous()


def _grad_target(w: torch.Tensor, weight_dtype) -> torch.Tensor | None:
    """The weight's existing .grad, when the backward may add its weight
    gradient there itself (as autograd's accumulation would, same rounding): w
    is the weight (not a converted copy), its gradient has w's dtype, shape and
    a dense layout, and no double backward is being recorded.  None otherwise."""
    if not w.is_leaf or torch.is_grad_enabled():
        return None
    g = w.grad
    if g is None or g.dtype != w.dtype or w.dtype != weight_dtype or g.shape != w.shape \
            or not g.is_contiguous():
        return None
    return g


class FusedRMSNorm(torch.autograd.Function):
    """y = round_x(x * rsqrt(mean(x^2, -1) + eps)) * weight.  With `grad_into`,
    the backward adds the weight gradient into the weight's existing .grad
    (mi_rmsnorm_bwd_acc) and returns none for it, as the model harness's
    projections do with their GEMMs; gradient hooks on the weight then see no
    gradient, so the drop-in default leaves it to autograd."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, weight: torch.Tensor, eps: float, grad_into: bool = False):
        if weight.dim() != 1 or x.shape[-1] != weight.shape[0]:
            raise ValueError(f"weight {tuple(weight.shape)} does not match the last dim of x "
                             f"{tuple(x.shape)}")
        _lib._require_gpu(x, weight)
        w = weight
        if w.dtype != x.dtype and w.dtype != torch.float32:
            w = w.float()  # x.to(dtype) * weight promotes both to fp32
        if x.dtype == torch.float32 and w.dtype != torch.float32:
            w = w.float()
        xr = _rows_view(x)
        w = w.contiguous()
        y = torch.empty(x.shape, dtype=w.dtype if w.dtype == torch.float32 else x.dtype,
                        device=x.device)
        rstd = torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device)
        _lib.rmsnorm_fwd(xr, w, eps, y, rstd)
        ctx.save_for_backward(xr, w, rstd)
        ctx.weight_dtype = weight.dtype
        ctx.grad_into = grad_into
        return y

    @staticmethod
    def backward(ctx, dy):
        xr, w, rstd = ctx.saved_tensors
        dy = _rows_view(dy)
        rows = rstd.numel()
        dx = torch.empty(xr.shape, dtype=xr.dtype, device=xr.device)
        ws = torch.empty(_lib.rmsnorm_workspace(rows, xr.shape[-1]), dtype=torch.float32,
                         device=xr.device)
        g = _grad_target(w, ctx.weight_dtype) if ctx.grad_into else None
        if g is not None:
            _lib.rmsnorm_bwd(xr, w, rstd, dy, dx, g, ws, accumulate=True)
            return dx, None, None, None
        dw = torch.empty(w.shape, dtype=w.dtype, device=w.device)
        _lib.rmsnorm_bwd(xr, w, rstd, dy, dx, dw, ws)
        return dx, dw.to(ctx.weight_dtype), None, None


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6,
             grad_into: bool = False) -> torch.Tensor:
    return FusedRMSNorm.apply(x, weight, eps, grad_into)


def _norm_weight(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """The weight in the dtype the kernels take for x: x's own or fp32 (any
    other pairing promotes both to fp32, as ``x.to(dtype) * weight`` does)."""
    w = weight
    if w.dtype != x.dtype and w.dtype != torch.float32:
        w = w.float()
    if x.dtype == torch.float32 and w.dtype != torch.float32:
        w = w.float()
    return w.contiguous()


class FusedAddRMSNorm(torch.autograd.Function):
    """(s, y) = (x + res, RMSNorm(x + res)): the residual add of
    core/transformer_layer.py:96 / :102 and the RMSNorm that follows it
    (core/normalization.py:13-25) in one kernel each way.  s is rounded to x's
    dtype as torch's add rounds it; the backward adds the gradient of s to the
    norm's dx, rounding each as autograd's two ops do, and returns that sum as
    the gradient of both x and res."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, res: torch.Tensor, weight: torch.Tensor, eps: float,
                grad_into: bool = False):
        if weight.dim() != 1 or x.shape[-1] != weight.shape[0]:
            raise ValueError(f"weight {tuple(weight.shape)} does not match the last dim of x "
                             f"{tuple(x.shape)}")
        if res.shape != x.shape or res.dtype != x.dtype:
            raise ValueError(f"res {res.dtype} {tuple(res.shape)} must match x {x.dtype} "
                             f"{tuple(x.shape)}")
        _lib._require_gpu(x, res, weight)
        w = _norm_weight(x, weight)
        xr, rr = _rows_view(x), _rows_view(res)
        s = torch.empty(x.shape, dtype=x.dtype, device=x.device)
        y = torch.empty(x.shape, dtype=w.dtype if w.dtype == torch.float32 else x.dtype,
                        device=x.device)
        rstd = torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device)
        _lib.rmsnorm_add_fwd(xr, rr, w, eps, s, y, rstd)
        ctx.save_for_backward(s, w, rstd)
        ctx.weight_dtype = weight.dtype
        ctx.grad_into = grad_into
        ctx.set_materialize_grads(False)
        return s, y

    @staticmethod
    def backward(ctx, ds, dy):
        s, w, rstd = ctx.saved_tensors
        if dy is None:  # only the sum is used: the norm contributes nothing
            dx = ds.to(s.dtype)
            return (dx, dx, torch.zeros(w.shape, dtype=ctx.weight_dtype, device=w.device), None,
                    None)
        dy = _rows_view(dy)
        rows = rstd.numel()
        dx = torch.empty(s.shape, dtype=s.dtype, device=s.device)
        ws = torch.empty(_lib.rmsnorm_workspace(rows, s.shape[-1]), dtype=torch.float32,
                         device=s.device)
        g = _grad_target(w, ctx.weight_dtype) if ctx.grad_into else None
        dw = g if g is not None else torch.empty(w.shape, dtype=w.dtype, device=w.device)
        if ds is None:  # only the normalised output is used (e.g. after the last add)
            _lib.rmsnorm_bwd(s, w, rstd, dy, dx, dw, ws, accumulate=g is not None)
        else:
            ds = _rows_view(ds.to(s.dtype))
            _lib.rmsnorm_add_bwd(s, w, rstd, dy, ds, dx, dw, ws, accumulate=g is not None)
        if g is not None:
            return dx, dx, None, None, None
        return dx, dx, dw.to(ctx.weight_dtype), None, None


def add_rms_norm(x: torch.Tensor, res: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6,
                 grad_into: bool = False):
    """``s = x + res; return s, RMSNorm(s)`` in one kernel (and one backward).
    `grad_into` as for FusedRMSNorm."""
    return FusedAddRMSNorm.apply(x, res, weight, eps, grad_into)


class RMSNorm(nn.Module):
    """RMSNorm(hidden_size, eps=1e-6) with an fp32 weight of ones, as
    core/normalization.py:8-11 (on the current GPU unless `device` is given)."""

    def __init__(self, hidden_size: int, eps: float = 1e-6, device=None):
        super().__init__()
        self.eps = eps
        if device is None:
            device = torch.cuda.current_device() if torch.cuda.is_available() else "cpu"
        self.weight = nn.Parameter(torch.ones(hidden_size, device=device, dtype=torch.float32))

    def forward(self, x):
        return FusedRMSNorm.apply(x, self.weight, self.eps)
