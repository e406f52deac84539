"""Rotary position embedding for MI355X: the drop-in for core/rope_triton.py.

``apply_rope(x, cos, sin)`` and ``apply_rope_qk(q, k, cos, sin)`` keep the
reference's API (core/rope_triton.py:144-148): x is ``[S, B, H, D]`` (any
strides, e.g. the q/k views the attention block cuts out of its fused qkv
projection), cos/sin are ``[S, D/2]`` tables, adjacent elements ``(2i, 2i+1)``
form the rotated pairs, the output is ``torch.empty_like(x)`` and the backward
applies the inverse rotation (rotation by -theta, :50-72).

``apply_rope_qk`` rotates q and k in one kernel launch (and their gradients in
one launch in backward) instead of two.  ``TritonRoPE`` is kept as an alias of
``RoPE`` so code written against the reference's class name keeps working; no
Triton is involved.
"""
from __future__ import annotations

import torch

from . import _lib


def _check(x, cos, sin):
    if x.dim() != 4:
        raise ValueError(f"x must be [SEQ_LEN, BATCH, HEADS, HEAD_DIM]; got shape {tuple(x.shape)}")
    S, _, _, D = x.shape
    if D % 2 != 0:
        raise AssertionError("HEAD_DIM must be even")
    for name, t in (("cos", cos), ("sin", sin)):
        if t.dim() != 2 or t.shape[0] < S or t.shape[1] < D // 2:
            raise ValueError(
                f"{name} must be [>= SEQ_LEN, >= HEAD_DIM // 2] = [>= {S}, >= {D // 2}]; got "
                f"{tuple(t.shape)}")


class RoPE(torch.autograd.Function):
    """Rotate x by the angles in (cos, sin); backward rotates by the negated angles."""

    @staticmethod
    def forward(ctx, x, cos, sin):
        _check(x, cos, sin)
        out = torch.empty_like(x)
        _lib.rope(x, cos, sin, out, inverse=False)
        ctx.save_for_backward(cos, sin)
        return out

    @staticmethod
    def backward(ctx, d_out):
        cos, sin = ctx.saved_tensors
        d_x = torch.empty_like(d_out)
        _lib.rope(d_out, cos, sin, d_x, inverse=True)
        return d_x, None, None


# Name used by core/rope_triton.py:7; same semantics.
TritonRoPE = RoPE


class RoPEQK(torch.autograd.Function):
    """q and k rotated together: one launch forward, one launch backward."""

    @staticmethod
    def forward(ctx, q, k, cos, sin):
        _check(q, cos, sin)
        if q.shape != k.shape or q.dtype != k.dtype:
            raise ValueError("q and k must have the same shape and dtype")
        q_out = torch.empty_like(q)
        k_out = torch.empty_like(k)
        _lib.rope_qk(q, k, cos, sin, q_out, k_out, inverse=False)
        ctx.save_for_backward(cos, sin)
        return q_out, k_out

    @staticmethod
    def backward(ctx, dq, dk):
        cos, sin = ctx.saved_tensors
        dq_in = torch.empty_like(dq)
        dk_in = torch.empty_like(dk)
        if dq.shape == dk.shape and dq.dtype == dk.dtype:
            _lib.rope_qk(dq, dk, cos, sin, dq_in, dk_in, inverse=True)
        else:
            _lib.rope(dq, cos, sin, dq_in, inverse=True)
            _lib.rope(dk, cos, sin, dk_in, inverse=True)
        return dq_in, dk_in, None, None


def apply_rope(x, cos, sin):
    """API of core/rope_triton.py:144-145."""
    return RoPE.apply(x, cos, sin)


def apply_rope_qk(q, k, cos, sin):
    """API of core/rope_triton.py:147-148 (one launch for both tensors)."""
    return RoPEQK.apply(q, k, cos, sin)
