"""Vocabulary cross entropy in two HIP kernels (forward, backward).

Drop-in for ``_VocabParallelCrossEntropy`` (core/tensor_parallel/loss.py:6-72)
at tensor-parallel size 1, called the same way (train.py:180-181)::

    loss = VocabParallelCrossEntropy.apply(logits, labels)   # [S, B]
    loss = loss.mean()

The reference makes about six passes over the ``[S, B, V]`` logits in forward
(max, subtract, exp, sum, gather, divide) and keeps the full softmax for
backward.  Here the forward reads the logits once (online max / sum-exp per
row, fp32) and saves only the fp32 log-sum-exp per row; the backward reads the
logits once more and writes the gradient, ``(exp(z - lse) - onehot) * dloss``.
A target outside ``[0, V)`` is masked as in the reference: its logit counts as
0 after the max shift and it gets no ``-1`` in the gradient.

``inplace_backward=True`` writes the gradient over the logits buffer (the
reference likewise overwrites its saved softmax, loss.py:69-70); use it only
when nothing else reads the logits after backward.
"""
from __future__ import annotations

import torch

from . import _lib


def _as_rows(t: torch.Tensor) -> torch.Tensor:
    try:
        _lib._rows(t)
        return t
    except ValueError:
        return t.contiguous()


class VocabParallelCrossEntropy(torch.autograd.Function):
    """loss[...] = logsumexp(logits[..., :]) - logits[..., target] (masked if out of range)."""

    @staticmethod
    def forward(ctx, logits: torch.Tensor, target: torch.Tensor, inplace_backward: bool = False):
        if logits.dim() < 1 or tuple(target.shape) != tuple(logits.shape[:-1]):
            raise ValueError(f"target shape {tuple(target.shape)} must be logits shape "
                             f"{tuple(logits.shape)} without the vocabulary dim")
        if target.dtype not in (torch.int64, torch.int32, torch.int16, torch.uint8, torch.int8):
            raise TypeError(f"target must be an integer tensor, got {target.dtype}")
        _lib._require_gpu(logits, target)
        z = _as_rows(logits)
        tgt = target.to(torch.int64).contiguous()
        loss = torch.empty(logits.shape[:-1], dtype=logits.dtype, device=logits.device)
        lse = torch.empty(logits.shape[:-1], dtype=torch.float32, device=logits.device)
        _lib.xent_fwd(z, tgt, loss, lse)
        ctx.save_for_backward(z, tgt, lse)
        ctx.inplace = bool(inplace_backward)
        return loss

    @staticmethod
    def backward(ctx, grad_output):
        z, tgt, lse = ctx.saved_tensors
        g = grad_output.to(z.dtype).contiguous()
        grad = z if ctx.inplace else torch.empty_like(z, memory_format=torch.contiguous_format)
        _lib.xent_bwd(z, tgt, lse, g, grad)
        return grad, None, None


# the reference's name (core/tensor_parallel/loss.py:6)
_VocabParallelCrossEntropy = VocabParallelCrossEntropy


def vocab_parallel_cross_entropy(logits, target, inplace_backward: bool = False):
    """Per-token loss ``[...]`` of logits ``[..., V]`` against integer targets ``[...]``."""
    return VocabParallelCrossEntropy.apply(logits, target, inplace_backward)
