"""CPU restatement of the reference's vocabulary cross entropy (test infrastructure).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's CPU-baseline leg import
this module; it is the checker, never the product.

Followed reference lines (core/tensor_parallel/loss.py, one tensor-parallel
rank, so every all_reduce is the identity):
  * :14-16  m = max_j z_j; z' = z - m;
  * :19-20  s = sum_j exp(z'_j);
  * :28-35  the target is in range iff 0 <= t < vocab; otherwise it is masked
            and its index replaced by 0;
  * :39-41  z'_t gathered, then set to 0 for a masked target;
  * :50     loss = log(s) - z'_t;
  * :54-56  the softmax exp(z')/s is saved;
  * :68-72  grad = (softmax - onehot(t) * in_range) * grad_output.

Computed in float64 (the reference computes in the logits dtype; the kernel
computes its row statistics in fp32).

Pinned by (tests/test_oracle.py): scipy's logsumexp; uniform logits give
log(vocab); invariance under a per-row shift; the gradient equals the central
finite difference of the loss; gradient rows of in-range targets sum to 0 and
rows of masked targets are the plain softmax.
"""
from __future__ import annotations

import numpy as np


def cross_entropy_forward(logits: np.ndarray, target: np.ndarray):
    """(loss [rows], lse [rows]) for logits [..., V] and int targets [...]; float64."""
    z = np.asarray(logits, dtype=np.float64)
    V = z.shape[-1]
    z2 = z.reshape(-1, V)
    t = np.asarray(target, dtype=np.int64).reshape(-1)
    m = z2.max(axis=-1)
    zs = z2 - m[:, None]
    s = np.exp(zs).sum(axis=-1)
    in_range = (t >= 0) & (t < V)
    tl = np.where(in_range, zs[np.arange(len(t)), np.where(in_range, t, 0)], 0.0)
    loss = np.log(s) - tl
    lse = m + np.log(s)
    return loss.reshape(z.shape[:-1]), lse.reshape(z.shape[:-1])


def cross_entropy_backward(logits: np.ndarray, target: np.ndarray, grad_loss: np.ndarray):
    """d loss / d logits, shape of logits, float64."""
    z = np.asarray(logits, dtype=np.float64)
    V = z.shape[-1]
    z2 = z.reshape(-1, V)
    t = np.asarray(target, dtype=np.int64).reshape(-1)
    g = np.asarray(grad_loss, dtype=np.float64).reshape(-1)
    m = z2.max(axis=-1, keepdims=True)
    p = np.exp(z2 - m)
    p /= p.sum(axis=-1, keepdims=True)
    rows = np.nonzero((t >= 0) & (t < V))[0]
    p[rows, t[rows]] -= 1.0
    return (p * g[:, None]).reshape(z.shape)
