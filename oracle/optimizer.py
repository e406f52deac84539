"""CPU restatement of the reference's optimizer step (test infrastructure).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's CPU-baseline leg import
this module; it is the checker, never the product.

Followed reference lines (core/optimizer.py at one data-parallel rank, with
torch.optim.AdamW as train.py:130-138 configures it):
  * :100-104  norm = sqrt(sum g^2); if norm > clip: g <- g * clip / (norm + 1e-6),
              rounded back to the gradient buffer's dtype (in-place mul_ on it);
  * :88-92    the AdamW step on the fp32 master copy (torch's algorithm:
              p *= 1 - lr wd; m = b1 m + (1 - b1) g; v = b2 v + (1 - b2) g^2;
              p -= lr / (1 - b1^t) * m / (sqrt(v) / sqrt(1 - b2^t) + eps));
  * :95       the master rounded into the parameter buffer's dtype.

Computed in float64 except for the roundings the reference performs.

Pinned by (tests/test_oracle.py): torch.optim.AdamW itself (float64 on the
CPU, several steps, with weight decay), the first-step closed form
(update = lr * g / (|g| + eps') -> lr * sign(g)), and the clip's scaling of the
norm to the threshold.
"""
from __future__ import annotations

import numpy as np
import torch


def _rnd(a, dtype):
    if dtype is None or dtype == torch.float64:
        return a
    if dtype == torch.float32:
        return a.astype(np.float32).astype(np.float64)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).double().numpy()


def clip_gradient(g: np.ndarray, clip: float, dtype=None):
    """(clipped g, norm) as core/optimizer.py:98-104 computes them."""
    g = np.asarray(g, dtype=np.float64)
    norm = float(np.sqrt((g * g).sum()))
    if clip and clip > 0 and norm > clip:
        g = _rnd(g * (clip / (norm + 1e-6)), dtype)
    return g, norm


def adamw_step(master, exp_avg, exp_avg_sq, grad, step: int, lr: float, betas, eps: float,
               weight_decay: float):
    """One AdamW step (step = t after incrementing); returns new (master, m, v)."""
    b1, b2 = betas
    p = np.asarray(master, dtype=np.float64) * (1 - lr * weight_decay)
    g = np.asarray(grad, dtype=np.float64)
    m = b1 * np.asarray(exp_avg, dtype=np.float64) + (1 - b1) * g
    v = b2 * np.asarray(exp_avg_sq, dtype=np.float64) + (1 - b2) * g * g
    bc1 = 1 - b1 ** step
    bc2 = 1 - b2 ** step
    p = p - (lr / bc1) * m / (np.sqrt(v) / np.sqrt(bc2) + eps)
    return p, m, v
