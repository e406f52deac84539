"""CPU restatement of the reference's RMSNorm (test infrastructure).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's CPU-baseline leg import
this module; it is the checker, never the product.

Followed reference lines (core/normalization.py):
  * :15-16  x upcast to fp32;
  * :19-21  r = rsqrt(mean_j x_j^2 + eps), n = x * r;
  * :23     n rounded to the input dtype;
  * :24     y = n * weight in the promoted dtype.
The backward is autograd's derivative of that composition (the rounding passes
gradients unchanged):
  dn = dy * w;  dx = r dn - x r^3 mean_j(dn_j x_j);  dw = sum_rows dy * round(n).

Here computed in float64 (rounding of n to the input dtype kept, as a float64
value), from numpy arrays of the already-rounded inputs.

Pinned by (tests/test_oracle.py): torch float64 autograd of the composition
(dx, dw); central finite differences; scale invariance of n (eps = 0); a
constant row normalising to +-1/sqrt(1 + eps/a^2); x . dx = 0 for eps = 0 and
w = 1; and the intermediate rounding on a case where it changes the result.
"""
from __future__ import annotations

import numpy as np
import torch


def _round_to(a: np.ndarray, dtype) -> np.ndarray:
    if dtype in (None, torch.float32, torch.float64):
        return a if dtype in (None, torch.float64) else a.astype(np.float32).astype(np.float64)
    return torch.from_numpy(a).to(dtype).double().numpy()


def rmsnorm_forward(x: np.ndarray, w: np.ndarray, eps: float, x_dtype=None):
    """(y, r) in float64; n is rounded to x_dtype (None: no rounding)."""
    x = np.asarray(x, dtype=np.float64)
    r = 1.0 / np.sqrt((x * x).mean(axis=-1) + eps)
    n = _round_to(x * r[..., None], x_dtype)
    return n * np.asarray(w, dtype=np.float64), r


def rmsnorm_backward(x: np.ndarray, w: np.ndarray, dy: np.ndarray, eps: float, x_dtype=None):
    """(dx, dw) in float64."""
    x = np.asarray(x, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    dy = np.asarray(dy, dtype=np.float64)
    H = x.shape[-1]
    r = 1.0 / np.sqrt((x * x).mean(axis=-1) + eps)
    dn = dy * w
    s = (dn * x).sum(axis=-1)
    dx = r[..., None] * dn - x * (r ** 3 * s / H)[..., None]
    n = _round_to(x * r[..., None], x_dtype)
    dw = (dy * n).reshape(-1, H).sum(axis=0)
    return dx, dw
