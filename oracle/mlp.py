"""CPU restatement of the reference's SwiGLU activation (test infrastructure).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's CPU-baseline leg import
this module; it is the checker, never the product.

Followed reference lines (core/mlp.py:24-28): ``gate, up = gate_up.chunk(2,
dim=-1)``, ``x = F.silu(gate) * up``.  In a 16-bit dtype torch rounds each op's
result: s = round(silu(g)), h = round(s * u).  Autograd's backward of the
product and of silu: d_up = round(dh * s), d_s = round(dh * u),
d_g = round(d_s * sig (1 + g (1 - sig))), sig = 1 / (1 + exp(-g)), and the
chunk's backward concatenates [d_g, d_up].

Computed in float64 with the intermediate roundings applied when `dtype` is a
16-bit torch dtype (None: no rounding).

Pinned by (tests/test_oracle.py): torch's float64 F.silu and its autograd,
central finite differences of the unrounded form, silu(0) = 0 and
silu(x) -> x for large x, and a case where rounding silu first changes h.
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


def swiglu_forward(gate_up: np.ndarray, dtype=None) -> np.ndarray:
    gu = np.asarray(gate_up, dtype=np.float64)
    inter = gu.shape[-1] // 2
    g, u = gu[..., :inter], gu[..., inter:]
    s = _rnd(g / (1.0 + np.exp(-g)), dtype)
    return s * u


def swiglu_backward(gate_up: np.ndarray, dh: np.ndarray, dtype=None) -> np.ndarray:
    gu = np.asarray(gate_up, dtype=np.float64)
    dh = np.asarray(dh, dtype=np.float64)
    inter = gu.shape[-1] // 2
    g, u = gu[..., :inter], gu[..., inter:]
    sig = 1.0 / (1.0 + np.exp(-g))
    s = _rnd(g * sig, dtype)
    d_up = dh * s
    d_s = _rnd(dh * u, dtype)
    d_g = d_s * sig * (1.0 + g * (1.0 - sig))
    return np.concatenate([d_g, d_up], axis=-1)
