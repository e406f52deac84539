"""CPU restatement of the reference's rotary embedding (test infrastructure).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's CPU-baseline leg import
this module; it is the checker, never the product.

Followed reference lines:
  * tables (core/position_embeddings.py:19, :34-40): freqs[i] = 1/base^(2i/D)
    in fp32; cos/sin(s * freqs[i]) in fp32; cast to the activation dtype on use
    (:51);
  * rotation (core/rope_triton.py:112-133): pairs are adjacent elements
    (2i, 2i+1); forward (e, o) -> (e c - o s, e s + o c); backward (inverse)
    (e, o) -> (e c + o s, o c - e s).

Pinned by (tests/test_oracle.py): the complex-multiplication form
(e + i o) * exp(i s theta); per-pair norm preservation; inverse(forward(x)) = x;
<R_m q, R_n k> depends only on m - n; position 0 is the identity; float64
numpy tables.
"""
from __future__ import annotations

import torch


def rope_tables(head_dim: int, seq_len: int, base: float = 10000.0, dtype=torch.float32):
    """cos, sin tables [seq_len, head_dim // 2] computed as the reference does (fp32)."""
    freqs = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    t = torch.arange(seq_len, dtype=torch.float32)
    thetas = torch.outer(t, freqs.to(torch.float32))
    return thetas.cos().to(dtype), thetas.sin().to(dtype)


def rope_tables_f64(head_dim: int, seq_len: int, base: float = 10000.0):
    """The same angles evaluated in float64 (independent of fp32 rounding)."""
    i = torch.arange(0, head_dim, 2, dtype=torch.float64)
    freqs = 1.0 / (base ** (i / head_dim))
    t = torch.arange(seq_len, dtype=torch.float64)
    thetas = torch.outer(t, freqs)
    return thetas.cos(), thetas.sin()


def rope_apply(x, cos, sin, inverse: bool = False, dtype=torch.float64):
    """Rotate x [S, B, H, D] with tables [>=S, D/2]; returns a tensor in `dtype`."""
    S, D = x.shape[0], x.shape[-1]
    x = x.to(dtype)
    c = cos[:S, : D // 2].to(dtype)[:, None, None, :]
    s = sin[:S, : D // 2].to(dtype)[:, None, None, :]
    e, o = x[..., 0::2], x[..., 1::2]
    if inverse:
        re, ro = e * c + o * s, o * c - e * s
    else:
        re, ro = e * c - o * s, e * s + o * c
    out = torch.empty_like(x)
    out[..., 0::2] = re
    out[..., 1::2] = ro
    return out
