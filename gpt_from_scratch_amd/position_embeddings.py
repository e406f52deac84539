"""Rotary tables: the counterpart of core/position_embeddings.py.

``RotaryEmbedding(head_dim, max_position_embeddings=2048, base=10000.0,
device=None)`` builds, in fp32,

    freqs[i]  = 1 / base ** (2i / head_dim)                 (:19)
    cos[s, i] = cos(s * freqs[i]),  sin[s, i] = sin(s * freqs[i])   (:34-40)

and ``forward(x, seq_len)`` returns the first ``seq_len`` rows cast to
``x.dtype`` (:45-51).  Unlike the reference, a ``seq_len`` beyond the cached
length regrows the cache (the reference's regrow call passes three arguments to
a one-argument method, :48 vs :29, and raises ``TypeError``).
"""
from __future__ import annotations

import torch
import torch.nn as nn


class RotaryEmbedding(nn.Module):
    def __init__(self, head_dim, max_position_embeddings=2048, base=10000.0, device=None):
        super().__init__()
        self.head_dim = head_dim
        self.max_position_embeddings = max_position_embeddings
        self.base = base
        if device is None:
            device = torch.cuda.current_device() if torch.cuda.is_available() else "cpu"
        freqs = 1.0 / (self.base ** (torch.arange(0, self.head_dim, 2, device=device,
                                                  dtype=torch.float32) / self.head_dim))
        self.register_buffer("freqs", freqs.to(torch.float32))
        self.max_seq_len_cached = 0
        self._set_cos_sin_cache(self.max_position_embeddings)

    def _set_cos_sin_cache(self, seq_len):
        self.max_seq_len_cached = seq_len
        t = torch.arange(seq_len, dtype=torch.float32, device=self.freqs.device)
        thetas = torch.outer(t, self.freqs)
        self.register_buffer("cos_cached", thetas.cos().to(torch.float32), persistent=False)
        self.register_buffer("sin_cached", thetas.sin().to(torch.float32), persistent=False)

    def forward(self, x, seq_len=None):
        if seq_len is None:
            seq_len = x.shape[0]
        if seq_len > self.max_seq_len_cached:
            self._set_cos_sin_cache(seq_len)
        return (self.cos_cached[:seq_len, :].to(x.dtype),
                self.sin_cached[:seq_len, :].to(x.dtype))
