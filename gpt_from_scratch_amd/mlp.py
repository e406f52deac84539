"""SwiGLU activation in one HIP kernel each way.

Replaces the activation of ``ParallelMLP.forward`` (core/mlp.py:24-28)::

    gate, up = gate_up.chunk(2, dim=-1)
    x = F.silu(gate) * up

with ``x = swiglu(gate_up)``.  The eager form runs silu and the product as two
passes and its backward adds a third (the concatenation of the chunk's two
gradients); here the forward reads ``gate_up`` once and writes ``h``, and the
backward reads ``gate_up`` and ``dh`` once and writes ``dgate_up`` in place of
the concatenation.  The arithmetic keeps torch's roundings: ``silu(gate)`` is
rounded to the tensor dtype before the product, and so is ``dh * up`` before
silu's derivative.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib


def _rows_view(t: torch.Tensor) -> torch.Tensor:
    try:
        _lib._rows(t)
        return t
    except ValueError:
        return t.contiguous()


class SwiGLU(torch.autograd.Function):
    """h [..., I] = silu(gate_up[..., :I]) * gate_up[..., I:]."""

    @staticmethod
    def forward(ctx, gate_up: torch.Tensor):
        if gate_up.dim() < 1 or gate_up.shape[-1] % 2:
            raise ValueError(f"gate_up's last dim must be even; got {tuple(gate_up.shape)}")
        _lib._require_gpu(gate_up)
        gu = _rows_view(gate_up)
        inter = gu.shape[-1] // 2
        h = torch.empty(gu.shape[:-1] + (inter,), dtype=gu.dtype, device=gu.device)
        _lib.swiglu_fwd(gu, h)
        ctx.save_for_backward(gu)
        return h

    @staticmethod
    def backward(ctx, dh):
        (gu,) = ctx.saved_tensors
        dh = _rows_view(dh.to(gu.dtype))
        dgu = torch.empty(gu.shape, dtype=gu.dtype, device=gu.device)
        _lib.swiglu_bwd(gu, dh, dgu)
        return dgu


def swiglu(gate_up: torch.Tensor) -> torch.Tensor:
    return SwiGLU.apply(gate_up)


class ParallelMLP(nn.Module):
    """The reference's MLP (core/mlp.py:9-33) at tensor-parallel size 1:
    gate_up projection [2I, H], fused SwiGLU, down projection [H, I]; weights
    xavier-uniform (core/tensor_parallel/layers.py), optional biases."""

    def __init__(self, config, device=None, dtype=torch.float32):
        super().__init__()
        self.hidden_size = config.hidden_size
        self.bias = getattr(config, "bias", False)
        self.intermediate_size = getattr(config, "intermediate_size", self.hidden_size * 4)
        if device is None:
            device = torch.cuda.current_device() if torch.cuda.is_available() else "cpu"
        gu = torch.empty(2 * self.intermediate_size, self.hidden_size, device=device, dtype=dtype)
        dn = torch.empty(self.hidden_size, self.intermediate_size, device=device, dtype=dtype)
        nn.init.xavier_uniform_(gu)
        nn.init.xavier_uniform_(dn)
        self.gate_up_weight = nn.Parameter(gu)
        self.down_weight = nn.Parameter(dn)
        self.gate_up_bias = (nn.Parameter(torch.zeros(2 * self.intermediate_size, device=device,
                                                      dtype=dtype)) if self.bias else None)
        self.down_bias = (nn.Parameter(torch.zeros(self.hidden_size, device=device, dtype=dtype))
                          if self.bias else None)

    def forward(self, x):
        gate_up = F.linear(x, self.gate_up_weight, self.gate_up_bias)
        return F.linear(swiglu(gate_up), self.down_weight, self.down_bias)
