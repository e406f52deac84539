"""The attention block's layout plumbing fused into the kernels' strides.

The reference's attention block (core/transformer_layer.py:36-67) views the
fused qkv projection ``[S, B, 3*H*D]`` as ``[S, B, 3, H, D]``, rotates q and k
(core/rope_triton.py), permutes q/k/v to ``[B, H, S, D]`` and copies them
contiguous (core/myFlashAttn.py:206-208), runs flash attention, and permutes
and reshapes ``O`` back to ``[S, B, H*D]`` for the output projection
(transformer_layer.py:61), which is another copy.  In backward, autograd then
assembles the qkv gradient from dQ, dK and dV with a stack, a third copy.

``attention_block(qkv, cos, sin, heads)`` computes the same thing with no
relayout copies, because every kernel here takes arbitrary strides:

* q and k are rotated (one launch) into a ``[S, B, 2, H, D]`` buffer; the
  attention reads those and v straight from the projection through
  ``[B, H, S, D]`` views;
* the forward writes ``O`` straight into ``[S, B, H, D]``, so the result is a
  free ``[S, B, H*D]`` view;
* the backward writes dQ, dK and dV straight into the slots of one
  ``[S, B, 3, H, D]`` gradient buffer, dQ and dK inverse-rotated by the
  attention kernels as they store them (no separate RoPE pass).

Results are bit-identical to ``apply_rope_qk`` followed by
``apply_flash_attn`` and the reshape: the same arithmetic in the same order
(the rotation fused into the backward's stores is the RoPE kernel's, applied
to the same rounded gradients); only the addresses differ.
"""
from __future__ import annotations

import torch

from . import _lib
from .rope import _check as _rope_check


def _viewable(t: torch.Tensor, shape) -> torch.Tensor:
    """t viewed as `shape`, through a contiguous copy if its strides do not allow it."""
    try:
        return t.view(shape)
    except RuntimeError:
        return t.contiguous().view(shape)


class AttentionBlock(torch.autograd.Function):
    """``[S, B, 3*H*D]`` qkv -> RoPE(q, k) -> flash attention -> ``[S, B, H*D]``."""

    @staticmethod
    def forward(ctx, qkv, cos, sin, heads: int, causal: bool = True):
        if qkv.dim() != 3 or qkv.shape[-1] % (3 * heads) != 0:
            raise ValueError(
                f"qkv must be [SEQ_LEN, BATCH, 3 * heads * HEAD_DIM]; got {tuple(qkv.shape)} "
                f"with heads={heads}")
        S, B, _ = qkv.shape
        D = qkv.shape[-1] // (3 * heads)
        if D % 2 != 0:
            raise AssertionError("HEAD_DIM must be even")
        qkv5 = _viewable(qkv, (S, B, 3, heads, D))
        q, k, v = qkv5.unbind(2)
        # the C ABI takes no table length: short or mis-shaped tables are refused here
        _rope_check(q, cos, sin)
        rot = torch.empty((S, B, 2, heads, D), dtype=qkv.dtype, device=qkv.device)
        _lib.rope_qk(q, k, cos, sin, rot[:, :, 0], rot[:, :, 1], inverse=False)
        o = torch.empty((S, B, heads, D), dtype=qkv.dtype, device=qkv.device)
        lse = torch.empty((B, heads, S), dtype=torch.float32, device=qkv.device)
        scale = 1.0 / (D ** 0.5)
        bhsd = (1, 2, 0, 3)
        _lib.attn_fwd(rot[:, :, 0].permute(bhsd), rot[:, :, 1].permute(bhsd), v.permute(bhsd),
                      o.permute(bhsd), lse, causal, scale)
        ctx.save_for_backward(rot, qkv5, o, lse, cos, sin)
        ctx.meta = (S, B, heads, D, bool(causal), scale)
        return o.view(S, B, heads * D)

    @staticmethod
    def backward(ctx, d_out):
        rot, qkv5, o, lse, cos, sin = ctx.saved_tensors
        S, B, heads, D, causal, scale = ctx.meta
        bhsd = (1, 2, 0, 3)
        d_o = _viewable(d_out, (S, B, heads, D))
        if d_o.stride(-1) != 1 or d_o.data_ptr() % 16 or any(
                (s * d_o.element_size()) % 16 for s in d_o.stride()[:-1]):
            d_o = d_o.contiguous()
        d_qkv = torch.empty((S, B, 3, heads, D), dtype=qkv5.dtype, device=qkv5.device)
        ws = _lib.bwd_workspace(lse)
        dq, dk, dv = d_qkv[:, :, 0], d_qkv[:, :, 1], d_qkv[:, :, 2]
        # dq, dk leave inverse-rotated: the gradients of q, k themselves
        _lib.attn_bwd_rope(rot[:, :, 0].permute(bhsd), rot[:, :, 1].permute(bhsd),
                           qkv5[:, :, 2].permute(bhsd), o.permute(bhsd), d_o.permute(bhsd), lse,
                           ws, dq.permute(bhsd), dk.permute(bhsd), dv.permute(bhsd), causal,
                           scale, cos, sin)
        return d_qkv.view(S, B, 3 * heads * D), None, None, None, None


def attention_block(qkv, cos, sin, heads: int, causal: bool = True):
    """``O = attention(RoPE(q), RoPE(k), v)`` as ``[S, B, H*D]`` from the fused
    qkv projection ``[S, B, 3*H*D]`` (the layout of core/transformer_layer.py:42-61);
    cos/sin are the ``[>= S, D/2]`` tables of ``RotaryEmbedding``."""
    return AttentionBlock.apply(qkv, cos, sin, heads, causal)
