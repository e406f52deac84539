"""Flash attention for MI355X: the drop-in for core/myFlashAttn.py.

``FlashAttn`` / ``apply_flash_attn`` keep the reference's names, signatures,
tensor layouts and error behaviour (core/myFlashAttn.py:194-441, :1321-1322):

* inputs Q, K, V are ``[B, H, S, D]`` of one dtype (bf16, fp16 or fp32); the
  shapes must match (the reference asserts it, :203);
* ``softmax_scale = 1 / sqrt(D)`` (:201);
* forward returns a contiguous ``O`` of the input dtype and saves
  ``(Q, K, V, M, O)`` with ``M = logsumexp`` as fp32 ``[B, H, S]`` (:240, :280);
* backward returns ``(dQ, dK, dV, None)`` (:441), contiguous, input dtype.

Differences that do not change results: Q/K/V and dO are consumed through
their strides (the reference copies Q/K/V with ``.contiguous()``, :206-208),
any S is accepted (the reference needs S to be a multiple of its tile), and
there is no autotuning pass.  Everything runs in the HIP kernels of
libmi_attn.so; there is no CPU path.
"""
from __future__ import annotations

import torch

from . import _lib


def _kernel_ready(t: torch.Tensor) -> torch.Tensor:
    """Return t, or a contiguous copy if its layout cannot be read in place.

    The kernels need a unit stride on the last dim; the matrix-core path also
    wants 16-byte aligned rows, which every contiguous bf16/fp16 tensor with
    D % 8 == 0 has.
    """
    if t.stride(-1) != 1:
        return t.contiguous()
    esz = t.element_size()
    if t.data_ptr() % 16 or any((s * esz) % 16 for s in t.stride()[:-1]):
        c = t.contiguous()
        return c
    return t


class FlashAttn(torch.autograd.Function):
    """Causal / non-causal attention, ``O = softmax(Q K^T / sqrt(D) + mask) V``."""

    @staticmethod
    def forward(ctx, Q, K, V, causal_mask=True):
        BATCH_SIZE, NUM_HEADS, SEQ_LEN, HEAD_DIM = Q.shape
        softmax_scale = 1.0 / (HEAD_DIM ** 0.5)
        if not (Q.shape == K.shape == V.shape):
            raise AssertionError(
                f"Q, K, V must have the same shape; got {tuple(Q.shape)}, {tuple(K.shape)}, "
                f"{tuple(V.shape)}")
        if not (Q.dtype == K.dtype == V.dtype):
            raise TypeError(f"Q, K, V must share a dtype; got {Q.dtype}, {K.dtype}, {V.dtype}")
        Q, K, V = _kernel_ready(Q), _kernel_ready(K), _kernel_ready(V)
        O = torch.empty((BATCH_SIZE, NUM_HEADS, SEQ_LEN, HEAD_DIM), dtype=Q.dtype,
                        device=Q.device)
        M = torch.empty((BATCH_SIZE, NUM_HEADS, SEQ_LEN), dtype=torch.float32, device=Q.device)
        _lib.attn_fwd(Q, K, V, O, M, causal_mask, softmax_scale)
        ctx.save_for_backward(Q, K, V, M, O)
        ctx.softmax_scale = softmax_scale
        ctx.causal_mask = causal_mask
        return O

    @staticmethod
    def backward(ctx, dO):
        Q, K, V, M, O = ctx.saved_tensors
        dO = _kernel_ready(dO)
        if dO.dtype != Q.dtype:
            dO = dO.to(Q.dtype)
        ws = _lib.bwd_workspace(M)  # D (the reference's delta, :323) and lse * log2(e)
        dQ = torch.empty(Q.shape, dtype=Q.dtype, device=Q.device)
        dK = torch.empty(K.shape, dtype=K.dtype, device=K.device)
        dV = torch.empty(V.shape, dtype=V.dtype, device=V.device)
        _lib.attn_bwd(Q, K, V, O, dO, M, ws, dQ, dK, dV, ctx.causal_mask, ctx.softmax_scale)
        return dQ, dK, dV, None


def apply_flash_attn(q, k, v, causal_mask=True):
    """API of core/myFlashAttn.py:1321-1322."""
    return FlashAttn.apply(q, k, v, causal_mask)


def flash_attn_forward(q, k, v, causal_mask=True):
    """Forward only, without autograd: returns ``(O, M)`` (M = fp32 logsumexp)."""
    B, H, S, D = q.shape
    if not (q.shape == k.shape == v.shape):
        raise AssertionError("Q, K, V must have the same shape")
    q, k, v = _kernel_ready(q), _kernel_ready(k), _kernel_ready(v)
    o = torch.empty((B, H, S, D), dtype=q.dtype, device=q.device)
    m = torch.empty((B, H, S), dtype=torch.float32, device=q.device)
    _lib.attn_fwd(q, k, v, o, m, causal_mask, 1.0 / (D ** 0.5))
    return o, m


def flash_attn_backward(q, k, v, o, m, do, causal_mask=True):
    """Backward only, without autograd: returns ``(dQ, dK, dV, delta)``."""
    B, H, S, D = q.shape
    q, k, v, do = _kernel_ready(q), _kernel_ready(k), _kernel_ready(v), _kernel_ready(do)
    ws = _lib.bwd_workspace(m)
    dq = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    dk = torch.empty_like(dq)
    dv = torch.empty_like(dq)
    _lib.attn_bwd(q, k, v, o, do, m, ws, dq, dk, dv, causal_mask, 1.0 / (D ** 0.5))
    return dq, dk, dv, ws[0]
