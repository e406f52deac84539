"""GPT train step that drives the attention hot path (config 5).

The caller of the path in the reference is its GPT training loop at TP=1 /
DP=1; this module is the build's own counterpart of that caller, so the new
kernels run inside a real train step:

* model (core/models/gpt.py:10-35, core/transformer_layer.py:14-105,
  core/mlp.py:9-33, core/normalization.py:6-25): token embedding -> N pre-norm
  blocks [RMSNorm -> attention -> residual, RMSNorm -> SwiGLU MLP -> residual]
  -> final RMSNorm -> untied output head; no biases, dropout 0; activations in
  the [S, B, H] layout the reference uses;
* attention block (core/transformer_layer.py:36-67): fused qkv projection
  viewed as [S, B, 3, heads, head_dim], RoPE on q and k in that layout,
  permute to [B, heads, S, head_dim], causal flash attention, back to
  [S, B, H], output projection.  `attention` and `rope` are injectable so a
  comparison run can substitute other implementations; the defaults are the
  HIP kernels;
* RMSNorm: fp32 mean square, rsqrt(ms + eps), cast back, times the weight
  (core/normalization.py:13-25), by default the fused HIP kernels;
* loss: softmax cross entropy on the (bf16) logits, mean over [S, B]
  (core/tensor_parallel/loss.py:9-72 at one rank; train.py:179-181), by
  default the fused HIP kernels (`loss_fn` injectable, e.g. the eager
  `SoftmaxCrossEntropy.apply` below);
* SwiGLU MLP (core/mlp.py:22-33), the activation by default on the fused HIP
  kernels;
* optimizer (core/optimizer.py:6-104 at one rank): parameters and gradients
  live in flat bf16 buffers the model computes in, an fp32 master copy takes
  the AdamW step, gradients are clipped by their global norm first, and the
  result is copied back to bf16; by default the fused HIP step
  (`DistributedOptimizer`), else `MixedPrecisionAdamW` on torch's AdamW;
* init: xavier-uniform for every projection and the embedding
  (core/tensor_parallel/layers.py:31,66,112), RMSNorm weights 1.

Everything here is ordinary PyTorch (the GEMMs, the embedding) except the
attention path, the loss, the RMSNorms, the SwiGLU activation and the
optimizer step.
"""
from __future__ import annotations

import dataclasses
import math
import time

import torch
import torch.nn as nn
import torch.nn.functional as F

from ..attention_block import attention_block
from ..cross_entropy import vocab_parallel_cross_entropy
from ..mlp import swiglu
from ..normalization import add_rms_norm, rms_norm
from ..optimizer import DistributedOptimizer
from ..flash_attn import apply_flash_attn
from ..position_embeddings import RotaryEmbedding
from ..rope import apply_rope_qk


class _LinearGradInto(torch.autograd.Function):
    """``F.linear(x, w)`` whose weight gradient the GEMM accumulates itself into
    ``w.grad`` when that already exists (the optimizer's flat gradient buffer):
    ``w.grad.addmm_(gy^T, x)``, beta = 1 in the GEMM's epilogue, instead of a
    separate gradient tensor that autograd then adds into the buffer with one
    more pass over it.  Without a usable ``w.grad`` (none yet, another dtype or
    layout, or a double backward) the gradient is returned as F.linear's is.

    The fused form rounds once, round(g + acc), where autograd's add rounds the
    gradient first, round(round(g) + acc).  The two agree bit for bit only when
    ``w.grad`` starts zeroed and the weight receives exactly one gradient per
    backward, as in this harness (the optimizer zeroes its flat buffer each step
    and every projection weight is used once).  With micro-batch accumulation or
    a weight used twice in one graph the results would differ in the last bit."""

    @staticmethod
    def forward(ctx, x, w):
        ctx.save_for_backward(x, w)
        return F.linear(x, w)

    @staticmethod
    def backward(ctx, gy):
        x, w = ctx.saved_tensors
        gx = gy.matmul(w) if ctx.needs_input_grad[0] else None
        if not ctx.needs_input_grad[1]:
            return gx, None
        gy2 = gy.reshape(-1, gy.shape[-1])
        x2 = x.reshape(-1, x.shape[-1])
        g = w.grad
        if (g is None or torch.is_grad_enabled() or g.dtype != gy.dtype or g.shape != w.shape
                or not g.is_contiguous()):
            return gx, gy2.t().matmul(x2)
        g.addmm_(gy2.t(), x2)
        return gx, None


def _linear_into_grad(x, w):
    return _LinearGradInto.apply(x, w)


@dataclasses.dataclass
class GPTConfig:
    """Defaults follow train.py:15-26 and BASELINE config 5 (vocab 50257)."""
    vocab_size: int = 50257
    hidden_size: int = 768
    num_layers: int = 12
    num_attention_heads: int = 12
    max_position_embeddings: int = 1024
    intermediate_size: int = 3072
    rms_norm_eps: float = 1e-5
    rope_base: float = 10000.0


def _xavier(out_features, in_features, device):
    w = torch.empty(out_features, in_features, device=device, dtype=torch.float32)
    nn.init.xavier_uniform_(w)
    return nn.Parameter(w)


class RMSNorm(nn.Module):
    """The HIP kernels by default; `eager=True` runs the reference's op sequence."""

    def __init__(self, hidden_size, eps, device, eager=False, grad_into=False):
        super().__init__()
        self.eps = eps
        self.eager = eager
        self.grad_into = grad_into  # weight gradient added into .grad by the kernel
        self.weight = nn.Parameter(torch.ones(hidden_size, device=device, dtype=torch.float32))

    def forward(self, x):
        if not self.eager:
            return rms_norm(x, self.weight, self.eps, self.grad_into)
        dtype = x.dtype
        xf = x.float()
        xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        return xf.to(dtype) * self.weight


class Attention(nn.Module):
    def __init__(self, cfg: GPTConfig, device, attention=None, rope=None, linear=F.linear):
        super().__init__()
        self.lin = linear
        self.heads = cfg.num_attention_heads
        self.head_dim = cfg.hidden_size // cfg.num_attention_heads
        self.qkv = _xavier(3 * cfg.hidden_size, cfg.hidden_size, device)
        self.out = _xavier(cfg.hidden_size, cfg.hidden_size, device)
        self.rotary = RotaryEmbedding(self.head_dim, cfg.max_position_embeddings, cfg.rope_base,
                                      device=device)
        self.attention = attention or apply_flash_attn
        self.rope = rope or apply_rope_qk
        # With the HIP kernels on both sides, the block runs fused: no relayout
        # copies of q/k/v, O or the qkv gradient.
        self.fused = attention is None and rope is None
        self._tables_key = None
        self._tables = None

    def tables(self, x, S):
        """RotaryEmbedding's tables in x's dtype.  It casts its fp32 tables on
        every call (position_embeddings.py, as the reference's does); the
        tables never change, so the cast is kept per (dtype, length)."""
        key = (x.dtype, S)
        if key != self._tables_key:
            self._tables = self.rotary(x, seq_len=S)
            self._tables_key = key
        return self._tables

    def forward(self, x):  # x: [S, B, H]
        S, B, _ = x.shape
        if self.fused:
            cos, sin = self.tables(x, S)
            return self.lin(attention_block(self.lin(x, self.qkv), cos, sin, self.heads),
                            self.out)
        qkv = self.lin(x, self.qkv).view(S, B, 3, self.heads, self.head_dim)
        q, k, v = qkv.unbind(2)
        cos, sin = self.tables(q, S)
        q, k = self.rope(q, k, cos, sin)
        o = self.attention(q.permute(1, 2, 0, 3), k.permute(1, 2, 0, 3), v.permute(1, 2, 0, 3))
        o = o.permute(2, 0, 1, 3).reshape(S, B, -1)
        return self.lin(o, self.out)


class SwiGLU(nn.Module):
    """The HIP activation kernels by default; `eager=True` runs the reference's ops."""

    def __init__(self, cfg: GPTConfig, device, eager=False, linear=F.linear):
        super().__init__()
        self.eager = eager
        self.lin = linear
        self.gate_up = _xavier(2 * cfg.intermediate_size, cfg.hidden_size, device)
        self.down = _xavier(cfg.hidden_size, cfg.intermediate_size, device)

    def forward(self, x):
        gate_up = self.lin(x, self.gate_up)
        if not self.eager:
            return self.lin(swiglu(gate_up), self.down)
        gate, up = gate_up.chunk(2, dim=-1)
        return self.lin(F.silu(gate) * up, self.down)


class Block(nn.Module):
    def __init__(self, cfg: GPTConfig, device, attention=None, rope=None, eager_ops=False,
                 linear=F.linear, grad_into=False):
        super().__init__()
        self.norm1 = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps, device, eager_ops, grad_into)
        self.attn = Attention(cfg, device, attention, rope, linear)
        self.norm2 = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps, device, eager_ops, grad_into)
        self.mlp = SwiGLU(cfg, device, eager=eager_ops, linear=linear)

    def forward(self, x):
        x = x + self.attn(self.norm1(x))
        return x + self.mlp(self.norm2(x))


class GPT(nn.Module):
    """input ids [B, S] -> logits [S, B, V]."""

    def __init__(self, cfg: GPTConfig, device, attention=None, rope=None, eager_ops=False,
                 fuse_add_norm=True, gemm_grad_accumulate=True):
        super().__init__()
        self.cfg = cfg
        # the projections' weight gradients accumulated by their GEMMs, and the
        # norms' by their backward kernels, into the optimizer's gradient buffer
        # (not with eager_ops, which keeps the reference's ops throughout)
        into = gemm_grad_accumulate and not eager_ops
        self.lin = _linear_into_grad if into else F.linear
        emb = torch.empty(cfg.vocab_size, cfg.hidden_size, device=device, dtype=torch.float32)
        nn.init.xavier_uniform_(emb)
        self.embedding = nn.Parameter(emb)
        self.blocks = nn.ModuleList(
            [Block(cfg, device, attention, rope, eager_ops, self.lin, into)
             for _ in range(cfg.num_layers)])
        self.norm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps, device, eager_ops, into)
        self.head = _xavier(cfg.vocab_size, cfg.hidden_size, device)
        self.eager_ops = eager_ops
        self.fuse_add_norm = fuse_add_norm and not eager_ops

    def forward(self, ids):
        x = F.embedding(ids, self.embedding).transpose(0, 1).contiguous()  # [S, B, H]
        if not self.fuse_add_norm:
            for blk in self.blocks:
                x = blk(x)
            return self.lin(self.norm(x), self.head)
        # The same blocks with each residual add fused into the RMSNorm that
        # reads its sum: this block's norm2, then the next block's norm1 (or
        # the final norm); `h` is the normalised input of the next branch.
        h = self.blocks[0].norm1(x)
        for i, blk in enumerate(self.blocks):
            x, h = add_rms_norm(x, blk.attn(h), blk.norm2.weight, blk.norm2.eps,
                                blk.norm2.grad_into)
            nxt = self.blocks[i + 1].norm1 if i + 1 < len(self.blocks) else self.norm
            x, h = add_rms_norm(x, blk.mlp(h), nxt.weight, nxt.eps, nxt.grad_into)
        return self.lin(h, self.head)


class SoftmaxCrossEntropy(torch.autograd.Function):
    """Per-token loss log(sum exp(z - max)) - (z_t - max) on the logits' dtype;
    gradient softmax - onehot."""

    @staticmethod
    def forward(ctx, logits, target):
        z = logits - logits.max(dim=-1, keepdim=True)[0]
        e = torch.exp(z)
        s = e.sum(dim=-1)
        zt = z.gather(-1, target.unsqueeze(-1)).squeeze(-1)
        loss = torch.log(s) - zt
        e.div_(s.unsqueeze(-1))
        ctx.save_for_backward(e, target)
        return loss

    @staticmethod
    def backward(ctx, grad):
        p, target = ctx.saved_tensors
        p = p.clone()
        p.scatter_add_(-1, target.unsqueeze(-1),
                       -torch.ones_like(target, dtype=p.dtype).unsqueeze(-1))
        return p * grad.unsqueeze(-1), None


class MixedPrecisionAdamW:
    """Flat bf16 parameter/gradient buffers for the model, fp32 master copy
    for AdamW, global-norm clipping (one data-parallel rank): the reference's
    sequence on torch's AdamW (the eager counterpart of the fused
    DistributedOptimizer)."""

    def __init__(self, model, lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1, clip=1.0,
                 dtype=torch.bfloat16):
        self.params = [p for p in model.parameters() if p.requires_grad]
        n = sum(p.numel() for p in self.params)
        dev = self.params[0].device
        self.param_buf = torch.zeros(n, dtype=dtype, device=dev)
        self.grad_buf = torch.zeros(n, dtype=dtype, device=dev)
        off = 0
        for p in self.params:
            k = p.numel()
            self.param_buf[off:off + k].copy_(p.data.reshape(-1))
            p.data = self.param_buf[off:off + k].view(p.shape)
            p.grad = self.grad_buf[off:off + k].view(p.shape)
            off += k
        self.master = self.param_buf.float().clone().requires_grad_(True)
        self.opt = torch.optim.AdamW([self.master], lr=lr, betas=betas, weight_decay=weight_decay)
        self.clip = clip
        self.dtype = dtype

    def zero_grad(self):
        self.grad_buf.zero_()

    def step(self):
        if self.clip and self.clip > 0:
            norm = torch.sqrt(torch.sum(self.grad_buf.float() ** 2))
            if norm > self.clip:
                self.grad_buf.mul_(self.clip / (norm + 1e-6))
        self.master.grad = self.grad_buf.float()
        self.opt.step()
        self.opt.zero_grad()
        self.param_buf.copy_(self.master.detach().to(self.dtype))


def synthetic_batch(batch, seq, vocab, seed, device):
    """uint16 ids [B, S+1] uniform in [0, vocab) -> (inputs [B,S], labels [B,S])
    (the one-token shift of core/data.py:40-43)."""
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, vocab, (batch, seq + 1), generator=g, dtype=torch.int64)
    ids = ids.to(torch.uint16).to(torch.int64)
    return ids[:, :-1].to(device), ids[:, 1:].to(device)


def train(cfg: GPTConfig, batch=8, seq=1024, steps=20, seed=5, device="cuda", attention=None,
          rope=None, warmup=0, loss_fn=None, eager_ops=False, fuse_add_norm=True,
          gemm_grad_accumulate=True, regions=None):
    """Build the model and optimizer from `seed`, run `warmup` untimed then
    `steps` timed train steps on one fixed synthetic batch.  Returns
    (losses, tokens_per_second).  `loss_fn(logits, target)` -> per-token loss
    defaults to the HIP cross entropy; `eager_ops` swaps the model's other HIP
    operators (RMSNorm, SwiGLU, the optimizer step) for the reference's eager
    op sequences; `fuse_add_norm=False` runs the residual adds as separate
    torch adds in front of the RMSNorm kernels; `gemm_grad_accumulate=False`
    leaves the projections' and the norms' weight gradients to autograd's
    accumulation;
    `regions` (resume() / pause()) brackets the timed steps for a profiler."""
    loss_fn = loss_fn or vocab_parallel_cross_entropy
    torch.manual_seed(seed)
    model = GPT(cfg, device, attention, rope, eager_ops, fuse_add_norm, gemm_grad_accumulate)
    if eager_ops:
        opt = MixedPrecisionAdamW(model)
    else:
        opt = DistributedOptimizer(model, torch.optim.AdamW,
                                   {"lr": 3e-4, "betas": (0.9, 0.95), "weight_decay": 0.1},
                                   clip_grad=1.0)
    inputs, labels = synthetic_batch(batch, seq, cfg.vocab_size, seed, device)
    labels_t = labels.transpose(0, 1).contiguous()

    def one_step():
        opt.zero_grad()
        logits = model(inputs)
        per_token = loss_fn(logits, labels_t)
        per_token.mean().backward()  # mean in the logits' dtype, as the reference does
        opt.step()
        return per_token.detach().float().mean()  # logged in fp32 for resolution

    for _ in range(warmup):
        one_step()
    torch.cuda.synchronize()
    if regions is not None:
        regions.resume()
    losses = []
    t0 = time.perf_counter()
    for _ in range(steps):
        losses.append(one_step())
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    if regions is not None:
        regions.pause()
    return [float(x) for x in losses], batch * seq * steps / dt
