"""Shared helpers of the GPU parity tests: seeded inputs, reference evaluation
and the tolerance metrics of the attention path.

Tolerances (north star): bf16/fp16 attention outputs and gradients within
max-abs 2e-2 and mean-rel 1e-2 of the fp32 reference, where
mean-rel = mean(|got - ref|) / mean(|ref|); fp32 attention within 1e-4;
RoPE within 1e-3 in fp32.
"""
import math

import torch

from oracle import attention_backward, attention_forward, rope_apply, rope_tables

MAX_ABS_BF16 = 2e-2
MEAN_REL_BF16 = 1e-2
TOL_FP32 = 1e-4


def seeded(shape, seed, std=1.0, dtype=torch.bfloat16):
    """N(0, std^2) drawn on the CPU from a seeded generator, rounded to dtype."""
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g, dtype=torch.float32) * std).to(dtype)


def metrics(got: torch.Tensor, ref: torch.Tensor):
    """(max-abs, mean-rel).  mean-rel is 0 when the reference is identically zero
    (e.g. dQ at S = 1): there only the absolute bound applies."""
    got, ref = got.float(), ref.float().to(got.device)
    err = (got - ref).abs()
    denom = float(ref.abs().mean())
    return float(err.max()), (float(err.mean()) / denom if denom > 0 else 0.0)


def assert_close_bf16(name, got, ref, max_abs=MAX_ABS_BF16, mean_rel=MEAN_REL_BF16):
    ma, mr = metrics(got, ref)
    assert ma <= max_abs and mr <= mean_rel, f"{name}: max-abs {ma:.3e} mean-rel {mr:.3e}"
    return ma, mr


def reference(q, k, v, do, causal=True, heads_per_chunk=8, with_backward=True):
    """fp32 evaluation of the oracle on q's device, a few heads at a time.

    q, k, v, do: [B, H, S, D] (any dtype).  Returns dict of fp32 tensors.
    """
    B, H, S, D = q.shape
    dev = q.device
    out = {"o": torch.empty(B, H, S, D, device=dev), "lse": torch.empty(B, H, S, device=dev)}
    if with_backward:
        for n in ("dq", "dk", "dv"):
            out[n] = torch.empty(B, H, S, D, device=dev)
    for b in range(B):
        for h0 in range(0, H, heads_per_chunk):
            sl = (b, slice(h0, h0 + heads_per_chunk))
            qq, kk, vv = (t[sl].float().contiguous() for t in (q, k, v))
            o, lse = attention_forward(qq, kk, vv, causal, dtype=torch.float32)
            out["o"][sl], out["lse"][sl] = o, lse
            del o, lse
            if with_backward:
                dq, dk, dv, _ = attention_backward(qq, kk, vv, do[sl].float().contiguous(), causal,
                                                   dtype=torch.float32)
                out["dq"][sl], out["dk"][sl], out["dv"][sl] = dq, dk, dv
    return out


def rope_inputs(B, H, S, D, seed, std=1.0, dtype=torch.bfloat16, device="cuda"):
    """q, k, v in the model's layout: views of one fused qkv [S, B, 3, H, D]
    tensor (core/transformer_layer.py:38-44), plus cos/sin in `dtype` and dO
    [B, H, S, D]."""
    qkv = seeded((S, B, 3, H, D), seed, std, dtype).to(device)
    q, k, v = qkv.unbind(2)
    cos, sin = rope_tables(D, S)
    do = seeded((B, H, S, D), seed + 1000, 1.0, dtype).to(device)
    return q, k, v, cos.to(dtype).to(device), sin.to(dtype).to(device), do


def scale_of(D):
    return 1.0 / math.sqrt(D)


def rescale_stress_inputs(S, D, device="cpu"):
    """q, k, v, dO (bf16, [1, 4, S, D]) whose scores grow along the key axis: q's
    axis-0 component is 8 and k's rises linearly to 100 * sqrt(D / 64), so the
    top score of a query rises by more than 8 log2 units per 64-key tile."""
    g = torch.Generator().manual_seed(71 + D)
    q = torch.randn(1, 4, S, D, generator=g) * 0.5
    k = torch.randn(1, 4, S, D, generator=g) * 0.5
    v = torch.randn(1, 4, S, D, generator=g)
    do = torch.randn(1, 4, S, D, generator=g)
    q[..., 0] = 8.0
    k[..., 0] = torch.linspace(0.0, 100.0 * math.sqrt(D / 64), S)
    return tuple(t.to(torch.bfloat16).to(device) for t in (q, k, v, do))


def grad_rounding_budget(q, k, v, do, o, causal):
    """fp32 gradients of attention and an element-wise bound on how far a
    computation that rounds like the reference may sit from them.

    The reference rounds P to bf16 before dV = P^T dO and scale * dS to bf16
    before dQ = dS K and dK = dS^T Q (core/myFlashAttn.py:1049, :1055, :1308), and
    computes delta = rowsum(dO * O) from the bf16 O.  The bound allows one bf16
    ulp (2^-8, twice round-to-nearest's half ulp) of each rounded term propagated
    through its product, the resulting error of delta, and the rounding of the
    gradient itself.  Returns (want, budget): dicts over "dq", "dk", "dv".
    """
    qf, kf, vf, dof = (t.float() for t in (q, k, v, do))
    S, D = q.shape[-2], q.shape[-1]
    sc = 1.0 / math.sqrt(D)
    sco = (qf @ kf.transpose(-1, -2)) * sc
    if causal:
        sco = sco.masked_fill(torch.ones(S, S, dtype=torch.bool, device=q.device).triu(1),
                              float("-inf"))
    pr = torch.softmax(sco, dim=-1)
    dp = dof @ vf.transpose(-1, -2)
    ds = pr * (dp - (pr * dp).sum(-1, keepdim=True))
    u = 2.0 ** -8
    ddelta = u * (dof.abs() * o.float().abs()).sum(-1, keepdim=True)
    want = {"dq": sc * (ds @ kf), "dk": sc * (ds.transpose(-1, -2) @ qf),
            "dv": pr.transpose(-1, -2) @ dof}
    budget = {
        "dq": sc * (u * (ds.abs() @ kf.abs()) + ddelta * (pr @ kf.abs())),
        "dk": sc * (u * (ds.abs().transpose(-1, -2) @ qf.abs())
                    + (pr * ddelta).transpose(-1, -2) @ qf.abs()),
        "dv": u * (pr.transpose(-1, -2) @ dof.abs()),
    }
    for n in budget:
        budget[n] = budget[n] + u * want[n].abs() + 1e-4
    return want, budget


def budget_ratio(got, want, budget):
    """Largest |got - want| / budget over the elements (<= 1 passes)."""
    return float(((got.float() - want).abs() / budget).max())
