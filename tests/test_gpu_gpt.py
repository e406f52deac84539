"""Config 5: the full GPT train step (12 layers, hidden 768, 12 heads, SwiGLU,
RMSNorm, vocab 50257, B=8, S=1024) with attention, RoPE, the loss, the
RMSNorms, the SwiGLU activation and the optimizer step on the HIP kernels, 20
steps from one seeded init and batch.

* Loss parity of the hot path (the north star's config-5 check): the same run
  with only attention and RoPE swapped for the reference's maths in fp32 (every
  other kernel identical), so the loss difference isolates the path.  Its
  scale is set by bf16 rounding: the same fp32 run against one that rounds P to
  bf16 before P V, as the reference's kernel does (core/myFlashAttn.py:717).
  The kernels round like the reference (P and dS in bf16), so they may move the
  loss by about as much; the bound is three times that plus 1e-3.
* End to end: the same run with every fused operator swapped for the
  reference's eager op sequence (attention, RoPE, loss, RMSNorm, SwiGLU,
  AdamW step), a loose sanity bound on the loss curve."""
import pytest
import torch

from gpt_from_scratch_amd.harness import GPTConfig, SoftmaxCrossEntropy, train
from oracle import attention_forward, rope_apply

pytestmark = pytest.mark.gpu


def eager_attention(q, k, v, round_p=False):
    """fp32 maths on the same bf16 inputs, result rounded to bf16; with round_p,
    P is rounded to the input dtype before P V (core/myFlashAttn.py:717)."""
    if not round_p:
        return attention_forward(q.float().contiguous(), k.float().contiguous(),
                                 v.float().contiguous(), True, dtype=torch.float32)[0].to(q.dtype)
    S, D = q.shape[-2], q.shape[-1]
    s = torch.matmul(q.float(), k.float().transpose(-1, -2).contiguous()) / D ** 0.5
    mask = torch.ones(S, S, dtype=torch.bool, device=q.device).tril()
    p = torch.softmax(s.masked_fill(~mask, float("-inf")), dim=-1).to(q.dtype).float()
    return torch.matmul(p, v.float()).to(q.dtype)


def eager_rope(q, k, cos, sin):
    return (rope_apply(q, cos, sin, dtype=torch.float32).to(q.dtype),
            rope_apply(k, cos, sin, dtype=torch.float32).to(k.dtype))


def test_config5_loss_parity(gpu):
    torch.backends.cuda.matmul.allow_tf32 = False
    cfg = GPTConfig()
    run = lambda **kw: train(cfg, batch=8, seq=1024, steps=20, seed=5, device=gpu, **kw)
    kern, tps = run()
    ref, _ = run(attention=eager_attention, rope=eager_rope)
    rnd, _ = run(attention=lambda q, k, v: eager_attention(q, k, v, True), rope=eager_rope)
    dl = max(abs(a - b) for a, b in zip(kern, ref))
    dr = max(abs(a - b) for a, b in zip(rnd, ref))
    print(f"config5 tokens/s {tps:.0f}; loss[0] {kern[0]:.4f} loss[19] {kern[-1]:.4f}; "
          f"max |dloss| vs fp32 attention {dl:.5f}, bf16-P rounding {dr:.5f}")
    assert all(torch.isfinite(torch.tensor(kern)))
    assert abs(kern[0] - 10.82) < 0.3          # ~ln(vocab) at xavier init
    assert kern[-1] < kern[0] - 1.0            # the fixed batch is being fit
    assert dl <= 3 * dr + 1e-3, (dl, dr, kern, ref)


def test_config5_end_to_end_eager_ops(gpu):
    torch.backends.cuda.matmul.allow_tf32 = False
    cfg = GPTConfig()
    kern, tps = train(cfg, batch=8, seq=1024, steps=20, seed=5, device=gpu)
    ref, ref_tps = train(cfg, batch=8, seq=1024, steps=20, seed=5, device=gpu,
                         attention=eager_attention, rope=eager_rope,
                         loss_fn=SoftmaxCrossEntropy.apply, eager_ops=True)
    diffs = [abs(a - b) for a, b in zip(kern, ref)]
    print(f"config5 tokens/s kernels {tps:.0f} eager {ref_tps:.0f}; max |dloss| {max(diffs):.5f}")
    assert max(diffs) < 0.05, diffs


def test_config5_fused_add_norm_matches_separate_ops(gpu):
    """The residual adds fused into the RMSNorms that read their sums give the
    same losses, bit for bit, as separate torch adds in front of the RMSNorm
    kernels (the same roundings in both directions)."""
    torch.backends.cuda.matmul.allow_tf32 = False
    cfg = GPTConfig()
    fused, tps_f = train(cfg, batch=8, seq=1024, steps=4, seed=5, device=gpu)
    sep, tps_s = train(cfg, batch=8, seq=1024, steps=4, seed=5, device=gpu, fuse_add_norm=False)
    print(f"config5 tokens/s fused add+norm {tps_f:.0f}, separate adds {tps_s:.0f}")
    assert fused == sep, (fused, sep)


def test_config5_gemm_grad_accumulate_matches_autograd(gpu):
    """The projections' weight gradients accumulated by their GEMMs into the
    optimizer's flat gradient buffer (addmm with beta = 1) give the same losses,
    bit for bit, as autograd's separate gradient plus in-place add into the
    zeroed buffer (x + 0 = x)."""
    torch.backends.cuda.matmul.allow_tf32 = False
    cfg = GPTConfig()
    acc, tps_a = train(cfg, batch=8, seq=1024, steps=4, seed=5, device=gpu)
    sep, tps_s = train(cfg, batch=8, seq=1024, steps=4, seed=5, device=gpu,
                       gemm_grad_accumulate=False)
    print(f"config5 tokens/s GEMM-accumulated weight grads {tps_a:.0f}, autograd adds {tps_s:.0f}")
    assert acc == sep, (acc, sep)


def test_linear_grad_into_falls_back_without_buffer(gpu):
    """Without an existing .grad the weight gradient is returned to autograd
    (a leaf gets it as with F.linear); with one, it is accumulated in place."""
    from gpt_from_scratch_amd.harness.gpt import _linear_into_grad
    g = torch.Generator(device=gpu).manual_seed(3)
    x = torch.randn(5, 3, 64, generator=g, device=gpu).to(torch.bfloat16).requires_grad_(True)
    w = torch.randn(32, 64, generator=g, device=gpu).to(torch.bfloat16).requires_grad_(True)
    gy = torch.randn(5, 3, 32, generator=g, device=gpu).to(torch.bfloat16)
    y = _linear_into_grad(x, w)
    y.backward(gy)
    xr, wr = x.detach().clone().requires_grad_(True), w.detach().clone().requires_grad_(True)
    torch.nn.functional.linear(xr, wr).backward(gy)
    assert torch.equal(x.grad, xr.grad)
    torch.testing.assert_close(w.grad.float(), wr.grad.float(), rtol=2 ** -7, atol=1e-3)
    first = w.grad.clone()
    _linear_into_grad(x.detach(), w).backward(gy)  # accumulated into the existing grad
    torch.testing.assert_close(w.grad.float(), 2 * first.float(), rtol=2 ** -7, atol=1e-2)
