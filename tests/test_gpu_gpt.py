"""Config 5: the full GPT train step (12 layers, hidden 768, 12 heads, SwiGLU,
RMSNorm, vocab 50257, B=8, S=1024) with attention, RoPE, the loss, the
RMSNorms, the SwiGLU activation and the optimizer step on the HIP kernels, 20
steps, against the same harness with the reference's eager ops swapped in for
all of them (same seed for init and data).  The two runs share
every other kernel, so the loss difference isolates the numerics of the
kernels."""
import pytest
import torch

from gpt_from_scratch_amd.harness import GPTConfig, SoftmaxCrossEntropy, train
from oracle import attention_forward, rope_apply

pytestmark = pytest.mark.gpu


def eager_attention(q, k, v):
    # fp32 math on the same bf16 inputs, result rounded to bf16
    return attention_forward(q.float().contiguous(), k.float().contiguous(),
                             v.float().contiguous(), True, dtype=torch.float32)[0].to(q.dtype)


def eager_rope(q, k, cos, sin):
    return (rope_apply(q, cos, sin, dtype=torch.float32).to(q.dtype),
            rope_apply(k, cos, sin, dtype=torch.float32).to(k.dtype))


def test_config5_loss_parity(gpu):
    torch.backends.cuda.matmul.allow_tf32 = False
    cfg = GPTConfig()
    losses, tps = train(cfg, batch=8, seq=1024, steps=20, seed=5, device=gpu)
    ref, ref_tps = train(cfg, batch=8, seq=1024, steps=20, seed=5, device=gpu,
                         attention=eager_attention, rope=eager_rope,
                         loss_fn=SoftmaxCrossEntropy.apply, eager_ops=True)
    diffs = [abs(a - b) for a, b in zip(losses, ref)]
    print(f"config5 tokens/s kernels {tps:.0f} eager {ref_tps:.0f}; "
          f"loss[0] {losses[0]:.4f} loss[19] {losses[-1]:.4f}; max |dloss| {max(diffs):.4f}")
    assert all(torch.isfinite(torch.tensor(losses)))
    assert abs(losses[0] - 10.82) < 0.3          # ~ln(vocab) at xavier init
    assert losses[-1] < losses[0] - 1.0          # the fixed batch is being fit
    assert max(diffs) < 0.05, diffs
