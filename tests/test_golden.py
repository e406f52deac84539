"""The oracle against the committed golden fixtures (CPU), and the HIP kernels
against the same fixtures (GPU)."""
import glob
import os

import numpy as np
import pytest
import torch

from oracle import attention_backward, attention_forward, rope_apply

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden")
ATTN = sorted(glob.glob(os.path.join(GOLD, "attn_*.npz")))
ROPE = sorted(glob.glob(os.path.join(GOLD, "rope_*.npz")))


def _load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: torch.from_numpy(z[k].copy()) for k in z.files}


def test_fixtures_present():
    assert len(ATTN) >= 4 and len(ROPE) >= 1


@pytest.mark.parametrize("path", ATTN, ids=os.path.basename)
def test_oracle_attention_matches_golden(path):
    f = _load(path)
    causal = bool(f["causal"])
    c, s = f["cos"].double(), f["sin"].double()
    qr = rope_apply(f["q_sbhd"], c, s).permute(1, 2, 0, 3)
    kr = rope_apply(f["k_sbhd"], c, s).permute(1, 2, 0, 3)
    o, lse = attention_forward(qr, kr, f["v"], causal)
    dq, dk, dv, _ = attention_backward(qr, kr, f["v"], f["do"], causal)
    for name, got in (("o", o), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert torch.allclose(got.float(), f[name], atol=2e-6, rtol=1e-5), name


@pytest.mark.parametrize("path", ROPE, ids=os.path.basename)
def test_oracle_rope_matches_golden(path):
    f = _load(path)
    assert torch.allclose(rope_apply(f["x"], f["cos"], f["sin"]).float(), f["fwd"], atol=1e-6)
    assert torch.allclose(rope_apply(f["x"], f["cos"], f["sin"], inverse=True).float(), f["inv"],
                          atol=1e-6)


@pytest.mark.gpu
@pytest.mark.parametrize("path", ATTN, ids=os.path.basename)
def test_kernel_fp32_attention_matches_golden(path, gpu):
    """fp32 through the full drop-in chain: RoPE -> permute -> FlashAttn, fwd + bwd."""
    from gpt_from_scratch_amd import apply_flash_attn, apply_rope_qk
    f = _load(path)
    causal = bool(f["causal"])
    q = f["q_sbhd"].to(gpu).requires_grad_()
    k = f["k_sbhd"].to(gpu).requires_grad_()
    v = f["v"].to(gpu).requires_grad_()
    cos, sin = f["cos"].to(gpu), f["sin"].to(gpu)
    qr, kr = apply_rope_qk(q, k, cos, sin)
    o = apply_flash_attn(qr.permute(1, 2, 0, 3), kr.permute(1, 2, 0, 3), v, causal)
    o.backward(f["do"].to(gpu))
    torch.cuda.synchronize()
    assert torch.allclose(o.detach().cpu(), f["o"], atol=1e-4), "o"
    assert torch.allclose(v.grad.cpu(), f["dv"], atol=1e-4), "dv"
    # q/k grads flow back through the inverse rotation
    dq_ref = rope_apply(f["dq"].permute(2, 0, 1, 3), f["cos"], f["sin"], inverse=True).float()
    dk_ref = rope_apply(f["dk"].permute(2, 0, 1, 3), f["cos"], f["sin"], inverse=True).float()
    assert torch.allclose(q.grad.cpu(), dq_ref, atol=1e-4), "dq"
    assert torch.allclose(k.grad.cpu(), dk_ref, atol=1e-4), "dk"


@pytest.mark.gpu
@pytest.mark.parametrize("path", ROPE, ids=os.path.basename)
def test_kernel_rope_matches_golden(path, gpu):
    from gpt_from_scratch_amd import apply_rope
    from gpt_from_scratch_amd.rope import RoPE
    f = _load(path)
    x = f["x"].to(gpu)
    cos, sin = f["cos"].to(gpu), f["sin"].to(gpu)
    y = apply_rope(x, cos, sin)
    torch.cuda.synchronize()
    assert torch.allclose(y.cpu(), f["fwd"], atol=1e-6)
    xg = x.clone().requires_grad_()
    RoPE.apply(xg, cos, sin).backward(x)
    assert torch.allclose(xg.grad.cpu(), f["inv"], atol=1e-6)
