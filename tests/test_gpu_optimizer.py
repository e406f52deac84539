"""GPU checks of the fused optimizer step (mi_grad_sumsq + mi_adamw_step behind
DistributedOptimizer) against the reference's own sequence (clone, fp32 copy,
torch's multi-tensor AdamW on the GPU, copy back) and the float64 oracle.

Tolerances: without clipping both paths run the same fp32 AdamW formula with
different fusion of the operations, so the fp32 master agrees within
1e-6 |p| + 1e-5 lr.  With clipping the scaled gradient is rounded to bf16 and
the norm's fp32 sum differs in its last bits between the two reductions, which
can flip that rounding for a few elements: each flip moves the first steps'
update by up to ~2^-7 lr, so the bound gains 2e-2 lr per step.
"""
import copy

import numpy as np
import pytest
import torch

from oracle import adamw_step, clip_gradient

pytestmark = pytest.mark.gpu

KW = {"lr": 2e-3, "weight_decay": 0.1, "betas": (0.9, 0.95)}


def _model(dev, seed=0):
    torch.manual_seed(seed)
    return torch.nn.Sequential(torch.nn.Linear(64, 301, bias=True),
                               torch.nn.Linear(301, 32, bias=False)).to(dev)


def _pair(dev, clip):
    from gpt_from_scratch_amd.optimizer import DistributedOptimizer
    a = DistributedOptimizer(_model(dev), torch.optim.AdamW, KW, clip_grad=clip)
    b = DistributedOptimizer(_model(dev), torch.optim.AdamW, KW, clip_grad=clip)
    b.fused = False  # the reference's sequence on torch's AdamW
    assert a.fused
    return a, b


def _grads(n, step, dev, scale):
    g = torch.Generator(device=dev).manual_seed(100 + step)
    return (torch.randn(n, generator=g, device=dev) * scale).to(torch.bfloat16)


@pytest.mark.parametrize("clip,scale", [(0.0, 1.0), (1.0, 1e-3), (1.0, 1.0)])
def test_fused_step_matches_reference_sequence(gpu, clip, scale):
    a, b = _pair(gpu, clip)
    n = a.grad_buffer.numel()
    assert n == b.grad_buffer.numel() and n % 4 == 1  # exercises the scalar tail
    lr = KW["lr"]
    m_flips = 0.0
    for step in range(1, 6):
        g = _grads(n, step, gpu, scale)
        if clip > 0 and scale >= 1.0:
            # a flip of the clipped gradient's rounding moves m by (1 - b1) ulp(g)
            gmax = float(g.float().abs().max()) * clip / float(g.float().norm())
            m_flips = m_flips * KW["betas"][0] + (1 - KW["betas"][0]) * 2 ** -7 * gmax
        a.grad_buffer.copy_(g)
        b.grad_buffer.copy_(g)
        a.step()
        b.step()
        pa, pb = a.fp32_master_shard.detach(), b.fp32_master_shard.detach()
        flips = 2e-2 * lr * step if clip > 0 and scale >= 1.0 else 0.0
        bound = 1e-6 * pb.abs() + 1e-5 * lr + flips
        assert bool(((pa - pb).abs() <= bound).all()), float((pa - pb).abs().max())
        # the bf16 parameter buffer is the rounded master
        assert torch.equal(a.param_buffer, pa.to(torch.bfloat16))
    sa = a.optimizer.state[a.fp32_master_shard]
    sb = b.optimizer.state[b.fp32_master_shard]
    assert float(sa["step"]) == float(sb["step"]) == 5.0
    dm = (sa["exp_avg"] - sb["exp_avg"]).abs()
    assert bool((dm <= 1e-5 * sb["exp_avg"].abs() + 1e-9 + m_flips).all()), float(dm.max())


def test_fused_step_matches_float64_oracle(gpu):
    from gpt_from_scratch_amd.optimizer import DistributedOptimizer
    opt = DistributedOptimizer(_model(gpu, 3), torch.optim.AdamW, KW, clip_grad=1.0)
    n = opt.grad_buffer.numel()
    p = opt.fp32_master_shard.detach().double().cpu().numpy()
    m, v = np.zeros(n), np.zeros(n)
    for step in range(1, 4):
        g = _grads(n, step, gpu, 0.05)
        opt.grad_buffer.copy_(g)
        opt.step()
        gc, norm = clip_gradient(g.double().cpu().numpy(), 1.0, torch.bfloat16)
        assert abs(float(opt.grad_norm()) - norm) <= 1e-5 * norm
        p, m, v = adamw_step(p, m, v, gc, step, KW["lr"], KW["betas"], 1e-8, KW["weight_decay"])
        got = opt.fp32_master_shard.detach().double().cpu().numpy()
        bound = 1e-6 * np.abs(p) + 2e-2 * KW["lr"] * step
        assert (np.abs(got - p) <= bound).all(), np.abs(got - p).max()


def test_state_dict_round_trip_and_determinism(gpu):
    from gpt_from_scratch_amd.optimizer import DistributedOptimizer
    runs = []
    for split in (False, True, False):
        opt = DistributedOptimizer(_model(gpu, 7), torch.optim.AdamW, KW, clip_grad=1.0)
        n = opt.grad_buffer.numel()
        for step in range(1, 6):
            if split and step == 4:
                sd = copy.deepcopy(opt.state_dict())
                master = opt.fp32_master_shard.detach().clone()
                opt = DistributedOptimizer(_model(gpu, 7), torch.optim.AdamW, KW, clip_grad=1.0)
                opt.fp32_master_shard.data.copy_(master)
                opt.load_state_dict(sd)
            opt.grad_buffer.copy_(_grads(n, step, gpu, 1.0))
            opt.step()
        runs.append(opt.fp32_master_shard.detach().clone())
    assert torch.equal(runs[0], runs[1]) and torch.equal(runs[0], runs[2])


def test_grad_sumsq_matches_torch(gpu):
    from gpt_from_scratch_amd import _lib
    ws = torch.empty(_lib.adamw_workspace(), dtype=torch.float32, device=gpu)
    for n in (1, 5, 1024, 4099, 3_000_001):
        g = _grads(n, n, gpu, 1.0)
        _lib.grad_sumsq(g, ws)
        ref = float(g.double().pow(2).sum())
        assert abs(float(ws[0]) - ref) <= 1e-5 * ref + 1e-30


def test_other_optimizers_and_variants_take_the_reference_sequence(gpu):
    """optimizer_cls other than AdamW, and AdamW with amsgrad, run torch's own step
    on the same flat buffers, as core/optimizer.py does for any optimizer_cls."""
    from gpt_from_scratch_amd.optimizer import DistributedOptimizer
    for cls, kw in ((torch.optim.SGD, {"lr": 1e-2, "momentum": 0.9}),
                    (torch.optim.AdamW, dict(KW, amsgrad=True))):
        opt = DistributedOptimizer(_model(gpu, 11), cls, kw, clip_grad=1.0)
        assert not opt.fused
        ref = opt.fp32_master_shard.detach().clone().requires_grad_(True)
        ref_opt = cls([ref], **kw)
        for step in range(1, 4):
            g = _grads(opt.grad_buffer.numel(), step, gpu, 1.0)
            opt.grad_buffer.copy_(g)
            opt.step()
            gc = g.clone()
            norm = torch.sqrt(torch.sum(gc.float() ** 2))
            if norm > 1.0:
                gc.mul_(1.0 / (norm + 1e-6))
            ref.grad = gc.float()
            ref_opt.step()
            assert torch.equal(opt.fp32_master_shard.detach(), ref.detach())
            assert torch.equal(opt.param_buffer, ref.detach().to(torch.bfloat16))
        with pytest.raises(RuntimeError, match="no fused step"):
            opt.grad_norm()
