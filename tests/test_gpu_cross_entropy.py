"""GPU parity of the fused vocabulary cross entropy (mi_xent_fwd / mi_xent_bwd)
against the float64 oracle (oracle/cross_entropy.py) on the same rounded inputs.

Tolerance: the kernels compute the row statistics and the softmax in fp32 and
round only their outputs, so a bf16/fp16 loss or gradient element is within one
rounding of the float64 value, |got - ref| <= 2^-8 |ref| (bf16) or 2^-11 |ref|
(fp16), plus the fp32 arithmetic's share: 1e-5 |ref| and an absolute 4e-6
(loss: the fp32 log-sum-exp; gradient: 4e-6 |dloss| for the fp32 softmax
probability, which matters where p - 1 cancels).
"""
import numpy as np
import pytest
import torch

from gpu_ref import seeded
from oracle import cross_entropy_backward, cross_entropy_forward

pytestmark = pytest.mark.gpu

ROUND = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11, torch.float32: 0.0}


def _check(name, got, ref, dtype, floor):
    got = got.detach().float().cpu().double().numpy()
    bound = np.abs(ref) * (ROUND[dtype] + 1e-5) + floor + 1e-30
    err = np.abs(got - ref)
    bad = err > bound
    assert not bad.any(), (f"{name}: {int(bad.sum())} of {bad.size} elements out of bound; "
                           f"worst err {err.max():.3e}")


def _run(logits, target, grad_loss, inplace=False):
    from gpt_from_scratch_amd import vocab_parallel_cross_entropy
    z = logits.detach().clone().requires_grad_(True)
    loss = vocab_parallel_cross_entropy(z, target, inplace_backward=inplace)
    loss.backward(grad_loss)
    return loss, z.grad


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("rows,V", [(64, 50257), (7, 1), (5, 7), (9, 8), (6, 9), (11, 33),
                                    (3, 1000)])
def test_matches_oracle(gpu, dtype, rows, V):
    z = seeded((rows, V), 11 + V, std=2.0, dtype=dtype)
    g = torch.Generator().manual_seed(V)
    t = torch.randint(0, V, (rows,), generator=g)
    dl = seeded((rows,), 12, dtype=dtype)
    loss, grad = _run(z.to(gpu), t.to(gpu), dl.to(gpu))
    assert loss.dtype == dtype and loss.shape == (rows,)
    ref_loss, _ = cross_entropy_forward(z.double().numpy(), t.numpy())
    ref_grad = cross_entropy_backward(z.double().numpy(), t.numpy(), dl.double().numpy())
    _check("loss", loss, ref_loss, dtype, 4e-6)
    _check("grad", grad, ref_grad, dtype, 4e-6 * np.abs(dl.double().numpy())[:, None])


def test_model_layout_masked_targets_and_strided_rows(gpu):
    """[S, B, V] logits that are a slice of a wider buffer (row stride != V, so
    rows start at every 2-byte offset mod 16), and targets outside [0, V)
    (masked: no -1 in the gradient, loss = lse - max)."""
    S, B, V = 24, 3, 50257
    wide = seeded((S, B, V + 5), 21, std=1.5).to(gpu)
    z = wide[..., 3:3 + V]
    assert not z.is_contiguous()
    g = torch.Generator().manual_seed(4)
    t = torch.randint(0, V, (S, B), generator=g)
    t[0, 0], t[5, 1], t[7, 2], t[9, 0] = -1, V, -100, V - 1
    dl = seeded((S, B), 22).to(gpu)
    loss, grad = _run(z, t.to(gpu), dl)
    zc = z.float().cpu().double().numpy()
    ref_loss, _ = cross_entropy_forward(zc, t.numpy())
    ref_grad = cross_entropy_backward(zc, t.numpy(), dl.float().cpu().double().numpy())
    _check("loss", loss, ref_loss, torch.bfloat16, 4e-6)
    _check("grad", grad, ref_grad, torch.bfloat16,
           4e-6 * np.abs(dl.float().cpu().double().numpy())[..., None])
    assert grad.shape == (S, B, V)


def test_inplace_backward_equals_out_of_place(gpu):
    V = 50257
    z = seeded((40, V), 31, std=3.0).to(gpu)
    t = torch.randint(0, V, (40,), generator=torch.Generator().manual_seed(5)).to(gpu)
    dl = torch.full((40,), 1.0 / 40, dtype=torch.bfloat16, device=gpu)
    loss_a, grad_a = _run(z, t, dl)
    loss_b, grad_b = _run(z, t, dl, inplace=True)
    assert torch.equal(loss_a, loss_b) and torch.equal(grad_a, grad_b)


def test_reference_call_site_and_torch_fp32(gpu):
    """train.py:180-181: `_VocabParallelCrossEntropy.apply(logits, labels).mean()`,
    against torch's fp32 cross entropy at config 5's shape [1024, 8, 50257]."""
    from gpt_from_scratch_amd import _VocabParallelCrossEntropy
    S, B, V = 1024, 8, 50257
    g = torch.Generator(device=gpu).manual_seed(9)
    z = (torch.randn(S, B, V, generator=g, device=gpu) * 2).to(torch.bfloat16).requires_grad_(True)
    t = torch.randint(0, V, (S, B), generator=g, device=gpu)
    loss = _VocabParallelCrossEntropy.apply(z, t)
    assert loss.shape == (S, B) and loss.dtype == torch.bfloat16
    loss.mean().backward()
    zf = z.detach().float().requires_grad_(True)
    ref = torch.nn.functional.cross_entropy(zf.view(-1, V), t.view(-1), reduction="none")
    ref.mean().backward()
    err = (loss.detach().float().view(-1) - ref.detach()).abs()
    assert float((err / ref.detach().abs()).max()) <= 2.0 ** -8 + 1e-5
    # gradient of the mean: the upstream 1/(S*B) is itself a bf16 value here
    gs = float(torch.tensor(1.0 / (S * B), dtype=torch.bfloat16)) * (S * B)
    gr = zf.grad * gs
    gerr = (z.grad.float() - gr).abs()
    bound = gr.abs() * (2.0 ** -8 + 1e-5) + 4e-6 * gs / (S * B)
    assert bool((gerr <= bound).all()), float(gerr.max())


def test_large_logits_are_stable(gpu):
    """Rows with logits near +-3e4 (bf16) stay finite: the max is subtracted."""
    V = 4099
    z = seeded((8, V), 41, std=1.0)
    z[:, 17] = 3.0e4
    z[4:] -= 3.0e4
    t = torch.tensor([17, 0, 5, 17, 17, 1, 2, 3])
    dl = torch.ones(8, dtype=torch.bfloat16)
    loss, grad = _run(z.to(gpu), t.to(gpu), dl.to(gpu))
    assert bool(torch.isfinite(loss).all()) and bool(torch.isfinite(grad).all())
    ref_loss, _ = cross_entropy_forward(z.double().numpy(), t.numpy())
    ref_grad = cross_entropy_backward(z.double().numpy(), t.numpy(), dl.double().numpy())
    _check("loss", loss, ref_loss, torch.bfloat16, 4e-6)
    np.testing.assert_allclose(grad.float().cpu().numpy(), ref_grad, atol=2.0 ** -8)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_minus_inf_logits(gpu, dtype):
    """-inf logits (masked vocabulary slots) in a row's scalar head, vector body
    and scalar tail: they contribute exp(-inf) = 0, the loss and the gradient
    stay finite and match the oracle.  Rows start at odd 2-byte offsets (a
    [S, B, V] slice), so every row has a head and a tail; one row has -inf as the
    first element a thread sees."""
    rows, V = 6, 1003
    base = seeded((rows, V + 5), 701, std=2.0, dtype=dtype)
    z = base[:, 3:3 + V].clone()
    ninf = float("-inf")
    z[0, 0] = ninf          # first element of the row (scalar head)
    z[1, V - 1] = ninf      # last element (scalar tail)
    z[2, 500:520] = ninf    # inside the vector body
    z[3, :8] = ninf         # several head elements
    z[4, ::7] = ninf        # spread over every part
    buf = torch.zeros(rows, V + 5, dtype=dtype)
    buf[:, 3:3 + V] = z
    t = torch.tensor([5, 6, 7, 9, 10, 11])
    dl = seeded((rows,), 702, dtype=dtype)
    zg = buf.to(gpu)[:, 3:3 + V]
    loss, grad = _run(zg, t.to(gpu), dl.to(gpu))
    assert torch.isfinite(loss).all() and torch.isfinite(grad).all()
    ref_loss, _ = cross_entropy_forward(z.double().numpy(), t.numpy())
    ref_grad = cross_entropy_backward(z.double().numpy(), t.numpy(), dl.double().numpy())
    _check("loss", loss, ref_loss, dtype, 4e-6)
    _check("grad", grad, ref_grad, dtype, 4e-6 * np.abs(dl.double().numpy())[:, None])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("rows,V", [(5, 1027), (3, 1024), (17, 2053), (2, 4096)])
def test_dense_rows_flat_backward(gpu, dtype, rows, V):
    """Dense rows of a vocabulary >= 1024 take the backward's flat path (the
    matrix as one run of 16-byte vectors): vectors that straddle a row boundary,
    the last n % 8 (or n % 4) elements, masked targets (-1, V, -100) and a
    target on a row's first and last element, out of place and in place."""
    z = seeded((rows, V), 801 + V, std=2.0, dtype=dtype)
    t = torch.randint(0, V, (rows,), generator=torch.Generator().manual_seed(V + rows))
    t[0] = 0
    t[-1] = V - 1
    if rows > 2:
        t[1] = -1
        t[2] = V
    if rows > 4:
        t[3] = -100
    dl = seeded((rows,), 802, dtype=dtype)
    ref_grad = cross_entropy_backward(z.double().numpy(), t.numpy(), dl.double().numpy())
    floor = 4e-6 * np.abs(dl.double().numpy())[:, None]
    _, grad = _run(z.to(gpu), t.to(gpu), dl.to(gpu))
    _check("grad", grad, ref_grad, dtype, floor)
    _, grad_in = _run(z.to(gpu), t.to(gpu), dl.to(gpu), inplace=True)
    assert torch.equal(grad_in, grad)
