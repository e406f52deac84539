"""GPU parity of the fused SwiGLU (mi_swiglu_fwd / mi_swiglu_bwd) against the
float64 oracle (oracle/mlp.py) on the same rounded inputs, and against the
reference's own torch ops on the GPU.

Tolerances (u = unit roundoff of the dtype: 2^-8 bf16, 2^-11 fp16): the kernel
rounds silu(g) to the dtype as torch does; its fp32 silu may differ from the
float64 one in the last bits and move that rounding, so h and d_up are within
3u |ref| (one flip, 2u, plus the final rounding, u); d_g = round(round(dh u)
silu'(g)) within u + 1e-5 relative, plus 1e-6 |d_s| (1 + |g|) absolute:
silu'(g) = sig (1 + g (1 - sig)) cancels near g = -1.28, where its fp32 error is
absolute.  At least 99% of the 16-bit outputs must equal the oracle's rounded
value exactly.  fp32 outputs within 1e-5 relative (plus that floor).
"""


def _dgate_floor(gu, dh, dtype):
    """1e-6 |round(dh u)| (1 + |g|) for the d_gate half."""
    inter = gu.shape[-1] // 2
    g, u = gu[..., :inter], gu[..., inter:]
    ds = dh * u
    if dtype != torch.float32:
        ds = torch.from_numpy(ds).to(dtype).double().numpy()
    return 1e-6 * np.abs(ds) * (1 + np.abs(g))
import numpy as np
import pytest
import torch

from gpu_ref import seeded
from oracle import swiglu_backward, swiglu_forward

pytestmark = pytest.mark.gpu

U = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11, torch.float32: 0.0}
TINY = {torch.bfloat16: 1e-30, torch.float16: 2.0 ** -22, torch.float32: 1e-30}


def _np(t):
    return t.detach().float().cpu().double().numpy()


def _close(name, got, ref, dtype, k_u, floor=0.0):
    g = _np(got)
    bound = np.abs(ref) * (k_u * U[dtype] + 1e-5) + TINY[dtype] + floor
    bad = np.abs(g - ref) > bound
    assert not bad.any(), f"{name}: {int(bad.sum())} elements out of bound, worst {np.abs(g - ref).max():.3e}"
    if dtype != torch.float32:
        exact = torch.from_numpy(ref).to(dtype).double().numpy()
        frac = np.mean(g == exact)
        assert frac >= 0.99, f"{name}: only {frac:.4f} exact"


def _run(gu, dh):
    from gpt_from_scratch_amd import swiglu
    x = gu.detach().clone().requires_grad_(True)
    h = swiglu(x)
    h.backward(dh)
    return h, x.grad


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("rows,inter", [(64, 3072), (7, 8), (5, 12), (33, 1000), (3, 5)])
def test_matches_oracle(gpu, dtype, rows, inter):
    gu = seeded((rows, 2 * inter), 40 + inter, std=2.0, dtype=dtype)
    dh = seeded((rows, inter), 41 + inter, dtype=dtype)
    h, dgu = _run(gu.to(gpu), dh.to(gpu))
    assert h.shape == (rows, inter) and dgu.shape == gu.shape
    rd = None if dtype == torch.float32 else dtype
    ref_h = swiglu_forward(_np(gu), rd)
    ref_d = swiglu_backward(_np(gu), _np(dh), rd)
    _close("h", h, ref_h, dtype, 3)
    _close("d_gate", dgu[:, :inter], ref_d[:, :inter], dtype, 1,
           _dgate_floor(_np(gu), _np(dh), dtype))
    _close("d_up", dgu[:, inter:], ref_d[:, inter:], dtype, 3)


def test_strided_rows(gpu):
    """gate_up as a slice of a wider buffer: 16-byte aligned rows (vector path)
    and 2-byte offset rows (scalar path)."""
    inter = 256
    for pad, off in ((8, 0), (3, 1)):
        wide = seeded((20, 2 * inter + pad), 50 + pad, std=2.0).to(gpu)
        gu = wide[:, off:off + 2 * inter]
        dh = seeded((20, inter), 51).to(gpu)
        h, dgu = _run(gu, dh)
        _close("h", h, swiglu_forward(_np(gu), torch.bfloat16), torch.bfloat16, 3)
        ref_d = swiglu_backward(_np(gu), _np(dh), torch.bfloat16)
        _close("d_gate", dgu[:, :inter], ref_d[:, :inter], torch.bfloat16, 1,
               _dgate_floor(_np(gu), _np(dh), torch.bfloat16))
        _close("d_up", dgu[:, inter:], ref_d[:, inter:], torch.bfloat16, 3)


def test_reference_ops_at_config5_shape(gpu):
    """core/mlp.py:25-28 in torch (bf16, on the GPU) at [1024, 8, 2 * 3072]."""
    g = torch.Generator(device=gpu).manual_seed(5)
    gu = (torch.randn(1024, 8, 6144, generator=g, device=gpu) * 2).to(torch.bfloat16)
    dh = torch.randn(1024, 8, 3072, generator=g, device=gpu).to(torch.bfloat16)
    h, dgu = _run(gu, dh)
    x = gu.detach().clone().requires_grad_(True)
    gate, up = x.chunk(2, dim=-1)
    ref = torch.nn.functional.silu(gate) * up
    ref.backward(dh)
    for got, want in ((h.detach(), ref.detach()), (dgu, x.grad)):
        eq = float((got == want).float().mean())
        assert eq >= 0.99, eq
        rel = ((got.float() - want.float()).abs() / want.float().abs().clamp_min(1e-30))
        assert float(rel.max()) <= 3 * 2 ** -8 + 1e-5


def test_more_rows_than_one_grid_column(gpu):
    """70000 rows: the row dimension of the grid is capped at 65535 and loops."""
    gu = seeded((70000, 32), 71, std=2.0)
    dh = seeded((70000, 16), 72)
    h, dgu = _run(gu.to(gpu), dh.to(gpu))
    _close("h", h, swiglu_forward(_np(gu), torch.bfloat16), torch.bfloat16, 3)
    ref_d = swiglu_backward(_np(gu), _np(dh), torch.bfloat16)
    _close("d_gate", dgu[:, :16], ref_d[:, :16], torch.bfloat16, 1,
           _dgate_floor(_np(gu), _np(dh), torch.bfloat16))
    _close("d_up", dgu[:, 16:], ref_d[:, 16:], torch.bfloat16, 3)


def test_row_broadcast_gradient(gpu):
    """dh with a stride-0 row axis (the gradient of (h.sum(0) * c).sum()): copied
    before the kernel, not refused by the C ABI."""
    rows, inter = 9, 3072
    gu = seeded((rows, 2 * inter), 601, std=2.0, dtype=torch.bfloat16)
    c = seeded((inter,), 602, dtype=torch.bfloat16)
    from gpt_from_scratch_amd import swiglu
    x = gu.to(gpu).requires_grad_(True)
    (swiglu(x).sum(0) * c.to(gpu)).sum().backward()
    dh = c.expand(rows, inter)
    ref_d = swiglu_backward(_np(gu), _np(dh), torch.bfloat16)
    _close("d_gate", x.grad[:, :inter], ref_d[:, :inter], torch.bfloat16, 1,
           _dgate_floor(_np(gu), _np(dh), torch.bfloat16))
    _close("d_up", x.grad[:, inter:], ref_d[:, inter:], torch.bfloat16, 3)
