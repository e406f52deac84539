"""GPU parity of the RoPE kernel against the oracle (fp32 within 1e-3, here
much tighter; bf16 within one bf16 rounding of the fp32 result)."""
import pytest
import torch

from gpu_ref import rope_inputs, seeded
from oracle import rope_apply, rope_tables, rope_tables_f64

pytestmark = pytest.mark.gpu


def _bf16_ulp_ok(got, ref):
    """|got - ref| within one bf16 rounding step of ref (plus a denormal floor)."""
    got, ref = got.float().cpu(), ref.float().cpu()
    bound = ref.abs() * 2.0 ** -7 + 1e-30
    return bool(((got - ref).abs() <= bound).all())


def test_fp32_forward_and_inverse(gpu):
    from gpt_from_scratch_amd import apply_rope
    from gpt_from_scratch_amd.rope import RoPE
    S, B, H, D = 256, 1, 12, 64
    x = seeded((S, B, H, D), 1, dtype=torch.float32)
    cos, sin = rope_tables(D, S)
    y = apply_rope(x.to(gpu), cos.to(gpu), sin.to(gpu))
    ref = rope_apply(x, cos, sin)
    assert float((y.cpu().double() - ref).abs().max()) < 1e-5
    # against exact float64 angles the budget is 1e-3
    c64, s64 = rope_tables_f64(D, S)
    assert float((y.cpu().double() - rope_apply(x, c64, s64)).abs().max()) < 1e-3
    xg = x.to(gpu).requires_grad_()
    g = seeded((S, B, H, D), 2, dtype=torch.float32)
    RoPE.apply(xg, cos.to(gpu), sin.to(gpu)).backward(g.to(gpu))
    assert float((xg.grad.cpu().double() - rope_apply(g, cos, sin, inverse=True)).abs().max()) < 1e-5


def test_bf16_model_layout_qk(gpu):
    """q/k are strided views of a fused qkv [S,B,3,H,D]; bf16 tables (the model casts
    them to the activation dtype)."""
    from gpt_from_scratch_amd import apply_rope, apply_rope_qk
    q, k, v, cos, sin, _ = rope_inputs(8, 12, 1024, 64, 2, 1.0, torch.bfloat16, gpu)
    assert not q.is_contiguous()
    qr, kr = apply_rope_qk(q, k, cos, sin)
    assert qr.shape == q.shape and qr.is_contiguous()
    for x, y in ((q, qr), (k, kr)):
        ref = rope_apply(x.cpu(), cos.cpu(), sin.cpu(), dtype=torch.float32)
        assert _bf16_ulp_ok(y, ref)
    # one launch for both == two single launches, bit for bit
    assert torch.equal(qr, apply_rope(q, cos, sin))
    assert torch.equal(kr, apply_rope(k, cos, sin))


@pytest.mark.parametrize("B,H,S,D", [(1, 5, 37, 64), (3, 7, 19, 128), (1, 1, 1, 64)])
def test_vector_path_ragged_grid(gpu, B, H, S, D):
    """Vector-path sizes whose 16-byte items do not fill the last workgroup (each
    lane takes several items, 256 lanes per workgroup): every element is written
    and matches the oracle; the last workgroup's missing items touch nothing."""
    from gpt_from_scratch_amd import apply_rope_qk
    q, k, _, cos, sin, _ = rope_inputs(B, H, S, D, 40 + S, 1.0, torch.bfloat16, gpu)
    items = 2 * S * B * H * D // 8
    assert items % (256 * 2) and items % (256 * 3) and items % (256 * 4)
    qr, kr = apply_rope_qk(q, k, cos, sin)
    for x, y in ((q, qr), (k, kr)):
        ref = rope_apply(x.cpu(), cos.cpu(), sin.cpu(), dtype=torch.float32)
        assert _bf16_ulp_ok(y, ref)


def test_qk_backward_is_inverse_rotation(gpu):
    from gpt_from_scratch_amd import apply_rope_qk
    q, k, v, cos, sin, _ = rope_inputs(2, 4, 128, 64, 3, 1.0, torch.bfloat16, gpu)
    q = q.detach().requires_grad_()
    k = k.detach().requires_grad_()
    qr, kr = apply_rope_qk(q, k, cos, sin)
    gq = seeded(qr.shape, 4).to(gpu)
    gk = seeded(kr.shape, 5).to(gpu)
    (qr.float() * gq.float()).sum().add((kr.float() * gk.float()).sum()).backward()
    assert _bf16_ulp_ok(q.grad, rope_apply(gq.cpu(), cos.cpu(), sin.cpu(), True, torch.float32))
    assert _bf16_ulp_ok(k.grad, rope_apply(gk.cpu(), cos.cpu(), sin.cpu(), True, torch.float32))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_odd_layouts(gpu, dtype):
    """Scalar pair path: D not a multiple of the vector width, transposed tables,
    non-unit dim stride, S = 1, fp32 tables with 16-bit x."""
    from gpt_from_scratch_amd import apply_rope
    for S, B, H, D in ((5, 2, 3, 6), (1, 1, 1, 2), (17, 3, 5, 10)):
        x = seeded((S, B, H, D), S + D, dtype=dtype).to(gpu)
        cos, sin = rope_tables(D, S)
        for c, s in ((cos, sin), (cos.t().contiguous().t(), sin.t().contiguous().t())):
            y = apply_rope(x, c.to(gpu), s.to(gpu))
            ref = rope_apply(x.cpu(), c, s, dtype=torch.float32)
            if dtype == torch.float32:
                assert float((y.cpu() - ref).abs().max()) < 1e-5
            else:
                tol = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10
                assert float(((y.cpu().float() - ref).abs() - ref.abs() * tol).max()) <= 1e-6
    # non-unit dim stride: every other element of a wider tensor
    wide = seeded((8, 2, 2, 16), 99, dtype=dtype).to(gpu)
    x = wide[..., ::2]
    cos, sin = rope_tables(8, 8)
    y = apply_rope(x, cos.to(gpu), sin.to(gpu))
    ref = rope_apply(x.cpu(), cos, sin, dtype=torch.float32)
    tol = {torch.float32: 0.0, torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}[dtype]
    assert float(((y.cpu().float() - ref).abs() - ref.abs() * tol).max()) <= 1e-5


def test_table_layouts_vector_x(gpu):
    """x that qualifies for the 16-byte vector path with angle tables that do and do not:
    contiguous tables, tables whose rows are padded to an odd stride, and tables whose base
    is not aligned to the angle vector (the last two take the pair path).  All three compute
    the same fp32 rotation with one rounding, so they must agree bit for bit, and match the
    oracle to one bf16 rounding."""
    from gpt_from_scratch_amd import apply_rope_qk
    S, B, H, D = 64, 2, 3, 64
    qkv = seeded((S, B, 3, H, D), 21, dtype=torch.bfloat16).to(gpu)
    q, k, _ = qkv.unbind(2)
    cos, sin = (t.to(torch.bfloat16).to(gpu) for t in rope_tables(D, S))
    variants = {"contiguous": (cos, sin)}
    padded = []
    for t in (cos, sin):
        buf = torch.zeros(S, D // 2 + 1, dtype=torch.bfloat16, device=gpu)
        buf[:, : D // 2] = t
        padded.append(buf[:, : D // 2])
    variants["padded rows"] = tuple(padded)
    shifted = []
    for t in (cos, sin):
        buf = torch.zeros(S * (D // 2) + 1, dtype=torch.bfloat16, device=gpu)
        buf[1:] = t.reshape(-1)
        shifted.append(buf[1:].view(S, D // 2))
    variants["unaligned base"] = tuple(shifted)
    assert variants["padded rows"][0].stride(0) == D // 2 + 1
    assert variants["unaligned base"][0].data_ptr() % 8 != 0

    outs = {name: apply_rope_qk(q, k, c, s) for name, (c, s) in variants.items()}
    for name in ("padded rows", "unaligned base"):
        for got, want in zip(outs[name], outs["contiguous"]):
            assert torch.equal(got, want), name
    for got, x in zip(outs["contiguous"], (q, k)):
        assert _bf16_ulp_ok(got, rope_apply(x.cpu(), cos.cpu().float(), sin.cpu().float(),
                                            dtype=torch.float32))


def test_long_sequence_invariants(gpu):
    """C4 shape: inverse(forward(x)) == x to rounding, per-pair norms preserved."""
    from gpt_from_scratch_amd import apply_rope
    from gpt_from_scratch_amd.rope import RoPE
    S, B, H, D = 8192, 1, 32, 128
    x = seeded((S, B, H, D), 8, dtype=torch.float32).to(gpu)
    cos, sin = (t.to(gpu) for t in rope_tables(D, S))
    y = apply_rope(x, cos, sin)
    n0 = x[..., 0::2] ** 2 + x[..., 1::2] ** 2
    n1 = y[..., 0::2] ** 2 + y[..., 1::2] ** 2
    assert float(((n1 - n0).abs() / n0.clamp_min(1e-6)).max()) < 1e-5
    xg = y.detach().requires_grad_()
    RoPE.apply(xg, cos, sin).backward(torch.zeros_like(y))  # exercise the graph
    from gpt_from_scratch_amd import _lib
    back = torch.empty_like(y)
    _lib.rope(y, cos, sin, back, inverse=True)
    assert float((back - x).abs().max()) < 1e-5


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 64), (torch.float32, 64),
                                     (torch.bfloat16, 6)])
def test_in_place(gpu, dtype, D):
    """out == x (same pointer and strides) is allowed: the result equals the
    out-of-place rotation bit for bit, for mi_rope and for mi_rope_qk, on the
    vector path (D = 64) and the scalar pair path (D = 6)."""
    from gpt_from_scratch_amd import _lib
    S, B, H = 200, 2, 3
    qkv = seeded((S, B, 3, H, D), 33 + D, dtype=dtype).to(gpu)
    cos, sin = (t.to(dtype).to(gpu) for t in rope_tables(D, S))
    q, k, _ = qkv.unbind(2)
    for inverse in (False, True):
        want_q, want_k = torch.empty_like(q), torch.empty_like(k)
        _lib.rope_qk(q, k, cos, sin, want_q, want_k, inverse)
        x = qkv.clone()
        xq, xk, _ = x.unbind(2)
        _lib.rope_qk(xq, xk, cos, sin, xq, xk, inverse)
        assert torch.equal(xq, want_q) and torch.equal(xk, want_k)
        y = qkv.clone()
        yq = y[:, :, 0]
        _lib.rope(yq, cos, sin, yq, inverse)
        assert torch.equal(yq, want_q)
        assert torch.equal(y[:, :, 1:], qkv[:, :, 1:])  # nothing else touched


@pytest.mark.parametrize("dtype,B,H,S,D", [(torch.bfloat16, 8, 12, 1024, 64),
                                           (torch.bfloat16, 1, 5, 37, 64),
                                           (torch.float32, 3, 7, 19, 128)])
def test_copy_qk_is_the_relayout(gpu, dtype, B, H, S, D):
    """mi_copy_qk (RoPE's launch without the rotation) writes exactly the dense
    copies of the strided q/k views, ragged last workgroup included, and leaves
    the bytes around its outputs alone; layouts it cannot stream are refused."""
    import ctypes
    from gpt_from_scratch_amd import _lib
    lib = _lib.lib()
    q, k, _, _, _, _ = rope_inputs(B, H, S, D, 60 + S, 1.0, dtype, gpu)
    pad = torch.full((2, S * B * H * D + 64), 7.0, dtype=dtype, device=gpu)
    outq = pad[0, :S * B * H * D].view(S, B, H, D)
    outk = pad[1, :S * B * H * D].view(S, B, H, D)
    st = lambda t: _lib._strides(t, 4)
    dt = _lib.dtype_code(q)
    r = lib.mi_copy_qk(dt, S, B, H, D, _lib._ptr(q), st(q), _lib._ptr(k), st(k),
                       _lib._ptr(outq), st(outq), _lib._ptr(outk), st(outk), _lib._stream(q))
    assert r == 0, lib.mi_last_error()
    torch.cuda.synchronize()
    assert torch.equal(outq, q) and torch.equal(outk, k)
    assert bool((pad[:, S * B * H * D:] == 7.0).all())
    # a row that is not a multiple of 16 bytes cannot take the 16-byte path
    bad = torch.zeros(S, B, H, 4, dtype=torch.bfloat16, device=gpu)
    r = lib.mi_copy_qk(2, S, B, H, 4, _lib._ptr(bad), st(bad), _lib._ptr(bad), st(bad),
                       _lib._ptr(bad), st(bad), _lib._ptr(bad), st(bad), _lib._stream(bad))
    assert r == 2 and b"16" in lib.mi_last_error()
