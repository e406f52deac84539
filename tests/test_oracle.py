"""Pins of the CPU oracle (runs without a GPU).

Every check here compares the oracle against something it does not share code
with: autograd, finite differences, pure-Python loops, closed-form special
cases, algebraic invariants.  A dropped term, a wrong sign, a transposed operand
or a wrong scale in oracle/ fails at least one of them.
"""
import math

import numpy as np
import pytest
import torch

from oracle import (attention_backward, attention_bruteforce, attention_forward,
                    attention_forward_backward_chunked, attention_probs, rope_apply, rope_tables,
                    rope_tables_f64)


def _randn(*shape, seed=0, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float64) * std


@pytest.mark.parametrize("causal", [True, False])
def test_forward_matches_bruteforce(causal):
    S, D = 9, 6
    q, k, v = (_randn(S, D, seed=s) for s in (1, 2, 3))
    o, lse = attention_forward(q, k, v, causal)
    ob, lb = attention_bruteforce(q, k, v, causal)
    assert torch.allclose(o, torch.tensor(ob, dtype=torch.float64), atol=1e-12)
    assert torch.allclose(lse, torch.tensor(lb, dtype=torch.float64), atol=1e-12)


def test_forward_matches_torch_sdpa_math():
    # torch's own math-path attention on the CPU: an independent implementation.
    q, k, v = (_randn(2, 3, 17, 8, seed=s) for s in (4, 5, 6))
    o, _ = attention_forward(q, k, v, True)
    ref = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True)
    assert torch.allclose(o, ref, atol=1e-12)
    o2, _ = attention_forward(q, k, v, False)
    ref2 = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=False)
    assert torch.allclose(o2, ref2, atol=1e-12)


def test_causal_row0_is_v0_and_s1_is_identity():
    q, k, v = (_randn(1, 2, 12, 8, seed=s) for s in (7, 8, 9))
    o, lse = attention_forward(q, k, v, True)
    assert torch.allclose(o[..., 0, :], v[..., 0, :], atol=1e-14)
    # lse of row 0 is the single scaled score
    assert torch.allclose(lse[..., 0], (q[..., 0, :] * k[..., 0, :]).sum(-1) / math.sqrt(8))
    o1, _ = attention_forward(q[..., :1, :], k[..., :1, :], v[..., :1, :], False)
    assert torch.allclose(o1, v[..., :1, :], atol=1e-14)


def test_zero_query_gives_prefix_means_and_log_counts():
    S, D = 16, 8
    q = torch.zeros(S, D, dtype=torch.float64)
    k, v = _randn(S, D, seed=10), _randn(S, D, seed=11)
    o, lse = attention_forward(q, k, v, True)
    prefix_mean = torch.cumsum(v, 0) / torch.arange(1, S + 1, dtype=torch.float64)[:, None]
    assert torch.allclose(o, prefix_mean, atol=1e-13)
    assert torch.allclose(lse, torch.log(torch.arange(1, S + 1, dtype=torch.float64)), atol=1e-13)
    o2, lse2 = attention_forward(q, k, v, False)
    assert torch.allclose(o2, v.mean(0).expand(S, D), atol=1e-13)
    assert torch.allclose(lse2, torch.full((S,), math.log(S), dtype=torch.float64), atol=1e-13)


def test_dominant_key_selects_its_value():
    S, D = 8, 4
    q = torch.zeros(S, D, dtype=torch.float64)
    q[:, 0] = 1.0
    k = torch.zeros(S, D, dtype=torch.float64)
    k[3, 0] = 400.0  # scaled score 200 for key 3, 0 elsewhere
    v = _randn(S, D, seed=12)
    o, _ = attention_forward(q, k, v, False)
    assert torch.allclose(o, v[3].expand(S, D), atol=1e-12)
    oc, _ = attention_forward(q, k, v, True)
    assert torch.allclose(oc[3:], v[3].expand(S - 3, D), atol=1e-12)
    # rows before 3 cannot see key 3: they average the visible prefix
    for i in range(3):
        assert torch.allclose(oc[i], v[: i + 1].mean(0), atol=1e-12)


def test_identical_keys_average_the_values():
    """Non-causal with every key equal: all scores of a row tie, so each output
    row is the plain mean of V and LSE = s + ln(S) for the common score s."""
    S, D = 10, 8
    q = _randn(S, D, seed=13)
    k = _randn(1, D, seed=14).expand(S, D).clone()
    v = _randn(S, D, seed=15)
    o, lse = attention_forward(q, k, v, False)
    assert torch.allclose(o, v.mean(0).expand(S, D), atol=1e-12)
    s = (q @ k[0]) / math.sqrt(D)
    assert torch.allclose(lse, s + math.log(S), atol=1e-12)


@pytest.mark.parametrize("causal", [True, False])
def test_closed_form_backward_matches_autograd(causal):
    q, k, v = (_randn(2, 2, 13, 8, seed=s).requires_grad_() for s in (13, 14, 15))
    do = _randn(2, 2, 13, 8, seed=16)
    o, _ = attention_forward(q, k, v, causal)
    gq, gk, gv = torch.autograd.grad(o, (q, k, v), do)
    dq, dk, dv, delta = attention_backward(q.detach(), k.detach(), v.detach(), do, causal)
    assert torch.allclose(dq, gq, atol=1e-12)
    assert torch.allclose(dk, gk, atol=1e-12)
    assert torch.allclose(dv, gv, atol=1e-12)
    assert torch.allclose(delta, (do * o.detach()).sum(-1), atol=1e-12)


def test_backward_finite_differences():
    S, D = 6, 4
    q, k, v = (_randn(S, D, seed=s) for s in (17, 18, 19))
    do = _randn(S, D, seed=20)
    dq, dk, dv, _ = attention_backward(q, k, v, do, True)
    eps = 1e-6

    def loss(args):
        return float((attention_forward(args["q"], args["k"], args["v"], True)[0] * do).sum())

    base = {"q": q, "k": k, "v": v}
    for name, g in (("q", dq), ("k", dk), ("v", dv)):
        for idx in [(0, 0), (2, 3), (5, 1), (3, 2)]:
            plus, minus = dict(base), dict(base)
            plus[name] = base[name].clone()
            minus[name] = base[name].clone()
            plus[name][idx] += eps
            minus[name][idx] -= eps
            fd = (loss(plus) - loss(minus)) / (2 * eps)
            assert abs(fd - float(g[idx])) < 1e-7, (name, idx, fd, float(g[idx]))


def test_ds_rows_sum_to_zero_and_delta_identity():
    q, k, v = (_randn(1, 1, 20, 8, seed=s) for s in (21, 22, 23))
    do = _randn(1, 1, 20, 8, seed=24)
    p = attention_probs(q, k, True)
    dp = do @ v.transpose(-1, -2)
    _, _, _, delta = attention_backward(q, k, v, do, True)
    assert torch.allclose(delta, (p * dp).sum(-1), atol=1e-12)
    ds = p * (dp - delta[..., None])
    assert torch.allclose(ds.sum(-1), torch.zeros_like(delta), atol=1e-12)
    # dV column sums: sum_j dV_j = sum_i dO_i (each P row sums to 1)
    _, _, dv, _ = attention_backward(q, k, v, do, True)
    assert torch.allclose(dv.sum(-2), do.sum(-2), atol=1e-12)


def test_chunked_matches_batched():
    q, k, v, do = (_randn(2, 3, 32, 8, seed=s) for s in (25, 26, 27, 28))
    out = attention_forward_backward_chunked(q, k, v, do, True, dtype=torch.float64)
    o, lse = attention_forward(q, k, v, True)
    dq, dk, dv, delta = attention_backward(q, k, v, do, True)
    for a, b in ((out["o"], o), (out["lse"], lse), (out["dq"], dq), (out["dk"], dk),
                 (out["dv"], dv), (out["delta"], delta)):
        assert torch.allclose(a, b, atol=1e-12)


# ------------------------------------------------------------------ RoPE


def test_rope_tables_match_float64_angles():
    c32, s32 = rope_tables(64, 1024)
    c64, s64 = rope_tables_f64(64, 1024)
    # fp32 angle rounding at s ~ 1000 is ~6e-5 rad; tables agree to that level
    assert float((c32.double() - c64).abs().max()) < 2e-4
    assert float((s32.double() - s64).abs().max()) < 2e-4
    # theta_i = 10000^(-2i/D): i = 0 is 1 rad / position, i = D/2-1 is the slowest
    assert torch.allclose(c64[:, 0], torch.cos(torch.arange(1024, dtype=torch.float64)))
    ang = math.pow(10000.0, -62.0 / 64.0)
    assert torch.allclose(s64[:, 31], torch.sin(torch.arange(1024, dtype=torch.float64) * ang))


def test_rope_is_complex_multiplication():
    S, B, H, D = 10, 2, 3, 8
    x = _randn(S, B, H, D, seed=29)
    c, s = rope_tables_f64(D, S)
    out = rope_apply(x, c, s)
    z = torch.complex(x[..., 0::2], x[..., 1::2])
    ang = torch.atan2(s, c)[:, None, None, :]
    w = z * torch.exp(1j * ang)
    assert torch.allclose(out[..., 0::2], w.real, atol=1e-12)
    assert torch.allclose(out[..., 1::2], w.imag, atol=1e-12)


def test_rope_invariants():
    S, B, H, D = 12, 1, 2, 16
    x = _randn(S, B, H, D, seed=30)
    c, s = rope_tables_f64(D, S)
    y = rope_apply(x, c, s)
    # pair norms preserved
    assert torch.allclose(y[..., 0::2] ** 2 + y[..., 1::2] ** 2,
                          x[..., 0::2] ** 2 + x[..., 1::2] ** 2, atol=1e-12)
    # inverse undoes forward
    assert torch.allclose(rope_apply(y, c, s, inverse=True), x, atol=1e-12)
    # position 0 is the identity
    assert torch.allclose(y[0], x[0], atol=1e-14)
    # relative-position property: <R_m q, R_n k> depends only on m - n
    q = _randn(D, seed=31)
    k = _randn(D, seed=32)
    qs = rope_apply(q.expand(S, 1, 1, D).clone(), c, s)[:, 0, 0]
    ks = rope_apply(k.expand(S, 1, 1, D).clone(), c, s)[:, 0, 0]
    dots = qs @ ks.T
    for m in range(3, S):
        assert abs(float(dots[m, m - 3] - dots[3, 0])) < 1e-10


def test_rope_gradient_is_inverse_rotation():
    S, B, H, D = 5, 2, 2, 8
    x = _randn(S, B, H, D, seed=33).requires_grad_()
    c, s = rope_tables_f64(D, S)
    g = _randn(S, B, H, D, seed=34)
    (gx,) = torch.autograd.grad(rope_apply(x, c, s), x, g)
    assert torch.allclose(gx, rope_apply(g, c, s, inverse=True), atol=1e-12)


# ---- vocabulary cross entropy (oracle/cross_entropy.py) ----

def _xent_inputs(rows=12, V=37, seed=3):
    rng = np.random.default_rng(seed)
    z = rng.normal(0.0, 3.0, size=(rows, V))
    t = rng.integers(0, V, size=rows)
    return z, t


def test_xent_matches_scipy_logsumexp():
    from scipy.special import logsumexp
    from oracle import cross_entropy_forward
    z, t = _xent_inputs()
    loss, lse = cross_entropy_forward(z, t)
    ref_lse = logsumexp(z, axis=-1)
    np.testing.assert_allclose(lse, ref_lse, rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(loss, ref_lse - z[np.arange(len(t)), t], rtol=1e-12, atol=1e-12)


def test_xent_uniform_logits_give_log_vocab_and_shift_invariance():
    from oracle import cross_entropy_forward
    V = 50257
    loss, _ = cross_entropy_forward(np.full((3, V), 7.25), np.array([0, 5, V - 1]))
    np.testing.assert_allclose(loss, math.log(V), rtol=1e-13)
    z, t = _xent_inputs()
    shift = np.linspace(-1e3, 1e3, z.shape[0])[:, None]
    np.testing.assert_allclose(cross_entropy_forward(z + shift, t)[0],
                               cross_entropy_forward(z, t)[0], rtol=1e-9, atol=1e-9)


def test_xent_masked_target_semantics():
    """loss.py:33-41: an out-of-range target contributes a shifted logit of 0,
    so the loss is log(sum exp(z - max)) = lse - max, and the gradient is the
    plain softmax."""
    from oracle import cross_entropy_backward, cross_entropy_forward
    z, t = _xent_inputs(rows=4)
    t = np.array([-1, 37, -100, 2])
    loss, lse = cross_entropy_forward(z, t)
    np.testing.assert_allclose(loss[:3], (lse - z.max(-1))[:3], rtol=1e-13)
    g = cross_entropy_backward(z, t, np.ones(4))
    p = np.exp(z - lse[:, None])
    np.testing.assert_allclose(g[:3], p[:3], rtol=1e-12, atol=1e-15)
    assert abs(g[3].sum()) < 1e-12 and g[3, 2] < 0


def test_xent_gradient_is_finite_difference():
    from oracle import cross_entropy_backward, cross_entropy_forward
    z, t = _xent_inputs(rows=3, V=11)
    w = np.array([0.5, -1.25, 2.0])  # d(sum_r w_r loss_r) / dz
    g = cross_entropy_backward(z, t, w)
    eps = 1e-6
    fd = np.zeros_like(z)
    for r in range(z.shape[0]):
        for j in range(z.shape[1]):
            zp, zm = z.copy(), z.copy()
            zp[r, j] += eps
            zm[r, j] -= eps
            fd[r, j] = (w @ cross_entropy_forward(zp, t)[0] - w @ cross_entropy_forward(zm, t)[0]) / (2 * eps)
    np.testing.assert_allclose(g, fd, rtol=1e-6, atol=1e-8)
    # rows with an in-range target sum to zero
    np.testing.assert_allclose(g.sum(-1), 0.0, atol=1e-12)


# ---- RMSNorm (oracle/normalization.py) ----

def test_rmsnorm_matches_torch_autograd_float64():
    from oracle import rmsnorm_backward, rmsnorm_forward
    g = torch.Generator().manual_seed(7)
    x = torch.randn(5, 3, 24, generator=g, dtype=torch.float64)
    w = torch.randn(24, generator=g, dtype=torch.float64)
    dy = torch.randn(5, 3, 24, generator=g, dtype=torch.float64)
    eps = 1e-6
    xr, wr = x.clone().requires_grad_(True), w.clone().requires_grad_(True)
    # torch's own ops, no rounding (x is float64)
    y = xr * torch.rsqrt(xr.pow(2).mean(-1, keepdim=True) + eps) * wr
    y.backward(dy)
    yo, _ = rmsnorm_forward(x.numpy(), w.numpy(), eps)
    dx, dw = rmsnorm_backward(x.numpy(), w.numpy(), dy.numpy(), eps)
    np.testing.assert_allclose(yo, y.detach().numpy(), rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(dx, xr.grad.numpy(), rtol=1e-11, atol=1e-12)
    np.testing.assert_allclose(dw, wr.grad.numpy(), rtol=1e-11, atol=1e-12)


def test_rmsnorm_finite_differences_and_invariants():
    from oracle import rmsnorm_backward, rmsnorm_forward
    rng = np.random.default_rng(8)
    x = rng.normal(size=(2, 9))
    w = rng.normal(size=9)
    dy = rng.normal(size=(2, 9))
    eps = 1e-3
    dx, dw = rmsnorm_backward(x, w, dy, eps)
    h = 1e-6
    fdx = np.zeros_like(x)
    for i in range(2):
        for j in range(9):
            xp, xm = x.copy(), x.copy()
            xp[i, j] += h
            xm[i, j] -= h
            fdx[i, j] = ((rmsnorm_forward(xp, w, eps)[0] - rmsnorm_forward(xm, w, eps)[0]) * dy).sum() / (2 * h)
    np.testing.assert_allclose(dx, fdx, rtol=1e-6, atol=1e-8)
    fdw = np.array([((rmsnorm_forward(x, w + h * np.eye(9)[j], eps)[0]
                      - rmsnorm_forward(x, w - h * np.eye(9)[j], eps)[0]) * dy).sum() / (2 * h)
                    for j in range(9)])
    np.testing.assert_allclose(dw, fdw, rtol=1e-6, atol=1e-8)
    # scale invariance (eps = 0) and x . dx = 0 for w = 1, eps = 0
    y1, _ = rmsnorm_forward(x, w, 0.0)
    y2, _ = rmsnorm_forward(37.5 * x, w, 0.0)
    np.testing.assert_allclose(y1, y2, rtol=1e-13)
    dx0, _ = rmsnorm_backward(x, np.ones(9), dy, 0.0)
    np.testing.assert_allclose((dx0 * x).sum(-1), 0.0, atol=1e-12)
    # a constant row a: n = a / sqrt(a^2 + eps)
    yc, _ = rmsnorm_forward(np.full((1, 16), -0.25), np.ones(16), eps)
    np.testing.assert_allclose(yc, -0.25 / math.sqrt(0.0625 + eps), rtol=1e-14)


def test_rmsnorm_rounds_n_to_the_input_dtype_before_the_weight():
    """normalization.py:23-24: y = bf16(n) * w, not n * w."""
    from oracle import rmsnorm_forward
    x = np.array([[1.0, 1.0 + 2.0 ** -6, 0.5, 3.0]])
    w = np.full(4, 1.0 + 2.0 ** -7)  # exactly representable in bf16
    y_round, r = rmsnorm_forward(x, w, 0.0, x_dtype=torch.bfloat16)
    n = x * r[:, None]
    nb = torch.from_numpy(n).to(torch.bfloat16).double().numpy()
    np.testing.assert_array_equal(y_round, nb * w)
    assert not np.array_equal(y_round, n * w)


# ---- SwiGLU (oracle/mlp.py) ----

def test_swiglu_matches_torch_float64_and_autograd():
    from oracle import swiglu_backward, swiglu_forward
    g = torch.Generator().manual_seed(21)
    gu = (torch.randn(6, 2 * 10, generator=g, dtype=torch.float64) * 3).requires_grad_(True)
    gate, up = gu.chunk(2, dim=-1)
    h = torch.nn.functional.silu(gate) * up
    dh = torch.randn(6, 10, generator=g, dtype=torch.float64)
    h.backward(dh)
    np.testing.assert_allclose(swiglu_forward(gu.detach().numpy()), h.detach().numpy(),
                               rtol=1e-14, atol=1e-15)
    np.testing.assert_allclose(swiglu_backward(gu.detach().numpy(), dh.numpy()),
                               gu.grad.numpy(), rtol=1e-12, atol=1e-14)


def test_swiglu_closed_forms_and_finite_differences():
    from oracle import swiglu_backward, swiglu_forward
    gu = np.array([[0.0, 40.0, -40.0, 2.0, 3.0, -1.5]])
    h = swiglu_forward(gu)
    np.testing.assert_allclose(h[0], [0.0, 40.0 * 3.0, -40.0 * np.exp(-40.0) * -1.5], rtol=1e-12,
                               atol=1e-300)
    rng = np.random.default_rng(22)
    x = rng.normal(size=(3, 8)) * 2
    dh = rng.normal(size=(3, 4))
    grad = swiglu_backward(x, dh)
    eps = 1e-6
    fd = np.zeros_like(x)
    for i in range(3):
        for j in range(8):
            xp, xm = x.copy(), x.copy()
            xp[i, j] += eps
            xm[i, j] -= eps
            fd[i, j] = ((swiglu_forward(xp) - swiglu_forward(xm)) * dh).sum() / (2 * eps)
    np.testing.assert_allclose(grad, fd, rtol=1e-6, atol=1e-9)


def test_swiglu_rounds_silu_before_the_product():
    from oracle import swiglu_forward
    g = torch.tensor([1.3, 0.7, 2.9, -0.4], dtype=torch.bfloat16).double()
    u = torch.tensor([1.01, 3.3, 0.51, 7.7], dtype=torch.bfloat16).double()
    gu = torch.cat([g, u]).numpy()[None]
    ref = (torch.nn.functional.silu(g.to(torch.bfloat16)) * u.to(torch.bfloat16)).double().numpy()
    got = torch.from_numpy(swiglu_forward(gu, torch.bfloat16)).to(torch.bfloat16).double().numpy()
    np.testing.assert_array_equal(got[0], ref)


# ---- optimizer step (oracle/optimizer.py) ----

def test_adamw_matches_torch_adamw_float64():
    from oracle import adamw_step
    g = torch.Generator().manual_seed(31)
    p0 = torch.randn(50, generator=g, dtype=torch.float64)
    ref = p0.clone().requires_grad_(True)
    opt = torch.optim.AdamW([ref], lr=3e-3, betas=(0.9, 0.95), weight_decay=0.1, eps=1e-8)
    p, m, v = p0.numpy(), np.zeros(50), np.zeros(50)
    for t in range(1, 6):
        grad = torch.randn(50, generator=g, dtype=torch.float64)
        ref.grad = grad.clone()
        opt.step()
        p, m, v = adamw_step(p, m, v, grad.numpy(), t, 3e-3, (0.9, 0.95), 1e-8, 0.1)
        np.testing.assert_allclose(p, ref.detach().numpy(), rtol=1e-13, atol=1e-15)
        np.testing.assert_allclose(m, opt.state[ref]["exp_avg"].numpy(), rtol=1e-13)
        np.testing.assert_allclose(v, opt.state[ref]["exp_avg_sq"].numpy(), rtol=1e-13)


def test_adamw_first_step_is_signed_lr_and_clip_scales_to_threshold():
    from oracle import adamw_step, clip_gradient
    grad = np.array([3.0, -0.02, 1e-3, -7.0])
    p, _, _ = adamw_step(np.zeros(4), np.zeros(4), np.zeros(4), grad, 1, 1e-2, (0.9, 0.95),
                         1e-12, 0.0)
    np.testing.assert_allclose(p, -1e-2 * np.sign(grad), rtol=1e-8)
    gc, norm = clip_gradient(grad, 1.0)
    assert abs(norm - np.sqrt((grad ** 2).sum())) < 1e-12
    np.testing.assert_allclose(np.sqrt((gc ** 2).sum()), 1.0 * norm / (norm + 1e-6), rtol=1e-12)
    g2, _ = clip_gradient(grad * 1e-3, 1.0)
    np.testing.assert_array_equal(g2, grad * 1e-3)  # below the threshold: unchanged


@pytest.mark.parametrize("causal", [True, False])
def test_grad_rounding_budget_admits_reference_rounding_rejects_mistakes(causal):
    """The gradient budget of the GPU rescale-stress test (gpu_ref.grad_rounding_budget)
    is neither vacuous nor too tight: a CPU restatement that rounds where the
    reference does (bf16 P before dV, bf16 scale*dS before dQ/dK, delta from the
    bf16 O; core/myFlashAttn.py:1049, :1055, :1308) stays inside it, and four
    plausible mistakes fall outside it."""
    from gpu_ref import budget_ratio, grad_rounding_budget, rescale_stress_inputs
    S, D = 256, 64
    q, k, v, do = rescale_stress_inputs(S, D)
    qf, kf, vf, dof = (t.float() for t in (q, k, v, do))
    sc = 1.0 / math.sqrt(D)
    mask = torch.ones(S, S, dtype=torch.bool).triu(1) if causal else torch.zeros(S, S, dtype=torch.bool)
    p = torch.softmax(((qf @ kf.transpose(-1, -2)) * sc).masked_fill(mask, float("-inf")), -1)
    o = (p @ vf).to(torch.bfloat16)
    want, budget = grad_rounding_budget(q, k, v, do, o, causal)
    bf = lambda t: t.to(torch.bfloat16).float()
    dp = dof @ vf.transpose(-1, -2)
    delta = (dof * o.float()).sum(-1, keepdim=True)
    ds = bf(p * (dp - delta) * sc)
    emul = {"dq": bf(ds @ kf), "dk": bf(ds.transpose(-1, -2) @ qf),
            "dv": bf(bf(p).transpose(-1, -2) @ dof)}
    for n in ("dq", "dk", "dv"):
        assert budget_ratio(emul[n], want[n], budget[n]) <= 1.0, n
    p_nomask = torch.softmax((qf @ kf.transpose(-1, -2)) * sc, -1)
    mistakes = {
        "dq without the delta term": ("dq", bf(bf(p * dp * sc) @ kf)),
        "dq against keys shifted by one row": ("dq", bf(ds @ torch.roll(kf, 1, dims=-2))),
        "dk without the softmax scale": ("dk", bf(bf(p * (dp - delta)).transpose(-1, -2) @ qf)),
        "dv with the probabilities transposed": ("dv", bf(bf(p) @ dof)),
    }
    if causal:
        mistakes["dv without the causal mask"] = ("dv", bf(bf(p_nomask).transpose(-1, -2) @ dof))
    for what, (n, got) in mistakes.items():
        assert budget_ratio(got, want[n], budget[n]) > 1.0, what
