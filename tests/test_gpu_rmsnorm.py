"""GPU parity of the fused RMSNorm (mi_rmsnorm_fwd / mi_rmsnorm_bwd) against the
float64 oracle (oracle/normalization.py) on the same rounded inputs.

Tolerances.
* Forward: the kernel rounds n = x * r to x's dtype as the reference does.
  Its fp32 r may differ from the float64 one in the last bits, which can move
  n across a rounding boundary, so a 16-bit n may differ by one unit in the
  last place (2 u relative), and y is rounded once more (u).  Bound:
  |y - ref| <= (3 u + 1e-5) |ref| against the unrounded float64 product, with
  u the unit roundoff of y's dtype (2^-8 bf16, 2^-11 fp16), plus 2^-22 for
  fp16 values below its smallest normal.  In addition, at least 99% of the
  elements must equal the oracle exactly after rounding, which a missing
  intermediate rounding or a wrong eps fails.  An fp32 y (fp32 weight) carries
  only the flip of n: within (2 u_x + 1e-5) |ref|.
* Backward: fp32 arithmetic, one final rounding: dx within u |ref| plus
  1e-5 of the magnitudes that cancel in it (r |dn| + |x| r^3 |mean(dn x)|);
  dw within u |ref| plus 1e-5 * sum_rows |dy n|, plus |dy| times the change of
  n for the elements whose rounding to x's dtype the fp32 r (within 5e-7 of
  the float64 one) can flip.
"""
import numpy as np
import pytest
import torch

from gpu_ref import seeded
from oracle import rmsnorm_backward, rmsnorm_forward

pytestmark = pytest.mark.gpu

U = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11, torch.float32: 0.0}
# below the smallest normal (fp16: 2^-14) the spacing is absolute, 2^-24 for fp16;
# an n flip there plus the final rounding stays under 2^-22
TINY = {torch.bfloat16: 1e-30, torch.float16: 2.0 ** -22, torch.float32: 1e-30}
EPS = 1e-6


def _np(t):
    return t.detach().float().cpu().double().numpy()


def _check_forward(y, x, w, eps):
    yd = y.dtype
    ref, _ = rmsnorm_forward(_np(x), _np(w), eps, x_dtype=x.dtype)
    got = _np(y)
    if yd == torch.float32:
        # 16-bit x: the n flip (2 u of x's dtype) is the only error left
        bound = np.abs(ref) * (2 * U[x.dtype] + 1e-5) + TINY[x.dtype]
        assert (np.abs(got - ref) <= bound).all(), np.abs(got - ref).max()
        if x.dtype != torch.float32:
            assert np.mean(got == ref.astype(np.float32)) >= 0.99
        return
    bound = np.abs(ref) * (3 * U[yd] + 1e-5) + TINY[yd]
    assert (np.abs(got - ref) <= bound).all(), np.abs(got - ref).max()
    exact = torch.from_numpy(ref).to(yd).double().numpy()
    assert np.mean(got == exact) >= 0.99, np.mean(got == exact)


def _check_backward(dx, dw, x, w, dy, eps):
    xn, wn, dyn = _np(x), _np(w), _np(dy)
    rdx, rdw = rmsnorm_backward(xn, wn, dyn, eps, x_dtype=x.dtype)
    H = xn.shape[-1]
    r = 1.0 / np.sqrt((xn * xn).mean(-1) + eps)
    dn = dyn * wn
    s = (dn * xn).sum(-1)
    scale = r[..., None] * np.abs(dn) + np.abs(xn) * (r ** 3 * np.abs(s) / H)[..., None]
    got = _np(dx)
    bound = np.abs(rdx) * (U[dx.dtype] + 1e-5) + 1e-5 * scale + 1e-30
    assert (np.abs(got - rdx) <= bound).all(), np.abs(got - rdx).max()
    def rnd(a):
        return torch.from_numpy(a).to(x.dtype).double().numpy() if x.dtype != torch.float32 else a
    xr = xn * r[..., None]
    n = rnd(xr)
    wscale = np.abs(dyn * n).reshape(-1, H).sum(0)
    # the kernel's fp32 r is within a few 1e-7 of r: where that moves x r across
    # a rounding boundary of x's dtype, n (and so dy * n) may take the other value
    flip = np.abs(dyn * (rnd(xr * (1 + 5e-7)) - rnd(xr * (1 - 5e-7)))).reshape(-1, H).sum(0)
    gw = _np(dw)
    bound = np.abs(rdw) * (U[dw.dtype] + 1e-5) + 1e-5 * wscale + flip + 1e-30
    assert (np.abs(gw - rdw) <= bound).all(), np.abs(gw - rdw).max()


def _run(x, w, dy, eps=EPS):
    from gpt_from_scratch_amd import rms_norm
    xg = x.detach().clone().requires_grad_(True)
    wg = w.detach().clone().requires_grad_(True)
    y = rms_norm(xg, wg, eps)
    y.backward(dy)
    return y, xg.grad, wg.grad


@pytest.mark.parametrize("xd,wd", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16),
                                   (torch.float32, torch.float32), (torch.bfloat16, torch.float32)])
@pytest.mark.parametrize("rows,H", [(37, 768), (5, 4), (19, 64), (33, 1000), (9, 2048),
                                    (6, 3072), (3, 5000), (21, 7)])
def test_matches_oracle(gpu, xd, wd, rows, H):
    x = seeded((rows, H), 100 + H, std=1.5, dtype=xd)
    w = (1.0 + 0.1 * seeded((H,), 200 + H, dtype=torch.float32)).to(wd)
    yd = torch.float32 if wd == torch.float32 else xd
    dy = seeded((rows, H), 300 + H, dtype=yd)
    y, dx, dw = _run(x.to(gpu), w.to(gpu), dy.to(gpu))
    assert y.dtype == yd and dx.dtype == xd and dw.dtype == wd
    _check_forward(y, x, w, EPS)
    _check_backward(dx, dw, x, w, dy, EPS)


def test_model_layout_module_and_reference_ops(gpu):
    """[S, B, H] activations as the blocks hand them over, weight bf16 as after the
    optimizer moved it into its flat buffer; forward against the reference's own
    torch op sequence (normalization.py:15-24) on the GPU."""
    from gpt_from_scratch_amd import RMSNorm
    S, B, H = 1024, 8, 768
    g = torch.Generator(device=gpu).manual_seed(3)
    x = torch.randn(S, B, H, generator=g, device=gpu).to(torch.bfloat16)
    norm = RMSNorm(H, eps=1e-6, device=gpu)
    with torch.no_grad():
        norm.weight.copy_(1 + 0.1 * torch.randn(H, generator=g, device=gpu))
    norm.weight.data = norm.weight.data.to(torch.bfloat16)
    y = norm(x).detach()
    xf = x.float()
    ref = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16) * norm.weight
    ref = ref.detach()
    assert y.dtype == ref.dtype == torch.bfloat16
    assert float((y == ref).float().mean()) >= 0.99
    assert float(((y.float() - ref.float()).abs() / ref.float().abs().clamp_min(1e-30)).max()) <= 3 * 2 ** -8 + 1e-5


def test_strided_rows_aliasing_and_determinism(gpu):
    from gpt_from_scratch_amd import _lib, rms_norm
    H = 768
    for pad in (4, 1):  # 4-element aligned rows (vector path), then misaligned (scalar)
        wide = seeded((50, H + pad), 7 + pad).to(gpu)
        x = wide[:, :H]
        w = (1 + 0.1 * seeded((H,), 8)).to(gpu)
        dy = seeded((50, H), 9).to(gpu)
        y, dx, dw = _run(x, w, dy)
        _check_forward(y, x, w, EPS)
        _check_backward(dx, dw, x, w, dy, EPS)
        _, dx2, dw2 = _run(x, w, dy)
        assert torch.equal(dx, dx2) and torch.equal(dw, dw2)
    # dx written over dy
    x = seeded((40, H), 10).to(gpu)
    w = (1 + 0.1 * seeded((H,), 11)).to(gpu)
    dy = seeded((40, H), 12).to(gpu)
    y = torch.empty_like(x)
    rstd = torch.empty(40, dtype=torch.float32, device=gpu)
    _lib.rmsnorm_fwd(x, w, EPS, y, rstd)
    ws = torch.empty(_lib.rmsnorm_workspace(40, H), dtype=torch.float32, device=gpu)
    dx, dw = torch.empty_like(x), torch.empty_like(w)
    _lib.rmsnorm_bwd(x, w, rstd, dy, dx, dw, ws)
    dy2, dw2 = dy.clone(), torch.empty_like(w)
    _lib.rmsnorm_bwd(x, w, rstd, dy2, dy2, dw2, ws)
    assert torch.equal(dx, dy2) and torch.equal(dw, dw2)


def test_backward_with_several_rows_per_wave(gpu):
    """5000 rows > 256 partial rows x 16 waves: every wave of the backward loops
    over more than one row, and the dw partials cover all of them."""
    rows, H = 5000, 768
    x = seeded((rows, H), 61, std=1.5)
    w = (1.0 + 0.1 * seeded((H,), 62, dtype=torch.float32)).to(torch.bfloat16)
    dy = seeded((rows, H), 63)
    y, dx, dw = _run(x.to(gpu), w.to(gpu), dy.to(gpu))
    _check_forward(y, x, w, EPS)
    _check_backward(dx, dw, x, w, dy, EPS)


def test_row_broadcast_gradient(gpu):
    """A valid autograd gradient whose row axis has stride 0 (the gradient of
    (y.sum(0) * c).sum() is one row broadcast over all rows): the module copies
    it before the kernels instead of handing overlapping rows to the C ABI."""
    rows, H = 17, 768
    x = seeded((rows, H), 501, std=1.5, dtype=torch.bfloat16).to(gpu)
    w = (1.0 + 0.1 * seeded((H,), 502, dtype=torch.float32)).to(torch.bfloat16).to(gpu)
    c = seeded((H,), 503, dtype=torch.bfloat16).to(gpu)
    from gpt_from_scratch_amd import rms_norm
    xg = x.clone().requires_grad_(True)
    wg = w.clone().requires_grad_(True)
    (rms_norm(xg, wg, EPS).sum(0) * c).sum().backward()
    dy = c.expand(rows, H)
    _check_backward(xg.grad, wg.grad, x, w, dy, EPS)
    # the same broadcast tensor as a forward input
    y = rms_norm(x[:1].expand(rows, H), w, EPS)
    _check_forward(y, x[:1].expand(rows, H).contiguous(), w, EPS)


def _add_norm_composition(x, r, w, ds, dy, eps=EPS):
    """The reference's op pair on the same kernels: s = x + r (torch's add), y =
    RMSNorm(s); autograd accumulates s's two gradients (ds and the norm's dx)."""
    from gpt_from_scratch_amd import rms_norm
    xg, rg, wg = (t.detach().clone().requires_grad_(True) for t in (x, r, w))
    s = xg + rg
    y = rms_norm(s, wg, eps)
    torch.autograd.backward([s, y], [ds, dy])
    return s.detach(), y.detach(), xg.grad, rg.grad, wg.grad


def _add_norm_fused(x, r, w, ds, dy, eps=EPS):
    from gpt_from_scratch_amd import add_rms_norm
    xg, rg, wg = (t.detach().clone().requires_grad_(True) for t in (x, r, w))
    s, y = add_rms_norm(xg, rg, wg, eps)
    torch.autograd.backward([s, y], [ds, dy])
    return s.detach(), y.detach(), xg.grad, rg.grad, wg.grad


@pytest.mark.parametrize("xd,wd", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16),
                                   (torch.float32, torch.float32), (torch.bfloat16, torch.float32)])
@pytest.mark.parametrize("rows,H,pad", [(37, 768, 0), (19, 64, 0), (6, 3072, 0), (3, 5000, 0),
                                        (21, 7, 0), (29, 768, 1)])
def test_add_norm_matches_composition_and_oracle(gpu, xd, wd, rows, H, pad):
    """mi_rmsnorm_add_fwd / _bwd against the two-op composition on the same
    kernels (torch's add, then the RMSNorm kernels; autograd's accumulation of
    the sum's gradients): the sum, y, both input gradients and dw bit for bit,
    on the vector path and (H = 7, 5000, or rows padded by one element) the
    scalar path.  y and the gradients also against the float64 oracle over the
    rounded sum, within the RMSNorm bounds plus the accumulation's rounding."""
    wide = seeded((rows, H + pad), 400 + H, std=1.5, dtype=xd).to(gpu)
    x = wide[:, :H]
    r = seeded((rows, H), 401 + H, std=0.7, dtype=xd).to(gpu)
    w = (1.0 + 0.1 * seeded((H,), 402 + H, dtype=torch.float32)).to(wd).to(gpu)
    yd = torch.float32 if wd == torch.float32 else xd
    dy = seeded((rows, H), 403 + H, dtype=yd).to(gpu)
    ds = seeded((rows, H), 404 + H, std=0.5, dtype=xd).to(gpu)
    fs, fy, fdx, fdr, fdw = _add_norm_fused(x, r, w, ds, dy)
    cs, cy, cdx, cdr, cdw = _add_norm_composition(x, r, w, ds, dy)
    torch.cuda.synchronize()
    assert fs.dtype == xd and fy.dtype == yd and fdx.dtype == xd and fdw.dtype == wd
    for name, a, b in (("sum", fs, cs), ("y", fy, cy), ("dx", fdx, cdx), ("dres", fdr, cdr),
                       ("dw", fdw, cdw)):
        assert torch.equal(a, b), (name, float((a.float() - b.float()).abs().max()))
    # the oracle over the rounded sum: y as RMSNorm's forward; dx - ds as its backward
    _check_forward(fy, fs, w, EPS)
    s64 = _np(fs)
    rdx, _ = rmsnorm_backward(s64, _np(w), _np(dy), EPS, x_dtype=xd)
    want = rdx + _np(ds)
    got = _np(fdx)
    u = U[xd]
    bound = (np.abs(rdx) + np.abs(want)) * (u + 1e-5) + 1e-5 * np.abs(rdx).max() + 1e-30
    assert (np.abs(got - want) <= bound).all(), np.abs(got - want).max()


def test_add_norm_in_place_and_model_stack(gpu):
    """The sum written over x (the residual stream updated in place) equals the
    out-of-place result; and a stack of blocks whose residual adds are fused
    into the following norms gives the same loss and parameter gradients, bit
    for bit, as the same stack with separate adds and norms (the model's
    layout [S, B, H], bf16 weights)."""
    from gpt_from_scratch_amd import _lib, add_rms_norm, rms_norm
    S, B, H = 128, 4, 768
    x = seeded((S, B, H), 601, dtype=torch.bfloat16).to(gpu)
    r = seeded((S, B, H), 602, dtype=torch.bfloat16).to(gpu)
    w = (1 + 0.1 * seeded((H,), 603, dtype=torch.float32)).to(torch.bfloat16).to(gpu)
    s, y = torch.empty_like(x), torch.empty_like(x)
    rstd = torch.empty(S, B, dtype=torch.float32, device=gpu)
    _lib.rmsnorm_add_fwd(x, r, w, EPS, s, y, rstd)
    xi = x.clone()
    y2, rstd2 = torch.empty_like(x), torch.empty_like(rstd)
    _lib.rmsnorm_add_fwd(xi, r, w, EPS, xi, y2, rstd2)
    assert torch.equal(xi, s) and torch.equal(y2, y) and torch.equal(rstd2, rstd)

    torch.manual_seed(7)
    ws = [(1 + 0.1 * torch.randn(H, device=gpu)).to(torch.bfloat16) for _ in range(5)]
    mats = [(0.02 * torch.randn(H, H, device=gpu)).to(torch.bfloat16) for _ in range(4)]

    def run(fused):
        wp = [t.clone().requires_grad_(True) for t in ws]
        mp = [t.clone().requires_grad_(True) for t in mats]
        h0 = x.clone().requires_grad_(True)
        if fused:
            h = rms_norm(h0, wp[0], EPS)
            xs = h0
            for i in range(4):
                xs, h = add_rms_norm(xs, torch.tanh(h @ mp[i]), wp[i + 1], EPS)
        else:
            xs = h0
            h = rms_norm(xs, wp[0], EPS)
            for i in range(4):
                xs = xs + torch.tanh(h @ mp[i])
                h = rms_norm(xs, wp[i + 1], EPS)
        loss = (h.float() ** 2).mean()
        loss.backward()
        return loss.detach(), h0.grad, [t.grad for t in wp + mp]

    l1, g1, p1 = run(True)
    l2, g2, p2 = run(False)
    assert torch.equal(l1, l2) and torch.equal(g1, g2)
    for a, b in zip(p1, p2):
        assert torch.equal(a, b)


@pytest.mark.parametrize("xd,wd", [(torch.bfloat16, torch.bfloat16), (torch.bfloat16, torch.float32),
                                   (torch.float16, torch.float16)])
@pytest.mark.parametrize("rows,H", [(37, 768), (45, 1024), (9, 2048), (13, 64)])
def test_forward_paths_agree_bit_for_bit(gpu, xd, wd, rows, H):
    """The forward's 16-byte path (bf16 rows 8-element aligned: half a wave per
    row) and its 8-byte path (rows only 4-element aligned: a wave per row) sum
    the squares in the same order, so y, rstd and the fused add's sum agree bit
    for bit; fp16 takes the 8-byte path at both strides.  Rows are laid out at
    strides H (16-byte aligned), H + 8 (aligned, padded) and H + 4 (4-element
    aligned only)."""
    import ctypes
    from gpt_from_scratch_amd import _lib
    lib = _lib.lib()
    x = seeded((rows, H), 700 + H, std=1.5, dtype=xd).to(gpu)
    r = seeded((rows, H), 701 + H, std=0.7, dtype=xd).to(gpu)
    w = (1.0 + 0.1 * seeded((H,), 702 + H, dtype=torch.float32)).to(wd).to(gpu)
    yd = torch.float32 if wd == torch.float32 else xd
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    sp = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    dx_, dw_ = _lib.dtype_code(x), _lib.dtype_code(w)
    outs = {}
    for pad in (0, 8, 4):
        ld = H + pad
        xb, rb = (torch.zeros(rows, ld, dtype=xd, device=gpu) for _ in range(2))
        xb[:, :H] = x
        rb[:, :H] = r
        yb, y2 = (torch.zeros(rows, ld, dtype=yd, device=gpu) for _ in range(2))
        sb = torch.zeros(rows, ld, dtype=xd, device=gpu)
        rs, rs2 = (torch.empty(rows, device=gpu) for _ in range(2))
        assert lib.mi_rmsnorm_fwd(dx_, dw_, rows, H, ctypes.c_float(EPS), P(xb), ld, P(w),
                                  P(yb), ld, P(rs), sp) == 0
        assert lib.mi_rmsnorm_add_fwd(dx_, dw_, rows, H, ctypes.c_float(EPS), P(xb), ld, P(rb),
                                      ld, P(w), P(sb), ld, P(y2), ld, P(rs2), sp) == 0
        torch.cuda.synchronize()
        outs[pad] = (yb[:, :H].clone(), rs.clone(), sb[:, :H].clone(), y2[:, :H].clone(),
                     rs2.clone())
    for pad in (8, 4):
        for name, a, b in zip(("y", "rstd", "sum", "add y", "add rstd"), outs[0], outs[pad]):
            assert torch.equal(a, b), (pad, name, float((a.float() - b.float()).abs().max()))
    _check_forward(outs[0][0], x, w, EPS)


@pytest.mark.parametrize("xd,wd", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16),
                                   (torch.float32, torch.float32), (torch.bfloat16, torch.float32)])
@pytest.mark.parametrize("rows,H", [(37, 768), (21, 7)])
def test_weight_gradient_accumulated_in_place(gpu, xd, wd, rows, H):
    """mi_rmsnorm_bwd_acc / mi_rmsnorm_add_bwd_acc against the non-accumulating
    entry points followed by the add autograd's accumulation performs
    (g + dw in w's dtype): dweight and dx bit for bit, on the vector path (H =
    768) and the scalar one (H = 7); and the opt-in autograd path
    (grad_into=True) against the default one on an existing .grad."""
    from gpt_from_scratch_amd import _lib
    from gpt_from_scratch_amd.normalization import add_rms_norm, rms_norm

    x = seeded((rows, H), 600 + H, std=1.5, dtype=xd).to(gpu)
    w = (1.0 + 0.1 * seeded((H,), 601 + H, dtype=torch.float32)).to(wd).to(gpu)
    yd = torch.float32 if wd == torch.float32 else xd
    dy = seeded((rows, H), 602 + H, dtype=yd).to(gpu)
    ds = seeded((rows, H), 603 + H, std=0.5, dtype=xd).to(gpu)
    g0 = seeded((H,), 604 + H, std=0.3, dtype=wd).to(gpu)
    rstd = torch.empty(rows, dtype=torch.float32, device=gpu)
    _lib.rmsnorm_fwd(x, w, EPS, torch.empty(rows, H, dtype=yd, device=gpu), rstd)
    ws = torch.empty(_lib.rmsnorm_workspace(rows, H), dtype=torch.float32, device=gpu)
    for add in (False, True):
        dx_a, dx_b = torch.empty_like(x), torch.empty_like(x)
        dw = torch.empty_like(w)
        acc = g0.clone()
        if add:
            _lib.rmsnorm_add_bwd(x, w, rstd, dy, ds, dx_a, dw, ws)
            _lib.rmsnorm_add_bwd(x, w, rstd, dy, ds, dx_b, acc, ws, accumulate=True)
        else:
            _lib.rmsnorm_bwd(x, w, rstd, dy, dx_a, dw, ws)
            _lib.rmsnorm_bwd(x, w, rstd, dy, dx_b, acc, ws, accumulate=True)
        torch.cuda.synchronize()
        assert torch.equal(dx_a, dx_b), add
        assert torch.equal(acc, g0 + dw), (add, float((acc.float() - (g0 + dw).float()).abs().max()))

    # autograd: the kernel adds into .grad and hands autograd none
    for add in (False, True):
        grads = []
        for into in (False, True):
            wp = torch.nn.Parameter(w.clone())
            wp.grad = g0.clone()
            xi = x.clone().requires_grad_()
            if add:
                s, y = add_rms_norm(xi, ds.clone(), wp, EPS, grad_into=into)
                torch.autograd.backward([s, y], [ds, dy])
            else:
                rms_norm(xi, wp, EPS, grad_into=into).backward(dy)
            grads.append((xi.grad, wp.grad))
        torch.cuda.synchronize()
        (xa, wa), (xb, wb) = grads
        assert torch.equal(xa, xb) and torch.equal(wa, wb), add
