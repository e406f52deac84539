"""ctypes binding of libmi_attn.so, the C ABI declared in include/mi_attn.h.

The library is built in-tree (``gpt_from_scratch_amd/libmi_attn.so``, see
``gpt_from_scratch_amd/build.py``).  There is no fallback: if the library is
missing or a tensor is not on a ROCm GPU, the calls below raise.

torch is imported before the library is loaded so that the library binds to the
HIP runtime torch already loaded (same SONAME), i.e. streams and device
pointers handed over from torch are valid in the library.
"""
from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmi_attn.so")

MI_OK = 0
_DTYPES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

# Every function declared in include/mi_attn.h.
EXPORTED = ("mi_version", "mi_status_str", "mi_last_error", "mi_attn_fwd", "mi_attn_bwd",
            "mi_attn_bwd_preprocess", "mi_attn_bwd_grads", "mi_attn_bwd_dkdv", "mi_attn_bwd_dq",
            "mi_rope", "mi_rope_qk", "mi_xent_fwd", "mi_xent_bwd", "mi_rmsnorm_fwd",
            "mi_rmsnorm_bwd_workspace", "mi_rmsnorm_bwd", "mi_swiglu_fwd", "mi_swiglu_bwd",
            "mi_adamw_workspace", "mi_grad_sumsq", "mi_adamw_step", "mi_attn_bwd_noalloc",
            "mi_rmsnorm_add_fwd", "mi_rmsnorm_add_bwd", "mi_attn_bwd_rope",
            "mi_rmsnorm_bwd_acc", "mi_rmsnorm_add_bwd_acc", "mi_copy_qk")

# B*H*S limit of mi_attn_bwd_noalloc (its static workspace array), include/mi_attn.h
NOALLOC_MAX_ROWS = 1 << 20

_lib = None


class MiError(RuntimeError):
    """A non-OK status returned by the C ABI."""


def _i64x4():
    return ctypes.c_int64 * 4


def _declare(lib):
    p, i, f, i64p = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.POINTER(ctypes.c_int64)
    lib.mi_version.restype = i
    lib.mi_version.argtypes = []
    lib.mi_status_str.restype = ctypes.c_char_p
    lib.mi_status_str.argtypes = [i]
    lib.mi_last_error.restype = ctypes.c_char_p
    lib.mi_last_error.argtypes = []
    lib.mi_attn_fwd.restype = i
    lib.mi_attn_fwd.argtypes = [i, i, i, i, i, i, f, p, i64p, p, i64p, p, i64p, p, i64p, p, p]
    lib.mi_attn_bwd.restype = i
    lib.mi_attn_bwd.argtypes = [i, i, i, i, i, i, f,
                                p, i64p, p, i64p, p, i64p, p, i64p, p, i64p,
                                p, p, p, i64p, p, i64p, p, i64p, p]
    lib.mi_attn_bwd_rope.restype = i
    lib.mi_attn_bwd_rope.argtypes = [i, i, i, i, i, i, f,
                                     p, i64p, p, i64p, p, i64p, p, i64p, p, i64p,
                                     p, p, p, i64p, p, i64p, p, i64p, i, p, i64p, p, i64p, p]
    lib.mi_attn_bwd_noalloc.restype = i
    lib.mi_attn_bwd_noalloc.argtypes = [i, i, i, i, i, i, f,
                                        p, i64p, p, i64p, p, i64p, p, i64p, p, i64p,
                                        p, p, i64p, p, i64p, p, i64p, p]
    lib.mi_attn_bwd_preprocess.restype = i
    lib.mi_attn_bwd_preprocess.argtypes = [i, i, i, i, i, p, i64p, p, i64p, p, p, p]
    lib.mi_attn_bwd_grads.restype = i
    lib.mi_attn_bwd_grads.argtypes = [i, i, i, i, i, i, f, p, i64p, p, i64p, p, i64p, p, i64p,
                                      p, p, p, i64p, p, i64p, p, i64p, p]
    lib.mi_attn_bwd_dkdv.restype = i
    lib.mi_attn_bwd_dkdv.argtypes = [i, i, i, i, i, i, f, p, i64p, p, i64p, p, i64p, p, i64p,
                                     p, p, p, i64p, p, i64p, p]
    lib.mi_attn_bwd_dq.restype = i
    lib.mi_attn_bwd_dq.argtypes = [i, i, i, i, i, i, f, p, i64p, p, i64p, p, i64p, p, i64p,
                                   p, p, p, i64p, p]
    lib.mi_rope.restype = i
    lib.mi_rope.argtypes = [i, i, i, i, i, i, i, p, i64p, p, i64p, p, i64p, p, i64p, p]
    lib.mi_rope_qk.restype = i
    lib.mi_rope_qk.argtypes = [i, i, i, i, i, i, i, p, i64p, p, i64p, p, i64p, p, i64p,
                               p, i64p, p, i64p, p]
    lib.mi_copy_qk.restype = i
    lib.mi_copy_qk.argtypes = [i, i, i, i, i, p, i64p, p, i64p, p, i64p, p, i64p, p]
    i64 = ctypes.c_int64
    lib.mi_xent_fwd.restype = i
    lib.mi_xent_fwd.argtypes = [i, i64, i64, p, i64, p, p, p, p]
    lib.mi_xent_bwd.restype = i
    lib.mi_xent_bwd.argtypes = [i, i64, i64, p, i64, p, p, p, p, i64, p]
    lib.mi_rmsnorm_fwd.restype = i
    lib.mi_rmsnorm_fwd.argtypes = [i, i, i64, i64, f, p, i64, p, p, i64, p, p]
    lib.mi_rmsnorm_bwd_workspace.restype = i64
    lib.mi_rmsnorm_bwd_workspace.argtypes = [i64, i64]
    lib.mi_rmsnorm_bwd.restype = i
    lib.mi_rmsnorm_bwd.argtypes = [i, i, i64, i64, p, i64, p, p, p, i64, p, i64, p, p, i64, p]
    lib.mi_rmsnorm_add_fwd.restype = i
    lib.mi_rmsnorm_add_fwd.argtypes = [i, i, i64, i64, f, p, i64, p, i64, p, p, i64, p, i64, p, p]
    lib.mi_rmsnorm_add_bwd.restype = i
    lib.mi_rmsnorm_add_bwd.argtypes = [i, i, i64, i64, p, i64, p, p, p, i64, p, i64, p, i64, p,
                                       p, i64, p]
    lib.mi_rmsnorm_bwd_acc.restype = i
    lib.mi_rmsnorm_bwd_acc.argtypes = lib.mi_rmsnorm_bwd.argtypes
    lib.mi_rmsnorm_add_bwd_acc.restype = i
    lib.mi_rmsnorm_add_bwd_acc.argtypes = lib.mi_rmsnorm_add_bwd.argtypes
    lib.mi_swiglu_fwd.restype = i
    lib.mi_swiglu_fwd.argtypes = [i, i64, i64, p, i64, p, i64, p]
    lib.mi_swiglu_bwd.restype = i
    lib.mi_swiglu_bwd.argtypes = [i, i64, i64, p, i64, p, i64, p, i64, p]
    lib.mi_adamw_workspace.restype = i64
    lib.mi_adamw_workspace.argtypes = []
    lib.mi_grad_sumsq.restype = i
    lib.mi_grad_sumsq.argtypes = [i, i64, p, p, i64, p]
    lib.mi_adamw_step.restype = i
    lib.mi_adamw_step.argtypes = [i, i, i64, p, p, p, p, p, f, f, f, f, f, f, f, f, p, p]


def lib():
    """Load (once) and return the C library.  Raises if it was not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; "
                "g.build()'` (or `make -C gpt_from_scratch_amd/csrc`)")
        handle = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_LOCAL)
        _declare(handle)
        _lib = handle
    return _lib


def _check(status: int, what: str):
    if status != MI_OK:
        l = lib()
        msg = l.mi_last_error().decode()
        name = l.mi_status_str(status).decode()
        raise MiError(f"{what}: {name} ({msg})")


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}: expected float32, float16 or bfloat16")


def _strides(t: torch.Tensor, n: int):
    arr = (ctypes.c_int64 * n)(*t.stride())
    return arr


def _ptr(t: torch.Tensor):
    return ctypes.c_void_p(t.data_ptr())


def _require_gpu(*ts: torch.Tensor):
    dev = ts[0].device
    if dev.type != "cuda":
        raise RuntimeError(
            f"gpt_from_scratch_amd kernels run on ROCm GPUs only; got a tensor on {dev}")
    for t in ts[1:]:
        if t.device != dev:
            raise RuntimeError(f"all tensors must be on {dev}; got one on {t.device}")


def _stream(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _check_attn_tensors(q, same, stats, ws=None):
    """Shapes and dtypes the attention kernels index by: every tensor of `same`
    is [B, H, S, D] in q's dtype; every one of `stats` (lse) is a dense fp32
    [B, H, S] (the kernels address it as (b*H + h)*S + s); the backward
    workspace `ws` is a dense fp32 [2, B, H, S] (delta, then lse * log2(e))."""
    if q.dim() != 4:
        raise ValueError(f"q must be [B, H, S, D]; got shape {tuple(q.shape)}")
    B, H, S, _ = q.shape
    for name, t in same:
        if t.shape != q.shape or t.dtype != q.dtype:
            raise ValueError(f"{name} must match q ({tuple(q.shape)}, {q.dtype}); got "
                             f"{tuple(t.shape)}, {t.dtype}")
    for name, t in stats:
        if t.dtype != torch.float32 or t.shape != (B, H, S) or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous float32 [B, H, S] = [{B}, {H}, {S}] "
                             f"tensor; got {t.dtype} {tuple(t.shape)} strides {t.stride()}")
    if ws is not None and (ws.dtype != torch.float32 or ws.shape != (2, B, H, S)
                           or not ws.is_contiguous()):
        raise ValueError(f"the backward workspace must be a contiguous float32 [2, B, H, S] = "
                         f"[2, {B}, {H}, {S}] tensor; got {ws.dtype} {tuple(ws.shape)} strides "
                         f"{ws.stride()}")


def attn_fwd(q, k, v, o, lse, causal: bool, scale: float):
    """Enqueue the forward on the current stream: writes o [B,H,S,D] and lse [B,H,S] fp32."""
    _check_attn_tensors(q, (("k", k), ("v", v), ("o", o)), (("lse", lse),))
    _require_gpu(q, k, v, o, lse)
    B, H, S, D = q.shape
    st = lib().mi_attn_fwd(dtype_code(q), B, H, S, D, int(bool(causal)), float(scale),
                           _ptr(q), _strides(q, 4), _ptr(k), _strides(k, 4),
                           _ptr(v), _strides(v, 4), _ptr(o), _strides(o, 4),
                           _ptr(lse), _stream(q))
    _check(st, "mi_attn_fwd")


def bwd_workspace(lse):
    """The backward workspace for a forward's lse [B, H, S]: fp32 [2, B, H, S]
    (delta = rowsum(dO * O), then lse * log2(e))."""
    return torch.empty((2,) + tuple(lse.shape), dtype=torch.float32, device=lse.device)


def attn_bwd(q, k, v, o, do, lse, ws, dq, dk, dv, causal: bool, scale: float):
    """Enqueue the backward on the current stream: writes the workspace ws
    ([2, B, H, S]: delta, lse * log2(e)) and dq, dk, dv."""
    _check_attn_tensors(q, (("k", k), ("v", v), ("o", o), ("do", do), ("dq", dq), ("dk", dk),
                            ("dv", dv)), (("lse", lse),), ws)
    _require_gpu(q, k, v, o, do, lse, ws, dq, dk, dv)
    B, H, S, D = q.shape
    st = lib().mi_attn_bwd(dtype_code(q), B, H, S, D, int(bool(causal)), float(scale),
                           _ptr(q), _strides(q, 4), _ptr(k), _strides(k, 4),
                           _ptr(v), _strides(v, 4), _ptr(o), _strides(o, 4),
                           _ptr(do), _strides(do, 4), _ptr(lse), _ptr(ws),
                           _ptr(dq), _strides(dq, 4), _ptr(dk), _strides(dk, 4),
                           _ptr(dv), _strides(dv, 4), _stream(q))
    _check(st, "mi_attn_bwd")


def attn_bwd_noalloc(q, k, v, o, do, lse, dq, dk, dv, causal: bool, scale: float):
    """mi_attn_bwd without a workspace argument (the library's static array): writes dq, dk, dv."""
    _check_attn_tensors(q, (("k", k), ("v", v), ("o", o), ("do", do), ("dq", dq), ("dk", dk),
                            ("dv", dv)), (("lse", lse),))
    _require_gpu(q, k, v, o, do, lse, dq, dk, dv)
    B, H, S, D = q.shape
    st = lib().mi_attn_bwd_noalloc(dtype_code(q), B, H, S, D, int(bool(causal)), float(scale),
                                   _ptr(q), _strides(q, 4), _ptr(k), _strides(k, 4),
                                   _ptr(v), _strides(v, 4), _ptr(o), _strides(o, 4),
                                   _ptr(do), _strides(do, 4), _ptr(lse),
                                   _ptr(dq), _strides(dq, 4), _ptr(dk), _strides(dk, 4),
                                   _ptr(dv), _strides(dv, 4), _stream(q))
    _check(st, "mi_attn_bwd_noalloc")


def rope(x, cos, sin, out, inverse: bool):
    """Enqueue one rotation of x [S,B,H,D] into out with tables cos/sin [S', D/2]."""
    _require_gpu(x, cos, sin, out)
    S, B, H, D = x.shape
    st = lib().mi_rope(dtype_code(x), dtype_code(cos), S, B, H, D, int(bool(inverse)),
                       _ptr(x), _strides(x, 4), _ptr(cos), _strides(cos, 2),
                       _ptr(sin), _strides(sin, 2), _ptr(out), _strides(out, 4), _stream(x))
    _check(st, "mi_rope")


def attn_bwd_rope(q, k, v, o, do, lse, ws, dq, dk, dv, causal: bool, scale: float, cos, sin):
    """attn_bwd with dq and dk inverse-rotated by the RoPE tables cos / sin
    ([>= S, D/2]): the gradients with respect to the unrotated q, k."""
    _check_attn_tensors(q, (("k", k), ("v", v), ("o", o), ("do", do), ("dq", dq), ("dk", dk),
                            ("dv", dv)), (("lse", lse),), ws)
    _require_gpu(q, k, v, o, do, lse, ws, dq, dk, dv, cos, sin)
    B, H, S, D = q.shape
    st = lib().mi_attn_bwd_rope(dtype_code(q), B, H, S, D, int(bool(causal)), float(scale),
                                _ptr(q), _strides(q, 4), _ptr(k), _strides(k, 4),
                                _ptr(v), _strides(v, 4), _ptr(o), _strides(o, 4),
                                _ptr(do), _strides(do, 4), _ptr(lse), _ptr(ws),
                                _ptr(dq), _strides(dq, 4), _ptr(dk), _strides(dk, 4),
                                _ptr(dv), _strides(dv, 4), dtype_code(cos), _ptr(cos),
                                _strides(cos, 2), _ptr(sin), _strides(sin, 2), _stream(q))
    _check(st, "mi_attn_bwd_rope")


def rope_qk(q, k, cos, sin, q_out, k_out, inverse: bool):
    """Enqueue the rotation of q and k (same shape and dtype) in one launch."""
    _require_gpu(q, k, cos, sin, q_out, k_out)
    S, B, H, D = q.shape
    st = lib().mi_rope_qk(dtype_code(q), dtype_code(cos), S, B, H, D, int(bool(inverse)),
                          _ptr(q), _strides(q, 4), _ptr(k), _strides(k, 4),
                          _ptr(cos), _strides(cos, 2), _ptr(sin), _strides(sin, 2),
                          _ptr(q_out), _strides(q_out, 4), _ptr(k_out), _strides(k_out, 4),
                          _stream(q))
    _check(st, "mi_rope_qk")


def _rows(t: torch.Tensor):
    """(rows, row stride) of t viewed as rows over its last dim (unit stride)."""
    if t.stride(-1) != 1:
        raise ValueError("the vocabulary dim must have unit stride")
    lead = t.shape[:-1]
    rows = 1
    for n in lead:
        rows *= n
    if t.dim() == 1:
        return 1, t.shape[-1]
    # the leading dims must collapse into one row index with a single stride
    rs = t.stride(-2)
    expect = rs
    for d in range(t.dim() - 2, -1, -1):
        if t.shape[d] != 1 and t.stride(d) != expect:
            raise ValueError(f"leading dims of {tuple(t.shape)} / {t.stride()} are not one row axis")
        expect *= t.shape[d]
    # rows that overlap (a broadcast row axis has stride 0) cannot be written
    # row by row and are refused by the C ABI: callers copy such tensors first
    if rows > 1 and rs < t.shape[-1]:
        raise ValueError(f"rows of {tuple(t.shape)} / {t.stride()} overlap (row stride {rs})")
    return rows, rs


def xent_fwd(logits, target, loss, lse):
    """Enqueue the cross-entropy forward: loss [rows] (logits dtype), lse [rows] fp32."""
    _require_gpu(logits, target, loss, lse)
    rows, rs = _rows(logits)
    st = lib().mi_xent_fwd(dtype_code(logits), rows, logits.shape[-1], _ptr(logits), rs,
                           _ptr(target), _ptr(loss), _ptr(lse), _stream(logits))
    _check(st, "mi_xent_fwd")


def xent_bwd(logits, target, lse, grad_loss, grad):
    """Enqueue the cross-entropy backward into grad (may be logits itself)."""
    _require_gpu(logits, target, lse, grad_loss, grad)
    rows, rs = _rows(logits)
    grows, grs = _rows(grad)
    assert grows == rows
    st = lib().mi_xent_bwd(dtype_code(logits), rows, logits.shape[-1], _ptr(logits), rs,
                           _ptr(target), _ptr(lse), _ptr(grad_loss), _ptr(grad), grs,
                           _stream(logits))
    _check(st, "mi_xent_bwd")


def rmsnorm_fwd(x, weight, eps: float, y, rstd):
    """Enqueue the RMSNorm forward over the last dim: y, rstd [rows] fp32."""
    _require_gpu(x, weight, y, rstd)
    rows, xs = _rows(x)
    _, ys = _rows(y)
    st = lib().mi_rmsnorm_fwd(dtype_code(x), dtype_code(weight), rows, x.shape[-1], float(eps),
                              _ptr(x), xs, _ptr(weight), _ptr(y), ys, _ptr(rstd), _stream(x))
    _check(st, "mi_rmsnorm_fwd")


def rmsnorm_workspace(rows: int, hidden: int) -> int:
    return int(lib().mi_rmsnorm_bwd_workspace(rows, hidden))


def rmsnorm_bwd(x, weight, rstd, dy, dx, dweight, workspace, accumulate=False):
    """Enqueue the RMSNorm backward: dx (x's shape and dtype), dweight [hidden]
    (added to its contents with `accumulate`)."""
    _require_gpu(x, weight, rstd, dy, dx, dweight, workspace)
    rows, xs = _rows(x)
    _, dys = _rows(dy)
    _, dxs = _rows(dx)
    fn = lib().mi_rmsnorm_bwd_acc if accumulate else lib().mi_rmsnorm_bwd
    st = fn(dtype_code(x), dtype_code(weight), rows, x.shape[-1], _ptr(x), xs,
            _ptr(weight), _ptr(rstd), _ptr(dy), dys, _ptr(dx), dxs,
            _ptr(dweight), _ptr(workspace), workspace.numel(), _stream(x))
    _check(st, "mi_rmsnorm_bwd_acc" if accumulate else "mi_rmsnorm_bwd")


def rmsnorm_add_fwd(x, res, weight, eps: float, sum_out, y, rstd):
    """Enqueue sum = x + res and the RMSNorm forward over it: sum (x's dtype),
    y, rstd [rows] fp32."""
    _require_gpu(x, res, weight, sum_out, y, rstd)
    rows, xs = _rows(x)
    rrows, rs = _rows(res)
    srows, ss = _rows(sum_out)
    assert rrows == rows and srows == rows and res.dtype == x.dtype == sum_out.dtype
    _, ys = _rows(y)
    st = lib().mi_rmsnorm_add_fwd(dtype_code(x), dtype_code(weight), rows, x.shape[-1],
                                  float(eps), _ptr(x), xs, _ptr(res), rs, _ptr(weight),
                                  _ptr(sum_out), ss, _ptr(y), ys, _ptr(rstd), _stream(x))
    _check(st, "mi_rmsnorm_add_fwd")


def rmsnorm_add_bwd(sum_in, weight, rstd, dy, dsum, dx, dweight, workspace, accumulate=False):
    """Enqueue the backward of rmsnorm_add_fwd: dx = norm backward over sum_in
    plus dsum (the gradient of x and of res), dweight [hidden] (added to its
    contents with `accumulate`)."""
    _require_gpu(sum_in, weight, rstd, dy, dsum, dx, dweight, workspace)
    rows, xs = _rows(sum_in)
    _, dys = _rows(dy)
    drows, dss = _rows(dsum)
    _, dxs = _rows(dx)
    assert drows == rows and dsum.dtype == sum_in.dtype
    fn = lib().mi_rmsnorm_add_bwd_acc if accumulate else lib().mi_rmsnorm_add_bwd
    st = fn(dtype_code(sum_in), dtype_code(weight), rows, sum_in.shape[-1], _ptr(sum_in), xs,
            _ptr(weight), _ptr(rstd), _ptr(dy), dys, _ptr(dsum), dss, _ptr(dx), dxs,
            _ptr(dweight), _ptr(workspace), workspace.numel(), _stream(sum_in))
    _check(st, "mi_rmsnorm_add_bwd_acc" if accumulate else "mi_rmsnorm_add_bwd")


def swiglu_fwd(gate_up, out):
    """Enqueue h = silu(gate) * up over the last dim of gate_up [..., 2I] into out [..., I]."""
    _require_gpu(gate_up, out)
    rows, gs = _rows(gate_up)
    _, os_ = _rows(out)
    st = lib().mi_swiglu_fwd(dtype_code(gate_up), rows, out.shape[-1], _ptr(gate_up), gs,
                             _ptr(out), os_, _stream(gate_up))
    _check(st, "mi_swiglu_fwd")


def swiglu_bwd(gate_up, dout, dgate_up):
    """Enqueue the SwiGLU gradient into dgate_up [..., 2I]."""
    _require_gpu(gate_up, dout, dgate_up)
    rows, gs = _rows(gate_up)
    _, ds = _rows(dout)
    _, dgs = _rows(dgate_up)
    st = lib().mi_swiglu_bwd(dtype_code(gate_up), rows, dout.shape[-1], _ptr(gate_up), gs,
                             _ptr(dout), ds, _ptr(dgate_up), dgs, _stream(gate_up))
    _check(st, "mi_swiglu_bwd")


def adamw_workspace() -> int:
    return int(lib().mi_adamw_workspace())


def grad_sumsq(grad, workspace):
    """Enqueue workspace[0] = sum(grad^2) (fp32) over the flat grad buffer."""
    _require_gpu(grad, workspace)
    st = lib().mi_grad_sumsq(dtype_code(grad), grad.numel(), _ptr(grad), _ptr(workspace),
                             workspace.numel(), _stream(grad))
    _check(st, "mi_grad_sumsq")


def adamw_step(grad, master, exp_avg, exp_avg_sq, param, hp, grad_sumsq_buf):
    """Enqueue one AdamW step over flat buffers; hp = (1 - lr*wd, 1 - beta1, beta2,
    1 - beta2, step_size, bias_correction2_sqrt, eps, clip)."""
    ts = [grad, master, exp_avg, exp_avg_sq] + ([param] if param is not None else [])
    _require_gpu(*ts)
    for t in ts:
        if not t.is_contiguous():
            raise ValueError("optimizer buffers must be contiguous")
    n = grad.numel()
    for t in ts[1:]:
        if t.numel() != n:
            raise ValueError("optimizer buffers must have the same number of elements")
    st = lib().mi_adamw_step(dtype_code(grad), dtype_code(param if param is not None else master),
                             n, _ptr(grad), _ptr(master), _ptr(exp_avg), _ptr(exp_avg_sq),
                             _ptr(param) if param is not None else None,
                             *[float(x) for x in hp],
                             _ptr(grad_sumsq_buf) if grad_sumsq_buf is not None else None,
                             _stream(grad))
    _check(st, "mi_adamw_step")
