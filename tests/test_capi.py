"""Host-side checks of the C ABI (no GPU needed, nothing is launched).

The library must load, export every function include/mi_attn.h declares, and
reject invalid arguments with the documented status codes before it touches
the GPU.
"""
import ctypes
import os
import re

import pytest

from gpt_from_scratch_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mi_attn.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(
        r"^\s*(?:mi_status|int|int64_t|const char\*)\s+(mi_\w+)\s*\(", text, re.M)))


def test_header_declares_expected_api():
    assert _declared() == sorted(_lib.EXPORTED)


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.mi_version() >> 16 == 2


def test_status_strings():
    lib = _lib.lib()
    assert lib.mi_status_str(0) == b"ok"
    assert lib.mi_status_str(1) == b"invalid argument"
    assert lib.mi_status_str(2) == b"unsupported"
    assert lib.mi_status_str(3) == b"launch failed"


def _i4(*v):
    return (ctypes.c_int64 * 4)(*v)


def test_fwd_rejects_bad_arguments_before_launch():
    lib = _lib.lib()
    st = _i4(0, 0, 64, 1)
    fake = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    # unknown dtype
    assert lib.mi_attn_fwd(7, 1, 1, 64, 64, 1, 0.125, fake, st, fake, st, fake, st, fake, st,
                           fake, None) == 1
    assert b"dtype" in lib.mi_last_error()
    # non-positive size
    assert lib.mi_attn_fwd(2, 1, 0, 64, 64, 1, 0.125, fake, st, fake, st, fake, st, fake, st,
                           fake, None) == 1
    # null pointer
    assert lib.mi_attn_fwd(2, 1, 1, 64, 64, 1, 0.125, None, st, fake, st, fake, st, fake, st,
                           fake, None) == 1
    assert b"q: null" in lib.mi_last_error()
    # non-unit dim stride
    bad = _i4(0, 0, 64, 2)
    assert lib.mi_attn_fwd(2, 1, 1, 64, 64, 1, 0.125, fake, bad, fake, st, fake, st, fake, st,
                           fake, None) == 1
    assert b"dim stride" in lib.mi_last_error()
    # unsupported head dim
    assert lib.mi_attn_fwd(0, 1, 1, 64, 48, 1, 0.125, fake, st, fake, st, fake, st, fake, st,
                           fake, None) == 2
    # bad scale
    assert lib.mi_attn_fwd(2, 1, 1, 64, 64, 1, 0.0, fake, st, fake, st, fake, st, fake, st,
                           fake, None) == 1


def test_rope_rejects_odd_head_dim():
    lib = _lib.lib()
    st = _i4(0, 0, 0, 1)
    ts = (ctypes.c_int64 * 2)(1, 1)
    fake = ctypes.c_void_p(16)
    assert lib.mi_rope(2, 2, 4, 1, 1, 7, 0, fake, st, fake, ts, fake, ts, fake, st, None) == 1
    assert b"even" in lib.mi_last_error()


def test_python_api_refuses_cpu_tensors():
    """No CPU fallback: the product raises on host tensors."""
    import torch
    from gpt_from_scratch_amd import apply_flash_attn, apply_rope
    q = torch.randn(1, 1, 64, 64)
    with pytest.raises(RuntimeError, match="ROCm GPUs only"):
        apply_flash_attn(q, q, q)
    x = torch.randn(4, 1, 1, 8)
    c = torch.ones(4, 4)
    with pytest.raises(RuntimeError, match="ROCm GPUs only"):
        apply_rope(x, c, c)


def test_python_api_shape_errors():
    import torch
    from gpt_from_scratch_amd import apply_flash_attn, apply_rope
    q = torch.randn(1, 1, 64, 64)
    with pytest.raises(AssertionError):
        apply_flash_attn(q, q[:, :, :32], q)
    with pytest.raises(AssertionError, match="even"):
        apply_rope(torch.randn(4, 1, 1, 7), torch.ones(4, 3), torch.ones(4, 3))


def test_attention_stats_and_gradient_checks():
    """lse must be dense fp32 [B, H, S] and dO must match q: checked before
    any launch (the kernels index them as (b*H + h)*S + s)."""
    import torch
    from gpt_from_scratch_amd import flash_attn_backward
    q = torch.randn(1, 2, 8, 16)
    m = torch.zeros(1, 2, 8)
    for bad_m in (m.double(), torch.zeros(1, 2, 16)[:, :, ::2], torch.zeros(2, 1, 8)):
        with pytest.raises(ValueError, match="lse"):
            flash_attn_backward(q, q, q, q, bad_m, q)
    with pytest.raises(ValueError, match="do"):
        flash_attn_backward(q, q, q, q, m, torch.randn(1, 2, 8, 8))
    with pytest.raises(ValueError, match="do"):
        flash_attn_backward(q, q, q, q, m, q.double())
    with pytest.raises(RuntimeError, match="ROCm GPUs only"):
        flash_attn_backward(q, q, q, q, m, q)


def test_attention_block_shape_errors():
    """The fused block checks its [S, B, 3*H*D] input before any launch."""
    import torch
    from gpt_from_scratch_amd import attention_block
    cos, sin = torch.ones(8, 2), torch.ones(8, 2)
    with pytest.raises(ValueError, match="3 \\* heads"):
        attention_block(torch.randn(8, 2, 10), cos, sin, 2)
    with pytest.raises(ValueError):
        attention_block(torch.randn(8, 30), cos, sin, 2)
    with pytest.raises(AssertionError, match="even"):
        attention_block(torch.randn(8, 2, 18), cos, sin, 2)
    # tables shorter than the sequence, narrower than D/2, or not 2-D
    qkv = torch.randn(8, 2, 24)
    for c in (torch.ones(7, 2), torch.ones(8, 1), torch.ones(8), torch.ones(1, 8, 2)):
        with pytest.raises(ValueError, match="cos"):
            attention_block(qkv, c, torch.ones(8, 2), 2)
    with pytest.raises(ValueError, match="sin"):
        attention_block(qkv, torch.ones(8, 2), torch.ones(4, 2), 2)


def test_rotary_embedding_tables_cpu():
    import torch
    from gpt_from_scratch_amd import RotaryEmbedding
    from oracle import rope_tables
    re_ = RotaryEmbedding(64, max_position_embeddings=16, device="cpu")
    x = torch.zeros(40, 1, 1, 64, dtype=torch.bfloat16)
    cos, sin = re_(x, seq_len=40)  # beyond the cache: regrows
    c, s = rope_tables(64, 40)
    assert cos.dtype == torch.bfloat16 and cos.shape == (40, 32)
    assert torch.equal(cos, c.to(torch.bfloat16)) and torch.equal(sin, s.to(torch.bfloat16))


def test_xent_rejects_bad_arguments_before_launch():
    lib = _lib.lib()
    fake = ctypes.c_void_p(16)
    V = 50257
    # rows <= 0, vocab <= 0
    assert lib.mi_xent_fwd(2, 0, V, fake, V, fake, fake, fake, None) == 1
    assert lib.mi_xent_fwd(2, 4, 0, fake, V, fake, fake, fake, None) == 1
    # row stride shorter than a row
    assert lib.mi_xent_fwd(2, 4, V, fake, V - 1, fake, fake, fake, None) == 1
    assert b"row_stride" in lib.mi_last_error()
    # null / misaligned pointers
    assert lib.mi_xent_fwd(2, 4, V, None, V, fake, fake, fake, None) == 1
    assert lib.mi_xent_fwd(2, 4, V, ctypes.c_void_p(17), V, fake, fake, fake, None) == 1
    assert b"misaligned" in lib.mi_last_error()
    assert lib.mi_xent_fwd(9, 4, V, fake, V, fake, fake, fake, None) == 1
    # backward: in-place needs the same row stride
    assert lib.mi_xent_bwd(2, 4, V, fake, V + 3, fake, fake, fake, fake, V, None) == 1
    assert b"in-place" in lib.mi_last_error()
    assert lib.mi_xent_bwd(2, 4, V, fake, V, fake, fake, None, fake, V, None) == 1


def test_cross_entropy_python_checks():
    import torch
    from gpt_from_scratch_amd import vocab_parallel_cross_entropy
    z = torch.randn(4, 3, 10)
    with pytest.raises(ValueError, match="target shape"):
        vocab_parallel_cross_entropy(z, torch.zeros(4, dtype=torch.int64))
    with pytest.raises(TypeError, match="integer"):
        vocab_parallel_cross_entropy(z, torch.zeros(4, 3))
    with pytest.raises(RuntimeError, match="ROCm GPUs only"):
        vocab_parallel_cross_entropy(z, torch.zeros(4, 3, dtype=torch.int64))


def test_model_op_entry_points_reject_bad_arguments():
    lib = _lib.lib()
    fake = ctypes.c_void_p(16)
    # RMSNorm: weight dtype must be x's or fp32; row stride >= hidden; workspace size
    assert lib.mi_rmsnorm_fwd(2, 1, 4, 768, 1e-6, fake, 768, fake, fake, 768, fake, None) == 1
    assert b"weight" in lib.mi_last_error()
    assert lib.mi_rmsnorm_fwd(2, 2, 4, 768, 1e-6, fake, 700, fake, fake, 768, fake, None) == 1
    assert lib.mi_rmsnorm_fwd(2, 2, 4, 768, -1.0, fake, 768, fake, fake, 768, fake, None) == 1
    assert b"eps" in lib.mi_last_error()
    need = lib.mi_rmsnorm_bwd_workspace(4, 768)
    assert need == 768 and lib.mi_rmsnorm_bwd_workspace(0, 768) == 0
    assert lib.mi_rmsnorm_bwd(2, 2, 4, 768, fake, 768, fake, fake, fake, 768, fake, 768, fake,
                              fake, need - 1, None) == 1
    assert b"workspace" in lib.mi_last_error()
    # SwiGLU: gate_up rows must hold 2 * inter elements
    assert lib.mi_swiglu_fwd(2, 4, 3072, fake, 3072, fake, 3072, None) == 1
    assert lib.mi_swiglu_bwd(2, 4, 3072, fake, 6144, None, 3072, fake, 6144, None) == 1
    assert b"dout" in lib.mi_last_error()
    # optimizer: workspace size, clip without a norm, non-finite hyperparameters
    ws = lib.mi_adamw_workspace()
    assert ws > 1
    assert lib.mi_grad_sumsq(2, 100, fake, fake, ws - 1, None) == 1
    hp = [0.99997, 0.1, 0.95, 0.05, 3e-3, 0.2236, 1e-8]
    assert lib.mi_adamw_step(2, 2, 100, fake, fake, fake, fake, fake, *hp, 1.0, None, None) == 1
    assert b"grad_sumsq" in lib.mi_last_error()
    assert lib.mi_adamw_step(2, 2, 100, fake, fake, fake, fake, fake, *hp[:-1], float("nan"),
                             0.0, None, None) == 1
    assert lib.mi_adamw_step(2, 2, 0, fake, fake, fake, fake, fake, *hp, 0.0, None, None) == 1


def test_model_op_python_checks():
    import torch
    from gpt_from_scratch_amd import DistributedOptimizer, rms_norm, swiglu
    with pytest.raises(ValueError, match="even"):
        swiglu(torch.randn(4, 7))
    with pytest.raises(RuntimeError, match="ROCm GPUs only"):
        swiglu(torch.randn(4, 8))
    with pytest.raises(ValueError, match="last dim"):
        rms_norm(torch.randn(4, 8), torch.ones(7))
    with pytest.raises(RuntimeError, match="ROCm GPUs only"):
        rms_norm(torch.randn(4, 8), torch.ones(8))
    with pytest.raises(RuntimeError, match="ROCm GPUs only"):
        DistributedOptimizer(torch.nn.Linear(4, 3), torch.optim.AdamW, {"lr": 1e-2})


def test_rows_view_of_model_op_tensors():
    """The row view the model-operator bindings hand to the C ABI: leading dims
    collapse into one row axis; overlapping rows (a broadcast row axis, stride
    0) and non-collapsible strides raise ValueError, which the modules answer
    with a contiguous copy."""
    import torch
    from gpt_from_scratch_amd import _lib
    x = torch.zeros(6, 4, 10)
    assert _lib._rows(x) == (24, 10)
    assert _lib._rows(torch.zeros(7, 10)[:, :5]) == (7, 10)
    assert _lib._rows(torch.zeros(10)) == (1, 10)
    assert _lib._rows(torch.zeros(10).expand(1, 10))[0] == 1  # one row: its stride is unused
    for bad in (torch.zeros(10).expand(5, 10), torch.zeros(3, 1, 10).expand(3, 4, 10),
                torch.zeros(4, 6, 10).transpose(0, 1)):
        with pytest.raises(ValueError):
            _lib._rows(bad)
    from gpt_from_scratch_amd.mlp import _rows_view as mlp_rows
    from gpt_from_scratch_amd.normalization import _rows_view as norm_rows
    b = torch.arange(10.).expand(5, 10)
    for f in (mlp_rows, norm_rows):
        c = f(b)
        assert c.is_contiguous() and torch.equal(c, b)


def test_new_entry_points_reject_bad_arguments():
    """mi_rmsnorm_add_fwd / _bwd and mi_attn_bwd_rope validate before any launch."""
    lib = _lib.lib()
    fake = ctypes.c_void_p(16)
    # fused add + RMSNorm: the residual and the sum are required, with full rows
    assert lib.mi_rmsnorm_add_fwd(2, 2, 4, 768, 1e-6, fake, 768, None, 768, fake, fake, 768,
                                  fake, 768, fake, None) == 1
    assert b"residual" in lib.mi_last_error()
    assert lib.mi_rmsnorm_add_fwd(2, 2, 4, 768, 1e-6, fake, 768, fake, 700, fake, fake, 768,
                                  fake, 768, fake, None) == 1
    assert b"row stride" in lib.mi_last_error()
    need = lib.mi_rmsnorm_bwd_workspace(4, 768)
    assert lib.mi_rmsnorm_add_bwd(2, 2, 4, 768, fake, 768, fake, fake, fake, 768, None, 768,
                                  fake, 768, fake, fake, need, None) == 1
    assert b"dsum" in lib.mi_last_error()
    assert lib.mi_rmsnorm_add_bwd(2, 2, 4, 768, fake, 768, fake, fake, fake, 768, fake, 768,
                                  fake, 768, fake, fake, need - 1, None) == 1
    assert b"workspace" in lib.mi_last_error()
    # backward with the fused inverse rotation: the tables are checked like the tensors
    st = _i4(0, 0, 64, 1)
    t2 = (ctypes.c_int64 * 2)(32, 1)
    args = [2, 1, 1, 64, 64, 1, 0.125] + [fake, st] * 5 + [fake, fake] + [fake, st] * 3
    assert lib.mi_attn_bwd_rope(*args, 7, fake, t2, fake, t2, None) == 1
    assert b"table dtype" in lib.mi_last_error()
    assert lib.mi_attn_bwd_rope(*args, 2, None, t2, fake, t2, None) == 1
    assert b"cos/sin" in lib.mi_last_error()
    odd = [2, 1, 1, 64, 63, 1, 0.125] + args[7:]
    assert lib.mi_attn_bwd_rope(*odd, 2, fake, t2, fake, t2, None) != 0
    # fp32 tables are rotated by a separate inverse-RoPE pass after the gradient
    # kernels; a shape past that pass's launch limit (2^31 angle pairs) is
    # refused before the preprocess or the gradients are enqueued
    big = [2, 1, 512, 65536, 64, 1, 0.125] + args[7:]
    assert lib.mi_attn_bwd_rope(*big, 0, fake, t2, fake, t2, None) == 2
    assert b"too large" in lib.mi_last_error()


def test_second_build_in_one_process_is_refused(tmp_path):
    """A process holds one build of the library: a second copy loaded from
    another path refuses every launching entry point (the first keeps working),
    and a child process makes its own claim."""
    import shutil
    import subprocess
    import sys
    dup = tmp_path / "libmi_attn_copy.so"
    shutil.copy(_lib.LIB_PATH, dup)
    code = f"""
import ctypes, torch
def load(path):
    lib = ctypes.CDLL(path)
    lib.mi_last_error.restype = ctypes.c_char_p
    return lib
a, b = load({_lib.LIB_PATH!r}), load({str(dup)!r})
st = (ctypes.c_int64 * 4)(0, 0, 64, 1)
f = ctypes.c_void_p(16)
args = (1, 1, 64, 64, 1, ctypes.c_float(0.125), f, st, f, st, f, st, f, st, f, None)
assert a.mi_attn_fwd(7, *args) == 1 and b"dtype" in a.mi_last_error()
assert b.mi_attn_fwd(7, *args) == 2, b.mi_last_error()
assert b"another build" in b.mi_last_error()
assert {os.path.realpath(_lib.LIB_PATH)!r}.encode() in b.mi_last_error()
print("ok")
"""
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stderr[-2000:]
