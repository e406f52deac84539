"""MI355X-native attention hot path of gpt_from_scratch.

Drop-ins for the reference's kernels (core/myFlashAttn.py, core/rope_triton.py,
core/position_embeddings.py), its vocabulary cross entropy
(core/tensor_parallel/loss.py), RMSNorm (core/normalization.py), SwiGLU
(core/mlp.py) and optimizer step (core/optimizer.py), backed by hand-written gfx950 HIP kernels in
libmi_attn.so behind the C ABI of include/mi_attn.h.
"""
from .attention_block import AttentionBlock, attention_block
from .cross_entropy import (VocabParallelCrossEntropy, _VocabParallelCrossEntropy,
                            vocab_parallel_cross_entropy)
from .mlp import ParallelMLP, SwiGLU, swiglu
from .normalization import FusedAddRMSNorm, FusedRMSNorm, RMSNorm, add_rms_norm, rms_norm
from .optimizer import DistributedOptimizer
from .flash_attn import FlashAttn, apply_flash_attn, flash_attn_backward, flash_attn_forward
from .position_embeddings import RotaryEmbedding
from .rope import RoPE, RoPEQK, TritonRoPE, apply_rope, apply_rope_qk

__all__ = [
    "FlashAttn", "apply_flash_attn", "flash_attn_forward", "flash_attn_backward",
    "RotaryEmbedding", "RoPE", "RoPEQK", "TritonRoPE", "apply_rope", "apply_rope_qk",
    "AttentionBlock", "attention_block",
    "VocabParallelCrossEntropy", "_VocabParallelCrossEntropy", "vocab_parallel_cross_entropy",
    "RMSNorm", "FusedRMSNorm", "rms_norm", "FusedAddRMSNorm", "add_rms_norm", "SwiGLU", "swiglu", "ParallelMLP",
    "DistributedOptimizer",
]
