"""Test infrastructure: CPU restatement of the reference's attention, RoPE,
vocabulary cross entropy, RMSNorm, SwiGLU and optimizer step.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg may
import this package, and only as the checker (or the timed CPU baseline).  The
product (gpt_from_scratch_amd) never imports it.
"""
from .attention import (attention_backward, attention_bruteforce, attention_forward,
                        attention_forward_backward_chunked, attention_probs)
from .cross_entropy import cross_entropy_backward, cross_entropy_forward
from .mlp import swiglu_backward, swiglu_forward
from .normalization import rmsnorm_backward, rmsnorm_forward
from .optimizer import adamw_step, clip_gradient
from .rope import rope_apply, rope_tables, rope_tables_f64

__all__ = ["attention_forward", "attention_backward", "attention_probs",
           "attention_bruteforce", "attention_forward_backward_chunked",
           "rope_apply", "rope_tables", "rope_tables_f64",
           "cross_entropy_forward", "cross_entropy_backward",
           "rmsnorm_forward", "rmsnorm_backward", "swiglu_forward", "swiglu_backward",
           "adamw_step", "clip_gradient"]
