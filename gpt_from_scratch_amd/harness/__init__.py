"""Config-5 harness: a GPT train step at TP=1/DP=1 that calls the attention
hot path (see gpt.py)."""
from .gpt import GPT, GPTConfig, MixedPrecisionAdamW, SoftmaxCrossEntropy, synthetic_batch, train

__all__ = ["GPT", "GPTConfig", "MixedPrecisionAdamW", "SoftmaxCrossEntropy", "synthetic_batch",
           "train"]
