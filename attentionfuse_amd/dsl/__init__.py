"""Attention DSL: decorator + combinators."""
from .api import (additive_bias, alibi, attention, block_sparse, causal, full,
                  relu_attention, rope, scaled_dot_product, sliding_window,
                  softmax)
from .tracer import trace_attention_fn

__all__ = ["attention", "scaled_dot_product", "additive_bias", "rope",
           "causal", "sliding_window", "full", "block_sparse", "alibi",
           "softmax", "relu_attention", "trace_attention_fn"]
