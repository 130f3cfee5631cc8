"""AttnFuse on MI355X: the attention DSL backed by hand-written gfx950 HIP
kernels.

Public surface (the reference's, attnfuse/__init__.py:26-58)::

    import attnfuse as af          # or: import attentionfuse_amd as af

    @af.attention
    def gpt2_attn(Q, K, V):
        return af.softmax(af.causal(af.scaled_dot_product(Q, K))) @ V

    out = gpt2_attn(q, k, v)       # runs the ahead-of-time compiled kernel
"""
from .dsl.api import (additive_bias, alibi, attention, block_sparse, causal,
                      full, relu_attention, rope, scaled_dot_product,
                      sliding_window, softmax)
from .runtime.block_mask import BlockMask, create_block_mask

__version__ = "1.0.0"

__all__ = [
    "attention", "scaled_dot_product", "additive_bias", "rope", "causal",
    "sliding_window", "full", "block_sparse", "alibi", "softmax",
    "relu_attention", "BlockMask", "create_block_mask", "__version__",
]
