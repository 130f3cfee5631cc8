"""Lowering: Graph -> SpecKey.

Same folding rules as the reference lowering
(reference: attnfuse/compiler/lowering.py:20-85):

* the score scale defaults to 1/sqrt(head_dim);
* causal + sliding_window lowers to one causal-window mask (key j visible to
  query i iff i - W < j <= i); any other pair of masks is rejected.  The
  reference folds this pair to the plain (two-sided) window
  (attnfuse/compiler/lowering.py:32-46), which lets each query see W-1 future
  keys -- a different function from the graph the user wrote;
* at most one bias op;
* ``rope_kind`` is 1 when the score op carries fused RoPE.
"""
from __future__ import annotations

import math

from ..ir.high_level import Graph, MaskKind, ScoreKind
from ..ir.spec import SpecKey
from .fusion import fuse_score_softmax
from .tiling import tile_for_key


def lower_to_key(graph: Graph) -> SpecKey:
    fuse_score_softmax(graph)
    score = graph.score()
    if score.kind is not ScoreKind.SCALED_DOT:
        raise NotImplementedError(f"score kind {score.kind} is not supported")
    head_dim = graph.q.head_dim
    scale = score.scale if score.scale is not None else 1.0 / math.sqrt(head_dim)

    masks = graph.collect_masks()
    kinds = {m.kind for m in masks}
    if len(masks) > 1:
        if kinds == {MaskKind.CAUSAL, MaskKind.SLIDING_WINDOW}:
            sw = next(m for m in masks if m.kind is MaskKind.SLIDING_WINDOW)
            mask_kind, window = MaskKind.CAUSAL_SLIDING_WINDOW, sw.window
        else:
            raise NotImplementedError(
                f"mask combination {sorted(k.value for k in kinds)} is not "
                "supported")
    elif masks:
        mask_kind, window = masks[0].kind, masks[0].window
    else:
        mask_kind, window = MaskKind.FULL, None

    biases = graph.collect_biases()
    if len(biases) > 1:
        raise NotImplementedError("at most one bias op per graph")
    bias_kind = biases[0].kind if biases else None
    bias_heads = biases[0].num_heads if biases else None

    key = SpecKey(
        head_dim=head_dim, dtype=graph.q.dtype, score_scale=float(scale),
        mask_kind=mask_kind, mask_window=window, bias_kind=bias_kind,
        bias_num_heads=bias_heads, norm_kind=graph.norm().kind,
        rope_kind=1 if score.rope else 0, cache_key=graph.signature())
    # the launch shape the library uses for this key (single source)
    key.config = tile_for_key(key.abi_tuple())
    return key


# Reference name of the lowering entry point.
lower_to_tiled = lower_to_key


def kernel_constexprs(key: SpecKey) -> dict:
    """The specialisation flags as a dict (reference field names,
    attnfuse/compiler/codegen.py:391-404)."""
    return {
        "HEAD_DIM": key.head_dim,
        "BLOCK_M": key.config.BLOCK_M,
        "BLOCK_N": key.config.BLOCK_N,
        "MASK_KIND": key.mask_code,
        "BIAS_KIND": key.bias_code,
        "NORM_KIND": key.norm_code,
        "ROPE_KIND": int(key.rope_kind),
        "WINDOW": key.mask_window or 0,
        "DTYPE": key.dtype_code,
    }
