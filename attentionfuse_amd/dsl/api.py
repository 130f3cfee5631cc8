"""User-facing DSL: the ``@attention`` decorator and its combinators.

The surface is the reference's (reference: attnfuse/dsl/api.py:36-201), so
code written for ``import attnfuse as af`` runs unchanged.  Combinators build
IR nodes while a function is traced; ``@attention`` traces once per
``(head_dim, dtype)`` and routes each call to

* the block-sparse kernels when the graph has ``af.block_sparse`` (a
  ``block_mask=`` is then required),
* the autograd path (forward saves the log-sum-exp, backward runs the HIP
  backward kernels) when an input requires grad and the graph is inside the
  backward scope -- which here includes fused RoPE and block-sparse masks,
* the inference forward otherwise (flash-decoding is chosen inside it for
  single-query calls).

Differences from the reference, all deliberate: a graph's custom ``scale``
is honoured on every route (the reference recomputes 1/sqrt(D) in its
autograd and block-sparse routes), RoPE is honoured on the block-sparse route,
and a graph outside the backward scope warns instead of silently returning an
output with no gradient.
"""
from __future__ import annotations

import functools
import os
import warnings
from typing import Callable

import torch

from ..ir.high_level import (BiasKind, BiasOp, Expr, Graph, MaskKind, MaskOp,
                             NormKind, NormOp, ScoreKind, ScoreOp, TensorSym)
from .tracer import trace_attention_fn


def scaled_dot_product(Q: TensorSym, K: TensorSym,
                       scale: float | None = None) -> Expr:
    """S = (Q @ K^T) * scale, scale defaulting to 1/sqrt(head_dim)."""
    return ScoreOp(kind=ScoreKind.SCALED_DOT, q=Q, k=K, scale=scale)


def rope(Q: TensorSym, K: TensorSym, scale: float | None = None) -> Expr:
    """S = (RoPE(Q) @ RoPE(K)^T) * scale with the rotation fused in-kernel.

    Pass the tables at call time: ``fn(Q, K, V, cos=cos, sin=sin)``, each of
    shape (N, D) or (1, 1, N, D) in Q's dtype (``rope_utils.build_rope_cache``).
    """
    return ScoreOp(kind=ScoreKind.SCALED_DOT, q=Q, k=K, scale=scale, rope=True)


def additive_bias(scores: Expr) -> Expr:
    """S + bias, with a (B, H, N_q, N_kv) ``bias=`` tensor given at call time."""
    return BiasOp(kind=BiasKind.ADDITIVE, scores=scores)


def causal(scores: Expr) -> Expr:
    """Key j is masked for query i when j > i."""
    return MaskOp(kind=MaskKind.CAUSAL, scores=scores)


def sliding_window(scores: Expr, window_size: int) -> Expr:
    """Key j is masked for query i when |i - j| >= window_size."""
    if window_size <= 0:
        raise ValueError("sliding_window: window_size must be positive")
    return MaskOp(kind=MaskKind.SLIDING_WINDOW, scores=scores,
                  window=window_size)


def full(scores: Expr) -> Expr:
    """No mask (explicit dense)."""
    return MaskOp(kind=MaskKind.FULL, scores=scores)


def block_sparse(scores: Expr) -> Expr:
    """Block-sparse mask supplied at call time as ``block_mask=BlockMask``
    (see ``create_block_mask``); only the listed tiles are visited."""
    return MaskOp(kind=MaskKind.BLOCK_SPARSE, scores=scores)


def alibi(scores: Expr, num_heads: int) -> Expr:
    """ALiBi bias -slope_h * |i - j| (Press et al., 2021)."""
    if num_heads <= 0:
        raise ValueError("alibi: num_heads must be positive")
    return BiasOp(kind=BiasKind.ALIBI, scores=scores, num_heads=num_heads)


def softmax(scores: Expr) -> Expr:
    """Row softmax, computed as an online (streaming) softmax in-kernel."""
    return NormOp(kind=NormKind.SOFTMAX, scores=scores)


def relu_attention(scores: Expr) -> Expr:
    """ReLU normalisation: max(S, 0) divided by its row sum."""
    return NormOp(kind=NormKind.RELU, scores=scores)


def _wants_grad(*ts) -> bool:
    return torch.is_grad_enabled() and any(
        isinstance(t, torch.Tensor) and t.requires_grad for t in ts)


def attention(fn: Callable) -> Callable:
    """Decorator: trace ``fn`` written with the combinators above."""
    graphs: dict = {}

    @functools.wraps(fn)
    def wrapper(Q, K, V, *, bias=None, cos=None, sin=None, block_mask=None,
                return_graph: bool = False, **kwargs):
        key = (Q.shape[-1], str(Q.dtype))
        graph = graphs.get(key)
        if graph is None:
            graph = trace_attention_fn(fn, Q, K, V)
            graphs[key] = graph
            if os.environ.get("ATTNFUSE_DEBUG"):
                from ..ir.printer import format_graph
                print(f"[AttnFuse] traced graph (head_dim={key[0]}, "
                      f"dtype={key[1]}):\n{format_graph(graph)}")
        if return_graph:
            return graph
        return _route(graph, Q, K, V, bias, cos, sin, block_mask, kwargs)

    wrapper.graph_fn = fn  # type: ignore[attr-defined]
    return wrapper


# Call-time keywords beyond the reference's (bias, cos, sin, block_mask):
# explicit ALiBi slopes on every route; an output buffer, a saved
# log-sum-exp and tile-visit counters on the inference forward only.
_INFERENCE_ONLY_KWARGS = ("out", "save_lse", "coverage")


def _route(graph: Graph, Q, K, V, bias, cos, sin, block_mask, kwargs):
    from ..runtime.backward import can_backward
    masks = {m.kind for m in graph.collect_masks()}
    grad = _wants_grad(Q, K, V)
    unknown = set(kwargs) - {"alibi_slopes", *_INFERENCE_ONLY_KWARGS}
    if unknown:
        raise TypeError(f"unexpected keyword arguments {sorted(unknown)}")
    slopes = kwargs.get("alibi_slopes")
    autograd = grad and can_backward(graph)
    if autograd and set(kwargs) & set(_INFERENCE_ONLY_KWARGS):
        raise ValueError(
            f"{sorted(set(kwargs) & set(_INFERENCE_ONLY_KWARGS))} are not "
            "supported when an input requires grad (the autograd path "
            "allocates its own output and log-sum-exp)")

    if MaskKind.BLOCK_SPARSE in masks:
        from ..runtime.block_mask import BlockMask, run_block_sparse_graph
        if block_mask is None:
            raise RuntimeError(
                "this graph uses af.block_sparse(); pass block_mask=<BlockMask> "
                "at call time (build one with "
                "attnfuse.create_block_mask(predicate, Q_LEN, KV_LEN))")
        if not isinstance(block_mask, BlockMask):
            raise TypeError("block_mask must be an attnfuse.BlockMask")
        if autograd:
            from ..runtime.autograd import AttnFuseFunction
            return AttnFuseFunction.apply(graph, Q, K, V, bias, cos, sin,
                                          block_mask, slopes)
        if grad:
            warnings.warn("AttnFuse: no backward for this block-sparse graph; "
                          "the output carries no gradient", stacklevel=3)
        if kwargs.get("coverage") is not None:
            raise ValueError("coverage= is taken by the dense/causal/windowed "
                             "forward; use runtime.run_block_sparse for "
                             "block-sparse counters")
        return run_block_sparse_graph(graph, Q, K, V, block_mask, cos=cos,
                                      sin=sin, out=kwargs.get("out"),
                                      save_lse=kwargs.get("save_lse"),
                                      alibi_slopes=slopes)

    if grad:
        if autograd:
            from ..runtime.autograd import AttnFuseFunction
            return AttnFuseFunction.apply(graph, Q, K, V, bias, cos, sin, None,
                                          slopes)
        warnings.warn("AttnFuse: this graph is outside the backward scope "
                      "(softmax with full/causal/sliding-window/block-sparse "
                      "masks and none/ALiBi bias); the output carries no "
                      "gradient", stacklevel=3)
    from ..runtime.dispatch import run_attention
    return run_attention(graph, Q, K, V, bias=bias, cos=cos, sin=sin, **kwargs)
