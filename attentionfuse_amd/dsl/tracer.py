"""Trace a user attention function on symbolic tensors into a Graph.

Behaviour follows the reference tracer (reference:
attnfuse/dsl/tracer.py:24-85): inputs must be 4-D (B, H, N, D), Q/K/V share
the head dimension, the function must return ``probs @ V`` and ``probs`` must
come from a normalisation combinator.
"""
from __future__ import annotations

from typing import Callable

from ..ir.high_level import Graph, MatMulPV, NormOp, TensorSym


def _sym(name: str, t) -> TensorSym:
    shape = tuple(t.shape)
    if len(shape) != 4:
        raise ValueError(
            f"AttnFuse expects Q/K/V of shape (B, H, N, D); {name} has {shape}")
    return TensorSym(name=name, batch=shape[0], num_heads=shape[1],
                     seqlen=shape[2], head_dim=shape[3],
                     dtype=str(t.dtype).replace("torch.", ""))


def trace_attention_fn(fn: Callable, Q, K, V) -> Graph:
    qs, ks, vs = _sym("Q", Q), _sym("K", K), _sym("V", V)
    if qs.head_dim != ks.head_dim:
        raise ValueError(f"head_dim mismatch: Q has {qs.head_dim}, "
                         f"K has {ks.head_dim}")
    if vs.head_dim != qs.head_dim:
        raise ValueError("AttnFuse requires Q.head_dim == V.head_dim")
    out = fn(qs, ks, vs)
    if not isinstance(out, MatMulPV):
        raise TypeError(
            "the attention function must return `probs @ V`, got "
            f"{type(out).__name__}; did you forget the value projection?")
    if not isinstance(out.probs, NormOp):
        raise TypeError(
            "the probabilities multiplied with V must come from a "
            "normalisation combinator (af.softmax / af.relu_attention)")
    return Graph(q=qs, k=ks, v=vs, root=out)
