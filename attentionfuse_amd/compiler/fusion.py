"""Fusion check: the graph must be the chain
``score -> (mask | bias)* -> norm -> @V`` so that one tiled online-softmax
kernel computes it (reference contract: attnfuse/compiler/fusion.py:28-56)."""
from __future__ import annotations

from ..ir.high_level import (BiasOp, Graph, MaskOp, MatMulPV, NormKind,
                             NormOp, ScoreOp)


class FusionError(RuntimeError):
    """The traced graph is not a fusable attention pipeline."""


def fuse_score_softmax(graph: Graph) -> Graph:
    root = graph.root
    if not isinstance(root, MatMulPV):
        raise FusionError("graph root must be MatMulPV (probs @ V)")
    norm = root.probs
    if not isinstance(norm, NormOp):
        raise FusionError("probs @ V needs probs from a normalisation "
                          "combinator (softmax / relu_attention)")
    if norm.kind not in (NormKind.SOFTMAX, NormKind.RELU):
        raise FusionError(f"unsupported normalisation {norm.kind}")
    node = norm.scores
    while isinstance(node, (MaskOp, BiasOp)):
        node = node.scores
    if not isinstance(node, ScoreOp):
        raise FusionError("expected norm <- (mask|bias)* <- score, reached "
                          f"{type(node).__name__}")
    return graph
