"""Attention IR: the traced dataflow graph and its lowered specialisation key."""
from .high_level import (BiasKind, BiasOp, Expr, Graph, MaskKind, MaskOp,
                         MatMulPV, NormKind, NormOp, ScoreKind, ScoreOp,
                         TensorSym)
from .printer import format_graph, format_key, format_tiled
from .spec import SpecKey, TileConfig, TiledKernel

__all__ = [
    "Expr", "TensorSym", "ScoreOp", "MaskOp", "BiasOp", "NormOp", "MatMulPV",
    "Graph", "ScoreKind", "MaskKind", "BiasKind", "NormKind",
    "SpecKey", "TiledKernel", "TileConfig",
    "format_graph", "format_key", "format_tiled",
]
