"""Text renderings of the IR, printed when ``ATTNFUSE_DEBUG`` is set
(reference behaviour: attnfuse/ir/printer.py:10-83, attnfuse/dsl/api.py:140-143)."""
from __future__ import annotations

from .high_level import (BiasOp, Graph, MaskOp, MatMulPV, NormOp, ScoreOp,
                         TensorSym)
from .spec import SpecKey


def _sym(t: TensorSym) -> str:
    return (f"{t.name}[{t.batch}x{t.num_heads}x{t.seqlen}x{t.head_dim} "
            f": {t.dtype}]")


def _node_lines(node, depth: int) -> list:
    pad = "  " * depth
    if isinstance(node, TensorSym):
        return [pad + _sym(node)]
    if isinstance(node, ScoreOp):
        head = f"ScoreOp({node.kind.value}, scale={node.scale}"
        head += ", rope)" if node.rope else ")"
        return ([pad + head] + _node_lines(node.q, depth + 1)
                + _node_lines(node.k, depth + 1))
    if isinstance(node, MaskOp):
        w = f", window={node.window}" if node.window is not None else ""
        return [pad + f"MaskOp({node.kind.value}{w})"] + _node_lines(
            node.scores, depth + 1)
    if isinstance(node, BiasOp):
        h = f", num_heads={node.num_heads}" if node.num_heads else ""
        return [pad + f"BiasOp({node.kind.value}{h})"] + _node_lines(
            node.scores, depth + 1)
    if isinstance(node, NormOp):
        return [pad + f"NormOp({node.kind.value})"] + _node_lines(
            node.scores, depth + 1)
    if isinstance(node, MatMulPV):
        return ([pad + "MatMulPV"] + _node_lines(node.probs, depth + 1)
                + _node_lines(node.v, depth + 1))
    return [pad + repr(node)]


def format_graph(g: Graph) -> str:
    lines = [f"# Graph(signature={g.signature()})",
             f"  Q : {_sym(g.q)}", f"  K : {_sym(g.k)}", f"  V : {_sym(g.v)}",
             "  root:"]
    lines += _node_lines(g.root, 2)
    return "\n".join(lines)


def format_key(k: SpecKey) -> str:
    c = k.config
    mask = k.mask_kind.value + (f" (window={k.mask_window})"
                                if k.mask_window else "")
    bias = (k.bias_kind.value if k.bias_kind else "none") + (
        f" (heads={k.bias_num_heads})" if k.bias_num_heads else "")
    return "\n".join([
        f"# SpecKey(cache_key={k.cache_key})",
        f"  dtype           = {k.dtype}",
        f"  head_dim        = {k.head_dim}",
        f"  score_scale     = {k.score_scale}",
        f"  mask            = {mask}",
        f"  bias            = {bias}",
        f"  norm            = {k.norm_kind.value}",
        f"  rope            = {k.rope_kind}",
        f"  BLOCK_M/BLOCK_N = {c.BLOCK_M}/{c.BLOCK_N}",
        f"  waves           = {c.waves}",
        f"  lds_stages      = {c.lds_stages}",
    ])


# Reference name for the lowered-record printer.
format_tiled = format_key
