"""High-level attention IR: the dataflow graph a traced ``@attention`` function
produces.

The node set and public names follow the reference DSL surface
(reference: attnfuse/ir/high_level.py:23-229) so user code and tests written
against ``attnfuse`` keep working: ``TensorSym`` leaves, ``ScoreOp`` ->
(``MaskOp`` | ``BiasOp``)* -> ``NormOp`` -> ``MatMulPV`` root, and a 16-hex-digit
structural ``Graph.signature()`` that ignores batch / head / sequence sizes.

Nothing here touches device memory; the graph is pure metadata.  The
compiler (``attentionfuse_amd.compiler``) folds a graph into a ``SpecKey`` that
selects one of the ahead-of-time compiled HIP kernel instantiations.
"""
from __future__ import annotations

import enum
import hashlib
from dataclasses import dataclass, field
from typing import Iterator, Optional


class ScoreKind(enum.Enum):
    SCALED_DOT = "scaled_dot"


class MaskKind(enum.Enum):
    FULL = "full"
    CAUSAL = "causal"
    SLIDING_WINDOW = "sliding_window"
    BLOCK_SPARSE = "block_sparse"
    # produced by lowering only: causal + sliding_window (keys i-W < j <= i)
    CAUSAL_SLIDING_WINDOW = "causal_sliding_window"


class BiasKind(enum.Enum):
    ADDITIVE = "additive"
    ALIBI = "alibi"


class NormKind(enum.Enum):
    SOFTMAX = "softmax"
    RELU = "relu"


@dataclass(eq=False)
class Expr:
    """Base node.  ``probs @ V`` inside a traced function builds the root."""

    def __matmul__(self, other):
        if not isinstance(other, TensorSym):
            raise TypeError(
                "the right operand of `@` must be the symbolic V tensor, got "
                f"{type(other).__name__}")
        return MatMulPV(probs=self, v=other)


@dataclass(eq=False)
class TensorSym(Expr):
    """Symbolic (batch, heads, seqlen, head_dim) tensor seen during tracing."""
    name: str
    batch: int
    num_heads: int
    seqlen: int
    head_dim: int
    dtype: str  # "float16" | "bfloat16" | "float32"

    @property
    def shape(self) -> tuple:
        return (self.batch, self.num_heads, self.seqlen, self.head_dim)


@dataclass(eq=False)
class ScoreOp(Expr):
    kind: ScoreKind
    q: TensorSym
    k: TensorSym
    scale: Optional[float] = None  # None means 1/sqrt(head_dim)
    rope: bool = False             # rotary embedding fused into the score


@dataclass(eq=False)
class MaskOp(Expr):
    kind: MaskKind
    scores: Expr
    window: Optional[int] = None   # SLIDING_WINDOW only


@dataclass(eq=False)
class BiasOp(Expr):
    kind: BiasKind
    scores: Expr
    bias: Optional[TensorSym] = None   # ADDITIVE: tensor supplied at call time
    num_heads: Optional[int] = None    # ALIBI only


@dataclass(eq=False)
class NormOp(Expr):
    kind: NormKind
    scores: Expr


@dataclass(eq=False)
class MatMulPV(Expr):
    """Root of every valid graph: ``probs @ V``."""
    probs: Expr
    v: TensorSym


def _children(node) -> list:
    if isinstance(node, ScoreOp):
        return [node.q, node.k]
    if isinstance(node, (MaskOp, NormOp)):
        return [node.scores]
    if isinstance(node, BiasOp):
        return [node.scores] + ([node.bias] if node.bias is not None else [])
    if isinstance(node, MatMulPV):
        return [node.probs, node.v]
    return []


def _node_token(node) -> Optional[str]:
    """Canonical text of one node for the structural signature."""
    if isinstance(node, ScoreOp):
        return f"S({node.kind.value},{node.scale!r},{int(node.rope)})"
    if isinstance(node, MaskOp):
        return f"M({node.kind.value},{node.window!r})"
    if isinstance(node, BiasOp):
        return f"B({node.kind.value},{node.num_heads!r})"
    if isinstance(node, NormOp):
        return f"N({node.kind.value})"
    if isinstance(node, MatMulPV):
        return "PV"
    return None


@dataclass(eq=False)
class Graph:
    q: TensorSym
    k: TensorSym
    v: TensorSym
    root: MatMulPV
    _signature: Optional[str] = field(default=None, repr=False)

    def walk(self) -> Iterator[tuple]:
        """Pre-order (node, parent) pairs from the root; shared nodes once."""
        seen: set = set()
        stack = [(self.root, None)]
        while stack:
            node, parent = stack.pop()
            if id(node) in seen:
                continue
            seen.add(id(node))
            yield node, parent
            for child in reversed(_children(node)):
                stack.append((child, node))

    def collect_masks(self) -> list:
        return [n for n, _ in self.walk() if isinstance(n, MaskOp)]

    def collect_biases(self) -> list:
        return [n for n, _ in self.walk() if isinstance(n, BiasOp)]

    def _only(self, cls, what: str):
        found = [n for n, _ in self.walk() if isinstance(n, cls)]
        if len(found) != 1:
            raise ValueError(
                f"graph must contain exactly one {what} op, found {len(found)}")
        return found[0]

    def norm(self) -> NormOp:
        return self._only(NormOp, "normalisation")

    def score(self) -> ScoreOp:
        return self._only(ScoreOp, "score")

    @property
    def has_rope(self) -> bool:
        return any(isinstance(n, ScoreOp) and n.rope for n, _ in self.walk())

    def signature(self) -> str:
        """16-hex-digit structural hash: variant + head_dim + dtype.

        Batch, head count and sequence lengths do not enter, so one kernel
        instantiation serves every size (reference behaviour,
        attnfuse/ir/high_level.py:183-207)."""
        if self._signature is None:
            toks = [f"dt={self.q.dtype}", f"hd={self.q.head_dim}"]
            toks += [t for t in (_node_token(n) for n, _ in self.walk()) if t]
            digest = hashlib.sha1(";".join(toks).encode()).hexdigest()
            self._signature = digest[:16]
        return self._signature
