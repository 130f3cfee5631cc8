"""torch.autograd bindings (reference: attnfuse/runtime/autograd.py:31-97).

``AttnFuseFunction`` covers every graph in the backward scope, block-sparse
included: forward runs the HIP forward with the log-sum-exp saved, backward
runs the HIP backward.  The graph's own score scale is used in both passes.
``AttnFuseBlockSparseFunction`` keeps the reference's block-sparse binding
signature.
"""
from __future__ import annotations

import torch

from .backward import run_backward


class AttnFuseFunction(torch.autograd.Function):

    @staticmethod
    def forward(ctx, graph, Q, K, V, bias, cos, sin, block_mask=None,
                alibi_slopes=None):
        from .dispatch import run_attention
        from .kernel_cache import get_or_compile
        B, Hq, Nq, _ = Q.shape
        L = torch.empty(B, Hq, Nq, dtype=torch.float32, device=Q.device)
        bundle = get_or_compile(graph)
        if block_mask is not None:
            from .block_mask import run_block_sparse_graph
            out = run_block_sparse_graph(graph, Q, K, V, block_mask, cos=cos,
                                         sin=sin, save_lse=L,
                                         alibi_slopes=alibi_slopes)
        else:
            out = run_attention(graph, Q, K, V, bias=bias, cos=cos, sin=sin,
                                save_lse=L, alibi_slopes=alibi_slopes)
        ctx.graph = graph
        ctx.sm_scale = bundle.sm_scale
        ctx.block_mask = block_mask
        ctx.rope = (cos, sin) if bundle.has_rope else (None, None)
        ctx.alibi_slopes = alibi_slopes if bundle.bias_kind == 1 else None
        ctx.save_for_backward(Q, K, V, out, L)
        return out

    @staticmethod
    def backward(ctx, dO):
        Q, K, V, O, L = ctx.saved_tensors
        cos, sin = ctx.rope
        dQ, dK, dV = run_backward(ctx.graph, Q, K, V, O, L, dO.contiguous(),
                                  ctx.sm_scale, cos=cos, sin=sin,
                                  block_mask=ctx.block_mask,
                                  alibi_slopes=ctx.alibi_slopes)
        return None, dQ, dK, dV, None, None, None, None, None


class AttnFuseBlockSparseFunction(torch.autograd.Function):
    """Block-sparse binding with the reference signature
    ``apply(Q, K, V, block_mask, bias_kind)`` (scale 1/sqrt(D))."""

    @staticmethod
    def forward(ctx, Q, K, V, block_mask, bias_kind: int):
        from .block_mask import run_block_sparse
        B, Hq, Nq, D = Q.shape
        scale = 1.0 / (D ** 0.5)
        L = torch.empty(B, Hq, Nq, dtype=torch.float32, device=Q.device)
        out = run_block_sparse(Q, K, V, block_mask, scale,
                               bias_kind=bias_kind, save_lse=L)
        ctx.block_mask, ctx.scale, ctx.bias_kind = block_mask, scale, bias_kind
        ctx.save_for_backward(Q, K, V, out, L)
        return out

    @staticmethod
    def backward(ctx, dO):
        from .block_mask import run_block_sparse_backward
        Q, K, V, O, L = ctx.saved_tensors
        dQ, dK, dV = run_block_sparse_backward(
            Q, K, V, O, L, dO.contiguous(), ctx.block_mask, ctx.scale,
            ctx.bias_kind)
        return dQ, dK, dV, None, None
