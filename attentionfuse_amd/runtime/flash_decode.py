"""Flash-decoding route: one query row per head, split-K over the cache.

Same predicate and signatures as the reference (reference:
attnfuse/runtime/flash_decode.py:46-187): ``Q.N == 1``, ``N_kv >= 256``,
dense mask, no bias or ALiBi, no RoPE -- plus softmax normalisation (the
reference also routes ReLU graphs here and then computes a softmax).

The split workspace is caller-provided at the C ABI.  Here it is one
allocation per call from torch's caching allocator on the current stream, as
the reference allocates its three workspaces per call
(flash_decode.py:134-139): the block is stream-ordered, so concurrent calls
on different streams never share partials, a call under graph capture draws
from the graph's private pool, and freeing it after the launch is safe.
Fixed-shape loops that want no per-call allocation use
``prepared.prepare_decode`` (its own workspace) or the C entry point
``af_decode_noalloc``.
"""
from __future__ import annotations

import torch

from ..ir.high_level import BiasKind, Graph, MaskKind, NormKind
from . import _native as N


def can_use_flash_decode(graph: Graph, Q: torch.Tensor, K: torch.Tensor) -> bool:
    if Q.shape[2] != 1 or K.shape[2] < 256:
        return False
    if {m.kind for m in graph.collect_masks()} - {MaskKind.FULL}:
        return False
    if {b.kind for b in graph.collect_biases()} - {BiasKind.ALIBI}:
        return False
    if graph.has_rope or graph.norm().kind is not NormKind.SOFTMAX:
        return False
    if Q.dtype == torch.float32:
        return Q.shape[-1] in (32, 64, 128)
    return Q.shape[-1] in (32, 64, 128, 256) and Q.dtype in (torch.float16,
                                                              torch.bfloat16)


def _pick_num_splits(B: int, H_q: int, N_kv: int, H_kv: int | None = None,
                     D: int = 128) -> int:
    return int(N.lib().af_decode_num_splits(B, H_q, H_kv or H_q, N_kv, D))


def decode_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """A fresh ``nbytes`` byte buffer from torch's caching allocator, owned
    by the current stream of ``device``."""
    return torch.empty(max(nbytes, 16), dtype=torch.uint8, device=device)


def run_flash_decode(graph: Graph, Q: torch.Tensor, K: torch.Tensor,
                     V: torch.Tensor, sm_scale: float, bias_kind: int,
                     num_heads_kv: int, out: torch.Tensor, *,
                     num_splits: int = 0, alibi_slopes=None,
                     workspace: torch.Tensor | None = None) -> torch.Tensor:
    from .dispatch import _slopes_f32, kernel_layout
    B, H_q, _, D = Q.shape
    _, H_kv, N_kv, _ = K.shape
    if H_kv != num_heads_kv:
        raise ValueError("num_heads_kv does not match K")
    S = num_splits or _pick_num_splits(B, H_q, N_kv, H_kv, D)
    # the library may drop empty trailing splits; size for the request
    nbytes = int(N.lib().af_decode_workspace_bytes(B, H_q, D, S))
    ws = workspace if workspace is not None else decode_workspace(Q.device, nbytes)
    slopes = _slopes_f32(H_q, Q, alibi_slopes) if bias_kind == 1 else None
    Qk, Kk, Vk = kernel_layout(Q), kernel_layout(K), kernel_layout(V)
    a = N.DecodeArgsC()
    dt = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}[Q.dtype]
    a.key = N.SpecKeyC(dt, D, 0, bias_kind, 0, 0)
    a.q, a.k, a.v, a.o = Qk.data_ptr(), Kk.data_ptr(), Vk.data_ptr(), out.data_ptr()
    a.alibi_slopes = N.ptr(slopes)
    a.q_stride[:] = Qk.stride()
    a.k_stride[:] = Kk.stride()
    a.v_stride[:] = Vk.stride()
    a.o_stride[:] = out.stride()
    a.batch, a.heads_q, a.heads_kv, a.seqlen_kv = B, H_q, H_kv, N_kv
    a.scale = float(sm_scale)
    a.num_splits = S
    N.check(N.lib().af_decode(a, ws.data_ptr(), ws.numel() * ws.element_size(),
                              N.stream_handle(Q.device)))
    return out
