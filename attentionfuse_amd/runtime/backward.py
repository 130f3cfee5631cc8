"""Backward route: (Q, K, V, O, L, dO) -> (dQ, dK, dV) via ``af_bwd``.

Keeps the reference signatures (reference: attnfuse/runtime/backward.py:69-192)
and widens the scope the reference accepts ({full, causal} x {none, ALiBi},
no RoPE) to softmax graphs with full, causal, sliding-window or block-sparse
masks, no bias or ALiBi, with or without fused RoPE.  With RoPE the kernels
differentiate through the rotation, so dQ/dK are gradients with respect to
the un-rotated inputs.  dK/dV of a GQA key/value head are summed over its
query-head group inside the kernel (no atomics).
"""
from __future__ import annotations

import torch

from ..ir.high_level import BiasKind, Graph, MaskKind, NormKind
from . import _native as N

_MASK_CODES = {MaskKind.FULL: 0, MaskKind.CAUSAL: 1,
               MaskKind.SLIDING_WINDOW: 2, MaskKind.BLOCK_SPARSE: 3}


def can_backward(graph: Graph) -> bool:
    if graph.norm().kind is not NormKind.SOFTMAX:
        return False
    masks = {m.kind for m in graph.collect_masks()}
    if masks - set(_MASK_CODES):
        return False
    if {b.kind for b in graph.collect_biases()} - {BiasKind.ALIBI}:
        return False
    return True


# Backward launch override, the counterpart of the reference's _BWD_TILE
# (reference: attnfuse/runtime/backward.py:18-47).  On gfx950 the block
# shapes and pipeline depths are fixed per instantiation (128-row dQ and
# 128-key dK/dV workgroups of four waves for 16-bit inputs, or the
# BlockMask's blocks); the runtime choice is how many dK/dV workgroups split
# one key block's GQA query heads.  With "auto" the library picks it
# (``_pick_backward_tile``); otherwise "group_split" (a power of two dividing
# H_q / H_kv) is used as given, e.g.
#     backward._BWD_TILE.update({"auto": False, "group_split": 2})
# The reference's own keys are kept: None means the launch's own value, and
# with "auto" off a set BLOCK_M / BLOCK_N / num_warps must equal the shape the
# launch uses; any other value, and any num_stages, raises ValueError rather
# than being silently ignored.
_BWD_TILE = {
    "BLOCK_M": None,
    "BLOCK_N": None,
    "num_warps": None,
    "num_stages": None,
    "group_split": 0,
    "auto": True,
}
_REFERENCE_KEYS = ("BLOCK_M", "BLOCK_N", "num_warps", "num_stages")

# The dense 16-bit launch shape: what _pick_backward_tile(N_q) reports, the
# reference's call form, which knows only the sequence length.
_DEFAULT_TILE = {"BLOCK_M": 128, "BLOCK_N": 128, "num_warps": 4,
                 "num_stages": None, "group_split": 0}


def _group_split_request() -> int:
    if _BWD_TILE.get("auto", True):
        return 0
    return int(_BWD_TILE.get("group_split", 0) or 0)


def _pick_backward_tile(args, block_mask=None) -> dict:
    """The backward launch shape: {"BLOCK_M", "BLOCK_N", "num_warps",
    "num_stages", "group_split"}.

    ``args`` is either the packed ``BwdArgsC`` of a launch (the shape the
    library will use for it, group split included) or, as in the reference
    (attnfuse/runtime/backward.py:35), the query length N_q: then the dense
    16-bit shape, whose block sizes do not depend on N_q on gfx950, and
    group_split 0 (chosen per launch).  num_stages is None: the pipeline
    depth is fixed by the instantiation."""
    if not isinstance(args, N.BwdArgsC):
        int(args)                       # the reference passes N_q
        return dict(_DEFAULT_TILE)
    import ctypes as C
    bm, bn, gs = C.c_int32(), C.c_int32(), C.c_int32()
    c_bm = block_mask._c() if block_mask is not None else None
    N.check(N.lib().af_bwd_tile(args, c_bm, C.byref(bm), C.byref(bn),
                                C.byref(gs)))
    return {"BLOCK_M": bm.value, "BLOCK_N": bn.value,
            "num_warps": bm.value // 32, "num_stages": None,
            "group_split": gs.value}


def _check_tile_request(args, block_mask=None) -> None:
    """Raise ValueError when _BWD_TILE (with "auto" off) asks for a reference
    key value this launch cannot honour."""
    if _BWD_TILE.get("auto", True):
        return
    want = {k: _BWD_TILE[k] for k in _REFERENCE_KEYS
            if _BWD_TILE.get(k) is not None}
    if not want:
        return
    have = _pick_backward_tile(args, block_mask)
    bad = sorted(k for k, v in want.items()
                 if k == "num_stages" or have.get(k) != v)
    if bad:
        raise ValueError(
            f"_BWD_TILE sets {', '.join(f'{k}={want[k]}' for k in bad)}, "
            f"which the gfx950 backward cannot use: its block shape is fixed "
            f"per instantiation (this launch: BLOCK_M={have['BLOCK_M']}, "
            f"BLOCK_N={have['BLOCK_N']}, num_warps={have['num_warps']}) and "
            f"its pipeline depth is not selectable; only 'group_split' can "
            f"be chosen")


def _bwd_workspace(device, nbytes: int) -> torch.Tensor:
    return torch.empty(max(nbytes, 16), dtype=torch.uint8, device=device)


def _run_backward_key(key, Q, K, V, O, L, dO, sm_scale, window, cos, sin,
                      block_mask, alibi_slopes):
    from .dispatch import _slopes_f32, check_qkv, kernel_layout, rope_tables
    check_qkv(Q, K, V)
    B, Hq, Nq, D = Q.shape
    Hkv, Nkv = K.shape[1], K.shape[2]
    if L.shape != (B, Hq, Nq) or L.dtype != torch.float32:
        raise ValueError("L must be the (B, H_q, N_q) float32 log-sum-exp")
    Qk, Kk, Vk = kernel_layout(Q), kernel_layout(K), kernel_layout(V)
    Ok, dOk = kernel_layout(O), kernel_layout(dO.to(Q.dtype))
    dQ = torch.empty_like(Qk)
    dK = torch.empty_like(Kk)
    dV = torch.empty_like(Vk)
    slopes = _slopes_f32(Hq, Q, alibi_slopes) if key[3] == 1 else None
    c = s = None
    if key[5]:
        c, s = rope_tables(cos, sin, Q)
    a = N.BwdArgsC()
    a.key = N.SpecKeyC(*key)
    a.q, a.k, a.v = Qk.data_ptr(), Kk.data_ptr(), Vk.data_ptr()
    a.o, a.dout, a.lse = Ok.data_ptr(), dOk.data_ptr(), L.data_ptr()
    a.dq, a.dk, a.dv = dQ.data_ptr(), dK.data_ptr(), dV.data_ptr()
    a.cos, a.sin = N.ptr(c), N.ptr(s)
    a.alibi_slopes = N.ptr(slopes)
    a.q_stride[:] = Qk.stride()
    a.k_stride[:] = Kk.stride()
    a.v_stride[:] = Vk.stride()
    a.o_stride[:] = Ok.stride()
    a.do_stride[:] = dOk.stride()
    a.dq_stride[:] = dQ.stride()
    a.dk_stride[:] = dK.stride()
    a.dv_stride[:] = dV.stride()
    a.lse_stride[:] = L.stride()
    a.rope_stride[:] = N.strides(c, 2)
    a.batch, a.heads_q, a.heads_kv = B, Hq, Hkv
    a.seqlen_q, a.seqlen_kv = Nq, Nkv
    a.rope_len = 0 if c is None else c.shape[0]
    a.scale = float(sm_scale)
    a.window = int(window or 0)
    a.group_split = _group_split_request()
    _check_tile_request(a, block_mask)
    bm = block_mask._c() if block_mask is not None else None
    nbytes = int(N.lib().af_bwd_workspace_bytes(a) if bm is None else
                 N.lib().af_bwd_blocksparse_workspace_bytes(a, bm))
    ws = _bwd_workspace(Q.device, nbytes)
    N.check(N.lib().af_bwd(a, bm, ws.data_ptr(), ws.numel(),
                           N.stream_handle(Q.device)))
    return dQ, dK, dV


def run_backward(graph: Graph, Q: torch.Tensor, K: torch.Tensor,
                 V: torch.Tensor, O: torch.Tensor, L: torch.Tensor,
                 dO: torch.Tensor, sm_scale: float, *, cos=None, sin=None,
                 block_mask=None, alibi_slopes=None) -> tuple:
    """Return (dQ, dK, dV) for a graph inside ``can_backward``'s scope."""
    from .kernel_cache import get_or_compile
    if not can_backward(graph):
        raise NotImplementedError("graph is outside the backward scope")
    bundle = get_or_compile(graph)
    key = bundle.key.abi_tuple()
    return _run_backward_key(key, Q, K, V, O, L, dO, sm_scale, bundle.window,
                             cos, sin, block_mask, alibi_slopes)
