"""Prepared launches: validate and marshal a call once, then enqueue it any
number of times with only a ctypes call of host work (and the call's
workspace allocated once).

For fixed-shape loops (serving decode steps, benchmarks) the per-call
Python dispatch of ``run_attention`` -- graph lookup, validation, layout
checks, argument packing -- costs tens of microseconds, comparable to a
decode kernel.  A prepared launcher keeps the packed C argument struct and
references to every tensor it points into, so each call is one
``af_fwd``/``af_decode`` on the stream current at call time.
"""
from __future__ import annotations

from typing import Callable, Optional

import torch

from ..ir.high_level import Graph
from . import _native as N


class PreparedLaunch:
    def __init__(self, fn, args, keep, device, extra=()):
        self._fn = fn
        self._args = args
        self._keep = keep          # tensors the struct points into
        self._device = device
        self._extra = extra

    def __call__(self) -> None:
        N.check(self._fn(self._args, *self._extra,
                         N.stream_handle(self._device)))


def prepare_attention(graph: Graph, Q, K, V, *, bias=None, cos=None, sin=None,
                      out: Optional[torch.Tensor] = None,
                      save_lse: Optional[torch.Tensor] = None,
                      alibi_slopes=None) -> tuple:
    """-> (launch, out): ``launch()`` recomputes ``out`` from the current
    contents of Q/K/V (same shapes and storage)."""
    from .dispatch import (_nbytes, _rows_ok, _slopes_f32, check_qkv,
                           fill_fwd_args, fwd_workspace, kernel_layout,
                           rope_tables)
    from .kernel_cache import get_or_compile
    check_qkv(Q, K, V)
    for t in (Q, K, V):
        if not _rows_ok(t):
            raise ValueError("prepared launches need kernel-ready layouts "
                             "(unit head-dim stride, 16-byte rows)")
    bundle = get_or_compile(graph)
    B, H, Nq, _ = Q.shape
    Nkv = K.shape[2]
    if out is None:
        out = torch.empty_like(Q)
    slopes = _slopes_f32(H, Q, alibi_slopes) if bundle.bias_kind == 1 else None
    b = None
    if bundle.has_additive_bias:
        if bias is None:
            raise RuntimeError("graph needs bias=")
        b = kernel_layout(bias.to(Q.dtype).expand(B, H, Nq, Nkv))
    c = s = None
    if bundle.has_rope:
        c, s = rope_tables(cos, sin, Q)
    args = N.FwdArgsC()
    fill_fwd_args(args, bundle.key.abi_tuple(), Q, K, V, out, save_lse, c, s,
                  slopes, b, None, bundle.sm_scale, bundle.window)
    ws = fwd_workspace(args, Q.device)
    keep = (Q, K, V, out, save_lse, c, s, slopes, b, ws)
    return PreparedLaunch(N.lib().af_fwd, args, keep, Q.device,
                          extra=(N.ptr(ws), _nbytes(ws))), out


def prepare_decode(graph: Graph, Q, K, V, *, out=None, num_splits: int = 0,
                   alibi_slopes=None) -> tuple:
    """-> (launch, out) for a flash-decoding call with its own workspace."""
    from .dispatch import _rows_ok, _slopes_f32, check_qkv
    from .flash_decode import _pick_num_splits, can_use_flash_decode
    from .kernel_cache import get_or_compile
    check_qkv(Q, K, V)
    if not can_use_flash_decode(graph, Q, K):
        raise ValueError("graph/shape is not a flash-decoding call")
    for t in (Q, K, V):
        if not _rows_ok(t):
            raise ValueError("prepared launches need kernel-ready layouts")
    bundle = get_or_compile(graph)
    B, Hq, _, D = Q.shape
    Hkv, Nkv = K.shape[1], K.shape[2]
    if out is None:
        out = torch.empty_like(Q)
    S = num_splits or _pick_num_splits(B, Hq, Nkv, Hkv, D)
    nbytes = int(N.lib().af_decode_workspace_bytes(B, Hq, D, S))
    ws = torch.empty(nbytes, dtype=torch.uint8, device=Q.device)
    slopes = _slopes_f32(Hq, Q, alibi_slopes) if bundle.bias_kind == 1 else None
    a = N.DecodeArgsC()
    a.key = N.SpecKeyC({torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}[Q.dtype], D, 0,
                       bundle.bias_kind, 0, 0)
    a.q, a.k, a.v, a.o = Q.data_ptr(), K.data_ptr(), V.data_ptr(), out.data_ptr()
    a.alibi_slopes = N.ptr(slopes)
    a.q_stride[:] = Q.stride()
    a.k_stride[:] = K.stride()
    a.v_stride[:] = V.stride()
    a.o_stride[:] = out.stride()
    a.batch, a.heads_q, a.heads_kv, a.seqlen_kv = B, Hq, Hkv, Nkv
    a.scale = bundle.sm_scale
    a.num_splits = S
    keep = (Q, K, V, out, ws, slopes)
    return PreparedLaunch(N.lib().af_decode, a, keep, Q.device,
                          extra=(ws.data_ptr(), nbytes)), out
