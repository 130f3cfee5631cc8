"""Forward dispatch: Graph + tensors -> one ``af_fwd`` call.

Mirrors the reference ``run_attention`` (reference:
attnfuse/runtime/dispatch.py:69-215): same signature, validation and
exception types, the flash-decoding route for single-query calls, the
cross-attention guard, the ALiBi slope recipe, and (1,1,N,D) -> (N,D) RoPE
tables.  The launch itself goes through the C ABI of libattnfuse_hip.so on
torch's current HIP stream.
"""
from __future__ import annotations

import functools
import math
from typing import Optional

import torch

from ..ir.high_level import Graph, MaskKind
from . import _native as N
from .kernel_cache import get_or_compile

_TORCH_DTYPES = {"float16": torch.float16, "bfloat16": torch.bfloat16,
                 "float32": torch.float32}


# ---------------------------------------------------------------------------
# ALiBi slopes (Press et al., 2021)
# ---------------------------------------------------------------------------
def _geometric_slopes(n: int) -> list:
    """Slopes for a power-of-two head count: r, r^2, ..., r^n, r = 2^(-8/n)."""
    r = 2.0 ** (-8.0 / n)
    return [r ** (i + 1) for i in range(n)]


def alibi_slope_values(n_heads: int) -> list:
    """Per-head ALiBi slopes as Python floats.

    Power-of-two H: the geometric sequence above.  Otherwise the sequence of
    the largest power of two below H, followed by every other slope of the
    sequence for twice that count (reference recipe,
    attnfuse/runtime/dispatch.py:24-40)."""
    if n_heads <= 0:
        raise ValueError("n_heads must be positive")
    if n_heads & (n_heads - 1) == 0:
        return _geometric_slopes(n_heads)
    p2 = 1 << (n_heads.bit_length() - 1)
    extra = _geometric_slopes(2 * p2)[0::2][: n_heads - p2]
    return _geometric_slopes(p2) + extra


@functools.lru_cache(maxsize=64)
def _alibi_slopes(n_heads: int, device_str: str, dtype_str: str) -> torch.Tensor:
    """Slopes as a 1-D tensor in the given dtype (the reference keeps them in
    Q's dtype, so the kernels see the rounded values)."""
    dtype = _TORCH_DTYPES[dtype_str.replace("torch.", "")]
    return torch.tensor(alibi_slope_values(n_heads), dtype=dtype,
                        device=device_str)


def _slopes_f32(H: int, Q: torch.Tensor, override) -> torch.Tensor:
    if override is not None:
        s = torch.as_tensor(override, device=Q.device)
        if s.numel() != H:
            raise ValueError(f"alibi_slopes has {s.numel()} values, need {H}")
        return s.reshape(H).to(torch.float32).contiguous()
    return _alibi_slopes(H, str(Q.device), str(Q.dtype)).to(torch.float32)


# ---------------------------------------------------------------------------
# Layout helpers: the kernels use 16-byte vector loads, so rows must be
# 16-byte aligned with a unit innermost stride.
# ---------------------------------------------------------------------------
def _rows_ok(t: torch.Tensor) -> bool:
    if t.stride(-1) != 1 or t.data_ptr() % 16:
        return False
    return all(s % 8 == 0 for s in t.stride()[:-1])


def kernel_layout(t: torch.Tensor) -> torch.Tensor:
    """Return ``t`` or a copy whose rows the kernels can vector-load."""
    if _rows_ok(t):
        return t
    c = t.contiguous()
    if _rows_ok(c):
        return c
    n = t.shape[-1]
    pad = (n + 7) // 8 * 8
    buf = torch.empty(*t.shape[:-1], pad, dtype=t.dtype, device=t.device)
    view = buf[..., :n]
    view.copy_(t)
    return view


def rope_tables(cos, sin, Q: torch.Tensor):
    if cos is None or sin is None:
        raise RuntimeError(
            "this attention graph was built with af.rope(); pass cos=<table> "
            "and sin=<table> at call time")
    c = cos.reshape(cos.shape[-2], cos.shape[-1]) if cos.dim() != 2 else cos
    s = sin.reshape(sin.shape[-2], sin.shape[-1]) if sin.dim() != 2 else sin
    if c.shape != s.shape or c.shape[-1] != Q.shape[-1]:
        raise ValueError(f"cos/sin tables must be (N, {Q.shape[-1]}); got "
                         f"{tuple(cos.shape)} and {tuple(sin.shape)}")
    if c.device != Q.device or s.device != Q.device:
        raise ValueError("cos/sin must live on Q's device")
    c = kernel_layout(c.to(Q.dtype))
    s = kernel_layout(s.to(Q.dtype))
    return c, s


def check_qkv(Q, K, V) -> None:
    if not (Q.is_cuda and K.is_cuda and V.is_cuda):
        raise RuntimeError("AttnFuse requires Q/K/V on a GPU (HIP) device")
    if Q.dim() != 4 or K.dim() != 4 or V.dim() != 4:
        raise ValueError("Q, K, V must be 4-D (B, H, N, D)")
    if K.shape != V.shape:
        raise ValueError(f"K and V must have the same shape; got "
                         f"{tuple(K.shape)}, {tuple(V.shape)}")
    if Q.shape[0] != K.shape[0] or Q.shape[3] != K.shape[3]:
        raise ValueError(f"Q and K/V must agree on (batch, head_dim); got "
                         f"Q={tuple(Q.shape)}, K={tuple(K.shape)}")
    if Q.shape[1] % K.shape[1] != 0:
        raise ValueError(f"Q heads ({Q.shape[1]}) must be a multiple of KV "
                         f"heads ({K.shape[1]}) for GQA")
    if not (Q.dtype == K.dtype == V.dtype):
        raise ValueError("Q, K, V must share one dtype")


def fill_fwd_args(a: "N.FwdArgsC", key_tuple, Q, K, V, out, lse, c, s, slopes,
                  bias, coverage, scale: float, window: int) -> None:
    a.key = N.SpecKeyC(*key_tuple)
    a.q, a.k, a.v, a.o = Q.data_ptr(), K.data_ptr(), V.data_ptr(), out.data_ptr()
    a.lse = N.ptr(lse)
    a.cos, a.sin = N.ptr(c), N.ptr(s)
    a.alibi_slopes = N.ptr(slopes)
    a.bias = N.ptr(bias)
    a.coverage = N.ptr(coverage)
    a.q_stride[:] = Q.stride()
    a.k_stride[:] = K.stride()
    a.v_stride[:] = V.stride()
    a.o_stride[:] = out.stride()
    a.lse_stride[:] = N.strides(lse, 3)
    a.rope_stride[:] = N.strides(c, 2)
    a.bias_stride[:] = N.strides(bias, 4)
    a.batch, a.heads_q, a.seqlen_q = Q.shape[0], Q.shape[1], Q.shape[2]
    a.heads_kv, a.seqlen_kv = K.shape[1], K.shape[2]
    a.rope_len = 0 if c is None else c.shape[0]
    a.scale = float(scale)
    a.window = int(window or 0)


def fwd_workspace(args: "N.FwdArgsC", device) -> Optional[torch.Tensor]:
    """Workspace the forward needs for these arguments (the rotated keys when
    RoPE is fused), or None.  Allocated on the caller's stream through torch's
    caching allocator, so releasing it after the launch is stream-ordered."""
    n = int(N.lib().af_fwd_workspace_bytes(args))
    return torch.empty(n, dtype=torch.uint8, device=device) if n else None


def _nbytes(ws: Optional[torch.Tensor]) -> int:
    return 0 if ws is None else ws.numel()


def run_attention(
    graph: Graph,
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    cos: Optional[torch.Tensor] = None,
    sin: Optional[torch.Tensor] = None,
    out: Optional[torch.Tensor] = None,
    save_lse: Optional[torch.Tensor] = None,
    *,
    alibi_slopes=None,
    coverage: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Run the fused forward and return O (B, H_q, N_q, D).

    ``save_lse`` -- a (B, H_q, N_q) fp32 buffer that receives L = m + ln(l).
    ``alibi_slopes`` -- optional explicit per-head slopes overriding the
    default recipe.  ``coverage`` -- optional uint32/int32 tile-visit counter
    buffer (B, H_q, ceil(N_q/32), ceil(N_kv/64)) for mask-coverage tests.
    """
    check_qkv(Q, K, V)
    bundle = get_or_compile(graph)
    B, H, Nq, D = Q.shape
    Nkv = K.shape[2]

    from .flash_decode import can_use_flash_decode, run_flash_decode
    if save_lse is None and coverage is None and can_use_flash_decode(graph, Q, K):
        if out is None:
            out = torch.empty_like(Q)
        return run_flash_decode(graph, Q, K, V, bundle.sm_scale,
                                bundle.bias_kind, K.shape[1], out,
                                alibi_slopes=alibi_slopes)

    if Nq != Nkv:
        masks = {m.kind for m in graph.collect_masks()}
        if masks - {MaskKind.FULL}:
            raise ValueError(
                f"cross-attention (N_q={Nq} != N_kv={Nkv}) supports only "
                f"dense masks; the graph uses {sorted(m.value for m in masks)}."
                " Use af.softmax(af.scaled_dot_product(Q, K)) @ V for "
                "KV-cache decoding.")

    if out is None:
        out = torch.empty_like(Q)
    if out.shape != Q.shape or out.dtype != Q.dtype:
        raise ValueError("out must match Q in shape and dtype")

    slopes = _slopes_f32(H, Q, alibi_slopes) if bundle.bias_kind == 1 else None
    b = None
    if bundle.has_additive_bias:
        if bias is None:
            raise RuntimeError(
                "this attention graph was built with af.additive_bias(); pass "
                "bias=<tensor of shape (B,H,N_q,N_kv)> at call time")
        b = kernel_layout(bias.to(Q.dtype).expand(B, H, Nq, Nkv))
    c = s = None
    if bundle.has_rope:
        c, s = rope_tables(cos, sin, Q)
    if save_lse is not None:
        if save_lse.shape != (B, H, Nq) or save_lse.dtype != torch.float32:
            raise ValueError("save_lse must be a (B, H_q, N_q) float32 tensor")

    Qk, Kk, Vk = kernel_layout(Q), kernel_layout(K), kernel_layout(V)
    o = out if _rows_ok(out) else torch.empty_like(Q)
    args = N.FwdArgsC()
    fill_fwd_args(args, bundle.key.abi_tuple(), Qk, Kk, Vk, o, save_lse, c, s,
                  slopes, b, coverage, bundle.sm_scale, bundle.window)
    ws = fwd_workspace(args, Q.device)
    N.check(N.lib().af_fwd(args, N.ptr(ws), _nbytes(ws),
                           N.stream_handle(Q.device)))
    if o is not out:
        out.copy_(o)
    return out
