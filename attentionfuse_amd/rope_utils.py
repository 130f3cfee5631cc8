"""Rotary position embedding tables and the host-side rotation.

Same convention as the reference (reference: attnfuse/rope_utils.py:33-73):
theta_i = base^(-2i/D) for i < D/2, angles t*theta_i duplicated over both
halves of the head dimension (rotate-half pairing d <-> d + D/2), tables
computed in fp32 and then cast.  The fused kernels consume these tables;
``apply_rope`` is the eager rotation for pre-rotating inputs.
"""
from __future__ import annotations

import torch


def build_rope_cache(seqlen: int, head_dim: int, base: float = 10_000.0,
                     device="cuda", dtype: torch.dtype = torch.float16):
    """(cos, sin), each (1, 1, seqlen, head_dim)."""
    if head_dim % 2:
        raise ValueError("RoPE needs an even head_dim")
    half = head_dim // 2
    exps = torch.arange(half, device=device, dtype=torch.float32) * 2 / head_dim
    inv = 1.0 / (base ** exps)
    ang = torch.outer(torch.arange(seqlen, device=device, dtype=torch.float32), inv)
    ang = torch.cat([ang, ang], dim=-1)
    return (ang.cos().to(dtype)[None, None], ang.sin().to(dtype)[None, None])


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    lo, hi = x.chunk(2, dim=-1)
    return torch.cat([-hi, lo], dim=-1)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    """x * cos + rotate_half(x) * sin; cos/sin (N, D) or (1, 1, N, D)."""
    return x * cos + _rotate_half(x) * sin
