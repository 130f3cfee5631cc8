"""CPU oracle for the fused-attention path.

TEST INFRASTRUCTURE ONLY.  Only tests/, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this module, and only as the
checker (or the timed CPU baseline) -- never as the thing measured or shipped.

A plain-torch restatement, always computed in float32 (or float64 when asked)
on upcast copies of the inputs, of:

* ``naive_attention`` -- reference attnfuse/reference/pytorch_naive.py:11-43
  (softmax(Q K^T * scale [+ ALiBi] [masks]) V), extended the way the
  reference's own tests extend it: GQA by repeating K/V heads
  (tests/test_gqa.py:34-40), an element mask (tests/test_block_sparse.py:35-48),
  an additive bias (tests/test_correctness.py:96-100), ReLU normalisation
  (attnfuse/compiler/codegen.py:230-233,368-371) and the decode ALiBi query
  position N_kv - 1 (attnfuse/compiler/codegen_decode.py:142-145).  Unlike
  the reference oracle, the ALiBi distance is never rounded to a 16-bit
  dtype (pytorch_naive.py:29 does that).
* the log-sum-exp L = m + ln(l) the forward saves
  (attnfuse/compiler/codegen.py:378-381);
* RoPE tables and rotation -- attnfuse/rope_utils.py:33-73;
* ALiBi slopes -- attnfuse/runtime/dispatch.py:24-40;
* the block-mask tile grid and its CSR / K-major lists --
  attnfuse/runtime/block_mask.py:100-202 (per-tile loop, as the reference);
* the split-K log-sum-exp combine -- attnfuse/compiler/codegen_decode.py:172-211;
* gradients -- autograd of the fp32/fp64 restatement (the reference's
  tests differentiate the naive oracle, tests/test_backward.py:42-58,143-158).

Every function is pinned by tests/test_oracle.py against closed forms, a
library routine (torch SDPA in float64), brute-force loops on tiny inputs,
the reference tests' known answers, and committed golden fixtures.
"""
from __future__ import annotations

import math
from typing import Optional

import torch


# ---------------------------------------------------------------------------
# RoPE (reference: attnfuse/rope_utils.py:33-73)
# ---------------------------------------------------------------------------
def rope_tables(seqlen: int, head_dim: int, base: float = 10000.0,
                dtype=torch.float32):
    """(cos, sin) of shape (seqlen, head_dim): angle t * base^(-2i/D) for
    i < D/2, repeated for the second half; fp32 math, then cast."""
    half = head_dim // 2
    i = torch.arange(half, dtype=torch.float32)
    theta = 1.0 / (base ** (2.0 * i / head_dim))
    t = torch.arange(seqlen, dtype=torch.float32)
    ang = torch.outer(t, theta)
    ang = torch.cat([ang, ang], dim=1)
    return ang.cos().to(dtype), ang.sin().to(dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat([-x[..., h:], x[..., :h]], dim=-1)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
               positions: Optional[torch.Tensor] = None) -> torch.Tensor:
    """x (.., N, D) rotated at positions 0..N-1 (or ``positions``)."""
    n = x.shape[-2]
    pos = torch.arange(n) if positions is None else positions
    c = cos.reshape(-1, cos.shape[-1])[pos].to(x.dtype)
    s = sin.reshape(-1, sin.shape[-1])[pos].to(x.dtype)
    return x * c + rotate_half(x) * s


# ---------------------------------------------------------------------------
# ALiBi slopes (reference: attnfuse/runtime/dispatch.py:24-40)
# ---------------------------------------------------------------------------
def alibi_slopes(n_heads: int) -> list:
    def pow2(n):
        first = 2.0 ** (-(2.0 ** -(math.log2(n) - 3)))
        return [first ** (k + 1) for k in range(n)]
    if n_heads & (n_heads - 1) == 0:
        return pow2(n_heads)
    lo = 2 ** int(math.floor(math.log2(n_heads)))
    return pow2(lo) + pow2(2 * lo)[0::2][: n_heads - lo]


# ---------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------
def expand_kv(t: torch.Tensor, group: int) -> torch.Tensor:
    """(B, H_kv, N, D) -> (B, H_kv * group, N, D), head h reading h // group."""
    return t.repeat_interleave(group, dim=1)


def score_bias_and_mask(Nq: int, Nkv: int, *, causal=False, window=None,
                        alibi=None, elem_mask=None, bias=None,
                        query_offset: int = 0, dtype=torch.float32):
    """Additive term (H or 1, Nq, Nkv) and boolean keep-mask (Nq, Nkv).

    Query i sits at position i + query_offset (0 for self-attention,
    N_kv - 1 for a single decode query)."""
    qi = torch.arange(Nq, dtype=torch.int64)[:, None] + query_offset
    kj = torch.arange(Nkv, dtype=torch.int64)[None, :]
    add = torch.zeros(1, Nq, Nkv, dtype=dtype)
    if alibi is not None:
        slopes = torch.as_tensor(alibi, dtype=dtype).reshape(-1, 1, 1)
        add = add - slopes * (qi - kj).abs().to(dtype)[None]
    keep = torch.ones(Nq, Nkv, dtype=torch.bool)
    if causal:
        keep &= kj <= qi
    if window is not None:
        keep &= (qi - kj).abs() < window
    if elem_mask is not None:
        keep &= elem_mask.to(torch.bool)
    return add, keep


def naive_attention(Q, K, V, *, causal: bool = False, window=None,
                    alibi_slopes=None, scale: Optional[float] = None,
                    elem_mask=None, bias=None, norm: str = "softmax",
                    rope=None, query_offset: int = 0,
                    dtype=torch.float32, return_lse: bool = False,
                    rope_round=None):
    """Reference attention on upcast CPU copies.

    Q (B, Hq, Nq, D); K, V (B, Hkv, Nkv, D) with Hq % Hkv == 0.
    ``rope`` = (cos, sin) tables, applied to Q and K at positions 0..N-1.
    ``rope_round`` -- optional 16-bit dtype the rotated q~, k~ are rounded to
    before the dot product, as the reference kernel does
    (attnfuse/compiler/codegen.py:126-135,195-204).
    Returns O (B, Hq, Nq, D) in ``dtype`` (and L (B, Hq, Nq) if asked)."""
    Q = Q.detach().to("cpu", dtype) if not Q.requires_grad else Q.to(dtype)
    K = K.detach().to("cpu", dtype) if not K.requires_grad else K.to(dtype)
    V = V.detach().to("cpu", dtype) if not V.requires_grad else V.to(dtype)
    B, Hq, Nq, D = Q.shape
    G = Hq // K.shape[1]
    if rope is not None:
        cos, sin = (t.to("cpu", dtype) for t in rope)
        Q = apply_rope(Q, cos, sin, torch.arange(Nq) + query_offset)
        K = apply_rope(K, cos, sin)
        if rope_round is not None:
            Q = Q.to(rope_round).to(dtype)
            K = K.to(rope_round).to(dtype)
    K, V = expand_kv(K, G), expand_kv(V, G)
    Nkv = K.shape[2]
    sc = 1.0 / math.sqrt(D) if scale is None else scale
    S = torch.matmul(Q, K.transpose(-2, -1)) * sc
    add, keep = score_bias_and_mask(
        Nq, Nkv, causal=causal, window=window,
        alibi=None if alibi_slopes is None else
        torch.as_tensor(alibi_slopes, dtype=dtype).cpu(),
        elem_mask=None if elem_mask is None else elem_mask.cpu(),
        query_offset=query_offset, dtype=dtype)
    S = S + add[None]
    if bias is not None:
        S = S + bias.to("cpu", dtype)
    S = S.masked_fill(~keep, float("-inf"))
    if norm == "softmax":
        m = S.amax(dim=-1, keepdim=True)
        m_safe = torch.where(torch.isinf(m), torch.zeros_like(m), m)
        P = torch.exp(S - m_safe)
        l = P.sum(dim=-1, keepdim=True)
        l_safe = torch.where(l == 0, torch.ones_like(l), l)
        O = torch.matmul(P / l_safe, V)
        L = (m + torch.log(l_safe)).squeeze(-1)
    elif norm == "relu":
        P = torch.clamp(S, min=0.0)
        l = P.sum(dim=-1, keepdim=True)
        l_safe = torch.where(l == 0, torch.ones_like(l), l)
        O = torch.matmul(P, V) / l_safe
        L = torch.full(O.shape[:-1], float("-inf"), dtype=dtype)
    else:
        raise ValueError(norm)
    return (O, L) if return_lse else O


def attention_grads(Q, K, V, dO, dtype=torch.float64, **kw):
    """(O, dQ, dK, dV) by autograd through ``naive_attention`` (RoPE and the
    GQA head expansion included, so dK/dV come out group-summed)."""
    q = Q.detach().to("cpu", dtype).requires_grad_(True)
    k = K.detach().to("cpu", dtype).requires_grad_(True)
    v = V.detach().to("cpu", dtype).requires_grad_(True)
    O = naive_attention(q, k, v, dtype=dtype, **kw)
    O.backward(dO.detach().to("cpu", dtype))
    return O.detach(), q.grad, k.grad, v.grad


# ---------------------------------------------------------------------------
# Split-K decode combine (reference: attnfuse/compiler/codegen_decode.py)
# ---------------------------------------------------------------------------
def decode_split_combine(Q, K, V, num_splits: int, *, alibi_slopes=None,
                         scale=None, dtype=torch.float64):
    """Single-query attention computed as per-split partial (m, l, acc) and
    merged by m* = max m_s, l* = sum e^(m_s-m*) l_s,
    O = sum e^(m_s-m*) acc_s / l*.  Splits are contiguous and exact."""
    Q, K, V = (t.detach().to("cpu", dtype) for t in (Q, K, V))
    B, Hq, _, D = Q.shape
    G = Hq // K.shape[1]
    K, V = expand_kv(K, G), expand_kv(V, G)
    Nkv = K.shape[2]
    sc = 1.0 / math.sqrt(D) if scale is None else scale
    S = torch.matmul(Q, K.transpose(-2, -1)) * sc          # (B,Hq,1,Nkv)
    if alibi_slopes is not None:
        sl = torch.as_tensor(alibi_slopes, dtype=dtype).reshape(1, -1, 1, 1)
        dist = ((Nkv - 1) - torch.arange(Nkv)).abs().to(dtype)
        S = S - sl * dist
    bounds = torch.linspace(0, Nkv, num_splits + 1).round().long().tolist()
    ms, ls, accs = [], [], []
    for lo, hi in zip(bounds[:-1], bounds[1:]):
        if hi <= lo:
            continue
        s = S[..., lo:hi]
        m = s.amax(dim=-1, keepdim=True)
        p = torch.exp(s - m)
        ms.append(m)
        ls.append(p.sum(dim=-1, keepdim=True))
        accs.append(torch.matmul(p, V[:, :, lo:hi]))
    m_all = torch.stack(ms)
    mstar = m_all.amax(dim=0)
    f = torch.exp(m_all - mstar)
    lstar = (f * torch.stack(ls)).sum(dim=0)
    return (f * torch.stack(accs)).sum(dim=0) / lstar


# ---------------------------------------------------------------------------
# Block masks (reference: attnfuse/runtime/block_mask.py:100-202)
# ---------------------------------------------------------------------------
def block_grid(pred, q_len: int, kv_len: int, bm: int, bn: int) -> torch.Tensor:
    """(n_q_blocks, n_kv_blocks) bool: a tile is active when any element of
    it satisfies ``pred`` (partial tiles round up to active)."""
    nqb, nkb = -(-q_len // bm), -(-kv_len // bn)
    qi = torch.arange(q_len)[:, None].expand(q_len, kv_len)
    kj = torch.arange(kv_len)[None, :].expand(q_len, kv_len)
    elem = torch.as_tensor(pred(qi, kj), dtype=torch.bool).expand(q_len, kv_len)
    grid = torch.zeros(nqb, nkb, dtype=torch.bool)
    for a in range(nqb):
        for b in range(nkb):
            tile = elem[a * bm:(a + 1) * bm, b * bn:(b + 1) * bn]
            grid[a, b] = bool(tile.any())
    return grid


def block_classes(pred, q_len: int, kv_len: int, bm: int, bn: int):
    """(full, partial) bool tile grids of an element predicate, by the
    per-tile loop of the reference's create_block_mask
    (attnfuse/runtime/block_mask.py:129-151) over tiles clipped to the
    sequence ends: full when every element of the tile is visible, partial
    when some but not all are (the reference then rounds partial up to full;
    an exact mask keeps them apart)."""
    nqb, nkb = -(-q_len // bm), -(-kv_len // bn)
    qi = torch.arange(q_len)[:, None].expand(q_len, kv_len)
    kj = torch.arange(kv_len)[None, :].expand(q_len, kv_len)
    elem = torch.as_tensor(pred(qi, kj), dtype=torch.bool).expand(q_len, kv_len)
    full = torch.zeros(nqb, nkb, dtype=torch.bool)
    part = torch.zeros(nqb, nkb, dtype=torch.bool)
    for a in range(nqb):
        for b in range(nkb):
            tile = elem[a * bm:(a + 1) * bm, b * bn:(b + 1) * bn]
            n = int(tile.sum())
            full[a, b] = n == tile.numel()
            part[a, b] = 0 < n < tile.numel()
    return full, part


def block_lists(grid: torch.Tensor):
    """Q-major rows and K-major columns of a tile grid as Python lists."""
    rows = [[b for b in range(grid.shape[1]) if grid[a, b]]
            for a in range(grid.shape[0])]
    cols = [[a for a in range(grid.shape[0]) if grid[a, b]]
            for b in range(grid.shape[1])]
    return rows, cols


def element_mask_from_grid(grid: torch.Tensor, q_len: int, kv_len: int,
                           bm: int, bn: int) -> torch.Tensor:
    """Element-level keep mask implied by visiting whole active tiles."""
    e = grid.repeat_interleave(bm, dim=0).repeat_interleave(bn, dim=1)
    return e[:q_len, :kv_len]


def bigbird_grid(n_blocks: int, n_random: int, seed: int) -> torch.Tensor:
    """Config-4 BigBird tile grid: block row 0, block column 0, the band
    |qb - kb| <= 1, plus ``n_random`` key blocks per row drawn in row order
    with ``torch.randperm(n_blocks, generator=g)[:n_random]``,
    g = torch.Generator().manual_seed(seed)."""
    g = torch.Generator().manual_seed(seed)
    grid = torch.zeros(n_blocks, n_blocks, dtype=torch.bool)
    grid[0, :] = True
    grid[:, 0] = True
    for a in range(n_blocks):
        for b in range(max(0, a - 1), min(n_blocks, a + 2)):
            grid[a, b] = True
        grid[a, torch.randperm(n_blocks, generator=g)[:n_random]] = True
    return grid


# ---------------------------------------------------------------------------
# Causal tile coverage (which (32-row, 64-key) tiles a kernel must visit)
# ---------------------------------------------------------------------------
def expected_coverage(Nq: int, Nkv: int, *, mask: str, window=None,
                      grid=None, bm=None, bn=None) -> torch.Tensor:
    """(ceil(Nq/32), ceil(Nkv/64)) int: 1 where the 32-query x 64-key tile
    holds at least one visible pair, for full / causal / sliding-window
    masks; for block-sparse, 1 for every 64-key stage of every listed tile."""
    nq, nk = -(-Nq // 32), -(-Nkv // 64)
    cov = torch.zeros(nq, nk, dtype=torch.int32)
    for a in range(nq):
        q_lo, q_hi = 32 * a, min(32 * a + 32, Nq) - 1
        for b in range(nk):
            k_lo, k_hi = 64 * b, min(64 * b + 64, Nkv) - 1
            if mask == "full":
                vis = True
            elif mask == "causal":
                vis = k_lo <= q_hi
            elif mask == "sliding_window":
                vis = (k_lo <= q_hi + window - 1) and (k_hi >= q_lo - window + 1)
            elif mask == "causal_sliding_window":
                vis = (k_lo <= q_hi) and (k_hi >= q_lo - window + 1)
            elif mask == "block_sparse":
                vis = bool(grid[(32 * a) // bm, (64 * b) // bn])
            else:
                raise ValueError(mask)
            cov[a, b] = int(vis)
    return cov
