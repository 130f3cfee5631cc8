"""Block-sparse masks: the ``BlockMask`` CSR format, its construction, and
the block-sparse forward/backward launches.

``BlockMask`` keeps the reference's fields and semantics (reference:
attnfuse/runtime/block_mask.py:74-202): Q-major lists of active key blocks
(``full_kv_*``; the ``kv_*`` partial lists stay empty because a tile with any
active element is rounded up to fully active), a K-major transpose
(``q_*``) for the dK/dV backward, zero-padded int32 rows of width
``max(1, longest row)``, indices ascending.

``create_block_mask`` evaluates the predicate on the (Q_LEN, KV_LEN) index
grid exactly like the reference, but reduces it to the block grid with one
reshape + ``any`` instead of a Python loop over tiles.  With ``exact=True``
(beyond the reference, which lists it as future work, PROGRESS.md:284-288)
tiles whose elements are only partly visible go to the partial lists
(``kv_*``) with their element masks as bit words (``part_row_bits`` for the
Q-major walks, ``q_col_bits`` + ``q_partial`` for the K-major one), and the
kernels apply those bits inside the tile: the result is attention under the
element predicate itself instead of its block-rounded upper bound.

Beyond the reference fields a mask carries a work plan (``BlockMaskPlan``,
from ``af_blockmask_plan``): lists much longer than the mean -- BigBird's
global query block visits every key block, and every query block visits the
global key block -- are cut into pieces that run as workgroups of their own
and whose fp32 partials a combine kernel merges, so that one long list no
longer holds up the end of the grid.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from typing import Callable, Optional

import torch

from . import _native as N


@dataclass
class BlockMaskPlan:
    """Work plans of the Q-major lists (forward, dQ) and the K-major lists
    (dK/dV): items (list, first entry, entries, slot) and splits (list,
    first slot, slots), int32 on the mask's device."""
    q_items: torch.Tensor
    q_splits: torch.Tensor
    n_q_slots: int
    kv_items: torch.Tensor
    kv_splits: torch.Tensor
    n_kv_slots: int

    def to(self, device) -> "BlockMaskPlan":
        return BlockMaskPlan(self.q_items.to(device), self.q_splits.to(device),
                             self.n_q_slots, self.kv_items.to(device),
                             self.kv_splits.to(device), self.n_kv_slots)


def _plan_lists(counts: torch.Tensor, chunk: int = 0):
    """af_blockmask_plan over host int32 counts -> (items, splits, slots)."""
    counts = counts.to(torch.int32).cpu().contiguous()
    n = counts.numel()
    lib = N.lib()
    sizes = (C.c_int32 * 3)()
    cp = C.c_void_p(counts.data_ptr() if n else None)
    N.check(lib.af_blockmask_plan(cp, n, chunk, None, None, sizes))
    items = torch.empty(max(sizes[0], 1), 4, dtype=torch.int32)
    splits = torch.zeros(max(sizes[1], 1), 3, dtype=torch.int32)
    N.check(lib.af_blockmask_plan(cp, n, chunk, C.c_void_p(items.data_ptr()),
                                  C.c_void_p(splits.data_ptr()), sizes))
    return items[: sizes[0]], splits[: sizes[1]], int(sizes[2])


def make_plan(q_counts: torch.Tensor, kv_counts: torch.Tensor, device,
              chunk: int = 0) -> BlockMaskPlan:
    """Plans for lists of ``q_counts`` (Q-major) and ``kv_counts`` (K-major)
    entries; ``chunk`` <= 0 lets the library choose the piece length."""
    qi, qs, qn = _plan_lists(q_counts, chunk)
    ki, ks, kn = _plan_lists(kv_counts, chunk)
    return BlockMaskPlan(qi.to(device), qs.to(device), qn, ki.to(device),
                         ks.to(device), kn)


@dataclass
class BlockMask:
    kv_num_blocks: torch.Tensor   # (n_q_blocks,) int32, partial tiles
    kv_indices: torch.Tensor      # (n_q_blocks, max_partial) int32
    full_kv_num: torch.Tensor     # (n_q_blocks,) int32
    full_kv_idx: torch.Tensor     # (n_q_blocks, max_full) int32
    q_num_blocks: torch.Tensor    # (n_kv_blocks,) int32
    q_indices: torch.Tensor       # (n_kv_blocks, max_q) int32
    BLOCK_M: int
    BLOCK_N: int
    n_q_blocks: int
    n_kv_blocks: int
    n_active: int
    n_full: int
    # work plan of the split walks; made from the list lengths on first use
    # when the mask was not built by block_mask_from_blocks.  A list the plan
    # keeps whole is walked to its current device-side count, so lists may be
    # edited in place (e.g. between graph replays); a list the plan splits
    # into pieces is walked by those pieces, clamped to its current count:
    # after changing such a list's length, call plan_work() again.
    plan: Optional[BlockMaskPlan] = field(default=None, repr=False,
                                          compare=False)
    # element masks of the partial tiles (create_block_mask(exact=True)):
    # int64 bit words (n_q_blocks, max_partial, BLOCK_M, BLOCK_N / 64) over
    # keys, (n_kv_blocks, max_q, BLOCK_N, ceil(BLOCK_M / 64)) over queries,
    # and int32 (n_kv_blocks, max_q) flags of the partial K-major entries
    part_row_bits: Optional[torch.Tensor] = field(default=None, repr=False)
    q_col_bits: Optional[torch.Tensor] = field(default=None, repr=False)
    q_partial: Optional[torch.Tensor] = field(default=None, repr=False)

    def to(self, device) -> "BlockMask":
        f = {k: (v.to(device) if isinstance(v, (torch.Tensor, BlockMaskPlan))
                 else v)
             for k, v in self.__dict__.items()}
        return BlockMask(**f)

    def plan_work(self, chunk: int = 0) -> BlockMaskPlan:
        """(Re)make the work plan from the list lengths (a host copy of the
        counts: one synchronisation) with piece length ``chunk`` (<= 0: the
        library's choice)."""
        qc = (self.full_kv_num.cpu().to(torch.int64)
              + self.kv_num_blocks.cpu().to(torch.int64))
        self.plan = make_plan(qc, self.q_num_blocks.cpu(),
                              self.full_kv_num.device, chunk)
        return self.plan

    def dense_blocks(self) -> torch.Tensor:
        """(n_q_blocks, n_kv_blocks) bool grid of visited tiles."""
        grid = torch.zeros(self.n_q_blocks, self.n_kv_blocks, dtype=torch.bool)
        for num, idx in ((self.full_kv_num, self.full_kv_idx),
                         (self.kv_num_blocks, self.kv_indices)):
            num, idx = num.cpu(), idx.cpu()
            for r in range(self.n_q_blocks):
                grid[r, idx[r, : int(num[r])].long()] = True
        return grid

    def _c(self) -> "N.BlockMaskC":
        bm = N.BlockMaskC()
        bm.full_kv_num = self.full_kv_num.data_ptr()
        bm.full_kv_idx = self.full_kv_idx.data_ptr()
        bm.kv_num_blocks = self.kv_num_blocks.data_ptr()
        bm.kv_indices = self.kv_indices.data_ptr()
        bm.q_num_blocks = self.q_num_blocks.data_ptr()
        bm.q_indices = self.q_indices.data_ptr()
        bm.full_kv_stride = self.full_kv_idx.stride(0)
        bm.kv_stride = self.kv_indices.stride(0)
        bm.q_stride = self.q_indices.stride(0)
        bm.block_m, bm.block_n = self.BLOCK_M, self.BLOCK_N
        bm.n_q_blocks, bm.n_kv_blocks = self.n_q_blocks, self.n_kv_blocks
        pl = self.plan if self.plan is not None else self.plan_work()
        bm.q_items, bm.q_splits = pl.q_items.data_ptr(), pl.q_splits.data_ptr()
        bm.kv_items = pl.kv_items.data_ptr()
        bm.kv_splits = pl.kv_splits.data_ptr()
        bm.n_q_items, bm.n_q_splits = pl.q_items.shape[0], pl.q_splits.shape[0]
        bm.n_q_slots = pl.n_q_slots
        bm.n_kv_items = pl.kv_items.shape[0]
        bm.n_kv_splits = pl.kv_splits.shape[0]
        bm.n_kv_slots = pl.n_kv_slots
        if self.part_row_bits is not None:
            bm.part_row_bits = self.part_row_bits.data_ptr()
            bm.q_col_bits = self.q_col_bits.data_ptr()
            bm.q_partial = self.q_partial.data_ptr()
        return bm


def _csr_rows(active: torch.Tensor):
    """Padded ascending index rows of a bool grid: (counts, indices)."""
    counts = active.sum(dim=1).to(torch.int32)
    width = max(1, int(counts.max()) if counts.numel() else 1)
    # a stable sort of ~active puts the active columns first, ascending
    order = torch.sort((~active).to(torch.int8), dim=1, stable=True).indices
    idx = order[:, :width].to(torch.int32)
    keep = torch.arange(width)[None, :] < counts[:, None].long()
    idx = torch.where(keep, idx, torch.zeros_like(idx))
    return counts, idx.contiguous()


def block_mask_from_blocks(active: torch.Tensor, BLOCK_M: int, BLOCK_N: int,
                           device="cuda") -> BlockMask:
    """Build a BlockMask from a (n_q_blocks, n_kv_blocks) bool tile grid."""
    active = active.to(torch.bool).cpu()
    nqb, nkb = active.shape
    full_num, full_idx = _csr_rows(active)
    q_num, q_idx = _csr_rows(active.t().contiguous())
    empty_num = torch.zeros(nqb, dtype=torch.int32)
    empty_idx = torch.zeros(nqb, 1, dtype=torch.int32)
    n = int(full_num.sum())
    # the plan is made here from the host-side counts, so that launching
    # the mask never copies them back (and can run under graph capture)
    plan = (make_plan(full_num, q_num, device)
            if torch.device(device).type == "cuda" else None)
    return BlockMask(
        kv_num_blocks=empty_num.to(device), kv_indices=empty_idx.to(device),
        full_kv_num=full_num.to(device), full_kv_idx=full_idx.to(device),
        q_num_blocks=q_num.to(device), q_indices=q_idx.to(device),
        BLOCK_M=BLOCK_M, BLOCK_N=BLOCK_N, n_q_blocks=nqb, n_kv_blocks=nkb,
        n_active=n, n_full=n, plan=plan)


def _pack_bits(bits: torch.Tensor) -> torch.Tensor:
    """(..., 64 w) bool -> (..., w) int64 words, element k of a word in bit
    k (bit 63 comes out as the int64 sign bit)."""
    *lead, n = bits.shape
    b = bits.reshape(*lead, n // 64, 64).to(torch.int64)
    return (b << torch.arange(64, dtype=torch.int64)).sum(dim=-1)


def block_mask_from_elements(elem: torch.Tensor, BLOCK_M: int, BLOCK_N: int,
                             device="cuda") -> BlockMask:
    """BlockMask that applies the (Q_LEN, KV_LEN) bool element mask ``elem``
    exactly: tiles with every element visible go to the full lists, tiles
    with some to the partial lists with their bits, tiles with none nowhere.
    Elements past the sequence ends count as visible for the full/partial
    test (the kernels mask them by length)."""
    if BLOCK_N % 64:
        raise NotImplementedError("element masks need BLOCK_N a multiple "
                                  "of 64")
    elem = elem.to(torch.bool).cpu()
    Q_LEN, KV_LEN = elem.shape
    nqb = (Q_LEN + BLOCK_M - 1) // BLOCK_M
    nkb = (KV_LEN + BLOCK_N - 1) // BLOCK_N
    vis = torch.zeros(nqb * BLOCK_M, nkb * BLOCK_N, dtype=torch.bool)
    vis[:Q_LEN, :KV_LEN] = elem
    dont_care = torch.ones_like(vis)
    dont_care[:Q_LEN, :KV_LEN] = elem
    tiles = vis.view(nqb, BLOCK_M, nkb, BLOCK_N).permute(0, 2, 1, 3)
    anyv = tiles.any(dim=3).any(dim=2)
    allv = dont_care.view(nqb, BLOCK_M, nkb, BLOCK_N).all(dim=3).all(dim=1)
    full = anyv & allv
    part = anyv & ~allv
    full_num, full_idx = _csr_rows(full)
    part_num, part_idx = _csr_rows(part)
    q_num, q_idx = _csr_rows(anyv.t().contiguous())
    # Q-major row bits: partial tile (qb, kb) is entry rank(kb) of row qb
    wr = BLOCK_N // 64
    row_bits = torch.zeros(nqb, part_idx.shape[1], BLOCK_M, wr,
                           dtype=torch.int64)
    qb, kb = part.nonzero(as_tuple=True)
    if qb.numel():
        e = (part.cumsum(dim=1) - 1)[qb, kb]
        row_bits[qb, e] = _pack_bits(tiles[qb, kb])
    # K-major column bits and partial flags: entry rank(qb) of column kb
    wc = (BLOCK_M + 63) // 64
    col_bits = torch.zeros(nkb, q_idx.shape[1], BLOCK_N, wc, dtype=torch.int64)
    q_partial = torch.zeros(nkb, q_idx.shape[1], dtype=torch.int32)
    if qb.numel():
        j = (anyv.t().cumsum(dim=1) - 1)[kb, qb]
        cols = tiles[qb, kb].transpose(1, 2)            # (n, BLOCK_N, BLOCK_M)
        if BLOCK_M % 64:
            cols = torch.cat([cols, torch.zeros(*cols.shape[:2], 64 * wc - BLOCK_M,
                                                dtype=torch.bool)], dim=2)
        col_bits[kb, j] = _pack_bits(cols)
        q_partial[kb, j] = 1
    plan = (make_plan(full_num + part_num, q_num, device)
            if torch.device(device).type == "cuda" else None)
    n_full, n_part = int(full_num.sum()), int(part_num.sum())
    return BlockMask(
        kv_num_blocks=part_num.to(device), kv_indices=part_idx.to(device),
        full_kv_num=full_num.to(device), full_kv_idx=full_idx.to(device),
        q_num_blocks=q_num.to(device), q_indices=q_idx.to(device),
        BLOCK_M=BLOCK_M, BLOCK_N=BLOCK_N, n_q_blocks=nqb, n_kv_blocks=nkb,
        n_active=n_full + n_part, n_full=n_full, plan=plan,
        part_row_bits=row_bits.to(device), q_col_bits=col_bits.to(device),
        q_partial=q_partial.to(device))


def create_block_mask(mask_fn: Callable, Q_LEN: int, KV_LEN: int,
                      BLOCK_M: int = 64, BLOCK_N: int = 64,
                      device="cuda", exact: bool = False) -> BlockMask:
    """BlockMask from an element predicate ``mask_fn(q_idx, kv_idx) -> bool``
    evaluated on (Q_LEN, KV_LEN) index grids.  A tile with any True element
    is active; by default it is visited whole (the reference's rounding),
    with ``exact=True`` partly visible tiles carry their element bits and
    the kernels apply the predicate itself."""
    nqb = (Q_LEN + BLOCK_M - 1) // BLOCK_M
    nkb = (KV_LEN + BLOCK_N - 1) // BLOCK_N
    qi = torch.arange(Q_LEN)[:, None].expand(Q_LEN, KV_LEN)
    kj = torch.arange(KV_LEN)[None, :].expand(Q_LEN, KV_LEN)
    elem = torch.as_tensor(mask_fn(qi, kj), dtype=torch.bool)
    elem = elem.expand(Q_LEN, KV_LEN)
    if exact:
        return block_mask_from_elements(elem, BLOCK_M, BLOCK_N, device)
    padded = torch.zeros(nqb * BLOCK_M, nkb * BLOCK_N, dtype=torch.bool)
    padded[:Q_LEN, :KV_LEN] = elem
    active = padded.view(nqb, BLOCK_M, nkb, BLOCK_N).any(dim=3).any(dim=1)
    return block_mask_from_blocks(active, BLOCK_M, BLOCK_N, device)


def _check_mask(Q, K, bm: BlockMask) -> None:
    if not isinstance(bm, BlockMask):
        raise TypeError("block_mask must be an attnfuse.BlockMask")
    if bm.full_kv_idx.device != Q.device:
        raise ValueError("block_mask lives on another device than Q; call "
                         "block_mask.to(Q.device)")
    nqb = (Q.shape[2] + bm.BLOCK_M - 1) // bm.BLOCK_M
    nkb = (K.shape[2] + bm.BLOCK_N - 1) // bm.BLOCK_N
    if (nqb, nkb) != (bm.n_q_blocks, bm.n_kv_blocks):
        raise ValueError(f"block_mask grid {bm.n_q_blocks}x{bm.n_kv_blocks} "
                         f"does not fit N_q={Q.shape[2]}, N_kv={K.shape[2]}")


def _bs_key(Q, bias_kind: int, rope: bool):
    dt = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}.get(Q.dtype)
    if dt is None:
        raise NotImplementedError(f"block-sparse kernels take fp16, bf16 or "
                                  f"fp32, got {Q.dtype}")
    return (dt, Q.shape[-1], 3, int(bias_kind), 0, int(rope))


def run_block_sparse(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor,
                     block_mask: BlockMask, sm_scale: float,
                     bias_kind: int = 0, out: Optional[torch.Tensor] = None,
                     save_lse: Optional[torch.Tensor] = None, *,
                     cos=None, sin=None, alibi_slopes=None,
                     coverage: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Block-sparse forward (reference signature,
    attnfuse/runtime/block_mask.py:205-210).  ``bias_kind`` 1 = ALiBi.
    ``cos``/``sin`` apply fused RoPE."""
    from .dispatch import (_nbytes, _rows_ok, _slopes_f32, check_qkv,
                           fill_fwd_args, kernel_layout, rope_tables)
    check_qkv(Q, K, V)
    _check_mask(Q, K, block_mask)
    B, H, Nq, D = Q.shape
    rope = cos is not None or sin is not None
    key = _bs_key(Q, bias_kind, rope)
    if out is None:
        out = torch.empty_like(Q)
    slopes = _slopes_f32(H, Q, alibi_slopes) if bias_kind == 1 else None
    c = s = None
    if rope:
        c, s = rope_tables(cos, sin, Q)
    Qk, Kk, Vk = kernel_layout(Q), kernel_layout(K), kernel_layout(V)
    o = out if _rows_ok(out) else torch.empty_like(Q)
    a = N.FwdArgsC()
    fill_fwd_args(a, key, Qk, Kk, Vk, o, save_lse, c, s, slopes, None,
                  coverage, sm_scale, 0)
    bm = block_mask._c()
    nb = int(N.lib().af_fwd_blocksparse_workspace_bytes(a, bm))
    ws = torch.empty(nb, dtype=torch.uint8, device=Q.device) if nb else None
    N.check(N.lib().af_fwd_blocksparse(a, bm, N.ptr(ws), _nbytes(ws),
                                       N.stream_handle(Q.device)))
    if o is not out:
        out.copy_(o)
    return out


def run_block_sparse_graph(graph, Q, K, V, block_mask: BlockMask, *, cos=None,
                           sin=None, out=None, save_lse=None,
                           alibi_slopes=None):
    """Block-sparse forward of a traced graph, honouring its scale, ALiBi
    (default slopes or ``alibi_slopes``) and RoPE."""
    from .kernel_cache import get_or_compile
    bundle = get_or_compile(graph)
    if bundle.bias_kind == 2:
        raise NotImplementedError("additive bias with block_sparse is not "
                                  "supported")
    if bundle.has_rope and (cos is None or sin is None):
        raise RuntimeError("this graph uses af.rope(); pass cos= and sin=")
    return run_block_sparse(Q, K, V, block_mask, bundle.sm_scale,
                            bias_kind=bundle.bias_kind, out=out,
                            save_lse=save_lse,
                            cos=cos if bundle.has_rope else None,
                            sin=sin if bundle.has_rope else None,
                            alibi_slopes=alibi_slopes)


def run_block_sparse_backward(Q, K, V, O, L, dO, block_mask: BlockMask,
                              sm_scale: float, bias_kind: int = 0, *,
                              cos=None, sin=None, alibi_slopes=None):
    """Block-sparse backward -> (dQ, dK, dV) (reference signature,
    attnfuse/runtime/block_mask.py:274-275)."""
    from .backward import _run_backward_key
    _check_mask(Q, K, block_mask)
    rope = cos is not None or sin is not None
    key = _bs_key(Q, bias_kind, rope)
    return _run_backward_key(key, Q, K, V, O, L, dO, sm_scale, 0, cos, sin,
                             block_mask, alibi_slopes)
