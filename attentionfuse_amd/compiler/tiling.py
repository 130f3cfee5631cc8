"""gfx950 tile shapes: what the launches actually use, read from the library.

Replaces the reference's Ampere/Hopper Triton tables
(reference: attnfuse/compiler/tiling.py:29-207).  There the tables feed code
generation, so a tile is a per-call choice.  Here every kernel is
instantiated ahead of time for one launch shape per specialisation key, and
the library is the single source of that shape: ``tile_for_key`` asks
``af_fwd_tile`` for the key's query rows per workgroup (32 per wave64) and
keys per LDS stage.  Block-sparse launches take BLOCK_M from the BlockMask
(the kernel walks the mask's rows).

The backward's one runtime choice -- how many dK/dV workgroups share a key
block's GQA query heads -- is read and overridden through
``runtime.backward._BWD_TILE`` / ``_pick_backward_tile`` (``af_bwd_tile``).
"""
from __future__ import annotations

import ctypes as C

from ..ir.high_level import Graph
from ..ir.spec import TileConfig

# Head dims with kernels in libattnfuse_hip.so (af_query accepts them).
SUPPORTED_HEAD_DIMS = (32, 64, 128, 256)
LDS_STAGES = 2


def tile_for_key(key_tuple) -> TileConfig:
    """Launch shape of the forward kernel for an ABI key tuple (dtype,
    head_dim, mask, bias, norm, rope); NotImplementedError when the key has
    no instantiation."""
    from ..runtime import _native as N
    bm, bn = C.c_int32(), C.c_int32()
    rc = N.lib().af_fwd_tile(N.SpecKeyC(*key_tuple), C.byref(bm), C.byref(bn))
    if rc != N.AF_OK:
        raise NotImplementedError(f"no gfx950 forward instantiation for key "
                                  f"{tuple(key_tuple)}: {N.last_error()}")
    return TileConfig(BLOCK_M=bm.value, BLOCK_N=bn.value,
                      waves=bm.value // 32, lds_stages=LDS_STAGES)


def tile_for(head_dim: int, block_m: int | None = None,
             dtype: str = "float16") -> TileConfig:
    """Shape for a plain (dense, softmax) key of ``head_dim``; with
    ``block_m`` the block-sparse walk over BlockMask rows of that height."""
    from ..ir.spec import DTYPE_CODES
    if block_m is not None:
        if block_m % 32 or not 32 <= block_m <= 128:
            raise NotImplementedError(
                f"block-sparse BLOCK_M={block_m}: the gfx950 kernels walk "
                "BlockMask rows of 32, 64 or 128 queries")
        cfg = tile_for_key((DTYPE_CODES[dtype], head_dim, 3, 0, 0, 0))
        return TileConfig(BLOCK_M=block_m, BLOCK_N=cfg.BLOCK_N,
                          waves=block_m // 32, lds_stages=LDS_STAGES)
    return tile_for_key((DTYPE_CODES[dtype], head_dim, 0, 0, 0, 0))


def choose_tile_config(graph: Graph) -> TileConfig:
    """The tile the forward launch of ``graph`` uses (reference name)."""
    from .lowering import lower_to_key
    return lower_to_key(graph).config
