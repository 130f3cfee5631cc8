"""gfx950 tile table for the forward kernel.

Replaces the reference's Ampere/Hopper Triton tables
(reference: attnfuse/compiler/tiling.py:29-207).  On MI355X every forward
instantiation uses wave64 workgroups whose waves each own 32 query rows (one
32x32 MFMA output block), 64-key K/V stages double-buffered in LDS, and the
number of waves per workgroup picked from the head dimension:

* D <= 128: 4 waves (BLOCK_M = 128) -- two workgroups fit a CU's 160 KiB LDS
  and 512-entry register file, so one workgroup's MFMA work overlaps the
  other's softmax VALU work.
* D == 256: 2 waves (BLOCK_M = 64) -- the 32x256 fp32 output accumulator
  alone is 128 registers per lane.

Block-sparse graphs take BLOCK_M from the BlockMask (the kernel walks the
mask's rows), so the table is consulted with ``block_m``.
"""
from __future__ import annotations

from ..ir.high_level import Graph
from ..ir.spec import TileConfig

SUPPORTED_HEAD_DIMS = (32, 64, 96, 128, 256)
KEYS_PER_STAGE = 64


def tile_for(head_dim: int, block_m: int | None = None) -> TileConfig:
    if block_m is not None:
        if block_m % 32 or not 32 <= block_m <= 128:
            raise NotImplementedError(
                f"block-sparse BLOCK_M={block_m}: the gfx950 kernels walk "
                "BlockMask rows of 32, 64 or 128 queries")
        return TileConfig(BLOCK_M=block_m, BLOCK_N=KEYS_PER_STAGE,
                          waves=block_m // 32, lds_stages=2)
    waves = 2 if head_dim > 128 else 4
    return TileConfig(BLOCK_M=32 * waves, BLOCK_N=KEYS_PER_STAGE, waves=waves,
                      lds_stages=2)


def choose_tile_config(graph: Graph) -> TileConfig:
    return tile_for(graph.q.head_dim)
