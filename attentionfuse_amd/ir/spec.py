"""Specialisation key: the lowered form of a graph.

The reference lowers a graph into a flat ``TiledKernel`` record of Triton
``constexpr`` flags (reference: attnfuse/ir/tiled.py:52-81).  Here the same
facts select one of the ahead-of-time instantiated HIP kernels in
``libattnfuse_hip.so``; there is no source generation and no JIT.  The field
names of the reference record are kept so code that inspects a lowered kernel
(``head_dim``, ``mask_kind``, ``score_scale``, ``config.BLOCK_M`` ...) keeps
working.

The integer codes below are the C-ABI enums of ``include/attnfuse_hip.h``.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

from .high_level import BiasKind, MaskKind, NormKind

DTYPE_CODES = {"float16": 0, "bfloat16": 1, "float32": 2}
MASK_CODES = {MaskKind.FULL: 0, MaskKind.CAUSAL: 1,
              MaskKind.SLIDING_WINDOW: 2, MaskKind.BLOCK_SPARSE: 3,
              MaskKind.CAUSAL_SLIDING_WINDOW: 4}
BIAS_CODES = {None: 0, BiasKind.ALIBI: 1, BiasKind.ADDITIVE: 2}
NORM_CODES = {NormKind.SOFTMAX: 0, NormKind.RELU: 1}


@dataclass
class TileConfig:
    """gfx950 launch shape of the forward kernel.

    ``BLOCK_M`` query rows per workgroup (32 per wave64), ``BLOCK_N`` keys per
    LDS stage, ``waves`` per workgroup, ``lds_stages`` K/V buffers in LDS."""
    BLOCK_M: int = 128
    BLOCK_N: int = 64
    waves: int = 4
    lds_stages: int = 2

    @property
    def num_warps(self) -> int:          # reference field name
        return self.waves

    @property
    def num_stages(self) -> int:         # reference field name
        return self.lds_stages


@dataclass
class SpecKey:
    head_dim: int
    dtype: str
    score_scale: float
    mask_kind: MaskKind = MaskKind.FULL
    mask_window: Optional[int] = None
    bias_kind: Optional[BiasKind] = None
    bias_num_heads: Optional[int] = None
    norm_kind: NormKind = NormKind.SOFTMAX
    rope_kind: int = 0
    config: TileConfig = field(default_factory=TileConfig)
    cache_key: str = ""

    # -- C-ABI codes ------------------------------------------------------
    @property
    def dtype_code(self) -> int:
        return DTYPE_CODES[self.dtype]

    @property
    def mask_code(self) -> int:
        return MASK_CODES[self.mask_kind]

    @property
    def bias_code(self) -> int:
        return BIAS_CODES[self.bias_kind]

    @property
    def norm_code(self) -> int:
        return NORM_CODES[self.norm_kind]

    def abi_tuple(self) -> tuple:
        """(dtype, head_dim, mask, bias, norm, rope) as the C struct wants."""
        return (self.dtype_code, self.head_dim, self.mask_code,
                self.bias_code, self.norm_code, int(self.rope_kind))


# The reference calls the lowered record a TiledKernel.
TiledKernel = SpecKey
