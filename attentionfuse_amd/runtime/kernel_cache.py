"""Graph signature -> launch bundle (specialisation key + scalar launch facts).

Replaces the reference's compile cache (reference:
attnfuse/runtime/kernel_cache.py:25-87).  Nothing is compiled at run time:
every kernel is instantiated ahead of time in libattnfuse_hip.so, so a cache
miss lowers the graph to a SpecKey, asks the library whether that key is
instantiated (``af_query``), and memoises the answer.
"""
from __future__ import annotations

import os
import threading
from dataclasses import dataclass

from ..compiler.lowering import lower_to_key
from ..ir.high_level import Graph
from ..ir.spec import SpecKey
from . import _native as N

_lock = threading.Lock()
_cache: dict = {}


@dataclass(frozen=True)
class LaunchBundle:
    key: SpecKey
    sm_scale: float
    block_m: int
    bias_kind: int            # 0 none, 1 ALiBi, 2 additive
    has_additive_bias: bool
    has_rope: bool
    window: int

    @property
    def kernel(self) -> SpecKey:   # reference field name
        return self.key


def get_or_compile(graph: Graph) -> LaunchBundle:
    sig = graph.signature()
    with _lock:
        hit = _cache.get(sig)
        if hit is not None:
            return hit
        key = lower_to_key(graph)
        ck = N.SpecKeyC(*key.abi_tuple())
        if not N.lib().af_query(ck):
            raise NotImplementedError(
                f"no gfx950 instantiation for {key.dtype} head_dim="
                f"{key.head_dim} mask={key.mask_kind.value}: "
                f"{N.last_error()}")
        if os.environ.get("ATTNFUSE_DEBUG"):
            from ..ir.printer import format_key
            print(f"[AttnFuse] specialisation key:\n{format_key(key)}")
        bundle = LaunchBundle(
            key=key, sm_scale=float(key.score_scale),
            block_m=key.config.BLOCK_M, bias_kind=key.bias_code,
            has_additive_bias=key.bias_code == 2,
            has_rope=bool(key.rope_kind), window=int(key.mask_window or 0))
        _cache[sig] = bundle
        return bundle


def clear_cache() -> None:
    with _lock:
        _cache.clear()
