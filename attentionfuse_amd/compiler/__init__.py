"""Compiler: Graph -> SpecKey (selects an ahead-of-time HIP instantiation)."""
from .fusion import FusionError, fuse_score_softmax
from .lowering import kernel_constexprs, lower_to_key, lower_to_tiled
from .tiling import choose_tile_config, tile_for

__all__ = ["FusionError", "fuse_score_softmax", "lower_to_key",
           "lower_to_tiled", "kernel_constexprs", "choose_tile_config",
           "tile_for"]
