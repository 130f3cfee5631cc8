"""CPU oracle for the fused-attention path.

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` as the checker / CPU baseline, never
by the product package.
"""
from .attention import (alibi_slopes, apply_rope, attention_grads,
                        bigbird_grid, block_classes, block_grid, block_lists,
                        decode_split_combine, element_mask_from_grid,
                        expand_kv, expected_coverage, naive_attention,
                        rope_tables, rotate_half)

__all__ = ["alibi_slopes", "apply_rope", "attention_grads", "bigbird_grid",
           "block_classes", "block_grid", "block_lists", "decode_split_combine",
           "element_mask_from_grid", "expand_kv", "expected_coverage",
           "naive_attention", "rope_tables", "rotate_half"]
