"""af_blockmask_plan, the work plan of split block-sparse walks (host code,
no GPU): every list entry is walked by exactly one piece, pieces are
near-equal and no longer than the chunk, split lists own contiguous partial
slots, and the items run longest first."""
import ctypes as C

import pytest
import torch

from attnfuse.runtime import _native as N
from attnfuse.runtime.block_mask import _plan_lists


def check_plan(counts, chunk):
    items, splits, slots = _plan_lists(torch.tensor(counts, dtype=torch.int32), chunk)
    items, splits = items.tolist(), splits.tolist()
    n = len(counts)
    if chunk <= 0:
        chunk = max(8, 2 * -(-sum(counts) // max(n, 1)))
    # exact cover of every list's entries
    seen = {i: [] for i in range(n)}
    for lst, e0, ne, slot in items:
        seen[lst].append((e0, ne, slot))
    for i, c in enumerate(counts):
        pieces = sorted(seen[i])
        assert pieces, f"list {i} has no item"
        covered = [e for e0, ne, _ in pieces for e in range(e0, e0 + ne)]
        assert covered == list(range(c)), (i, pieces)
        lens = [ne for _, ne, _ in pieces]
        assert max(lens) <= max(chunk, c if len(pieces) == 1 else 0)
        assert max(lens) - min(lens) <= 1
        if len(pieces) == 1:
            assert pieces[0][2] == -1 and c <= chunk
        else:
            assert c > chunk
    # splits: one per multi-piece list, contiguous disjoint slots
    multi = {i for i in range(n) if len(seen[i]) > 1}
    assert {s[0] for s in splits} == multi
    used = []
    for lst, s0, k in splits:
        got = sorted(slot for _, _, slot in seen[lst])
        assert got == list(range(s0, s0 + k))
        used += got
    assert sorted(used) == list(range(slots))
    # longest first
    lens = [ne for _, _, ne, _ in items]
    assert lens == sorted(lens, reverse=True)
    return items, splits, slots


@pytest.mark.parametrize("chunk", [0, 1, 2, 3, 8, 1000])
def test_plan_covers_every_entry(chunk):
    g = torch.Generator().manual_seed(0)
    for trial in range(20):
        n = int(torch.randint(1, 40, (1,), generator=g))
        counts = torch.randint(0, 12, (n,), generator=g).tolist()
        if trial % 3 == 0:
            counts[0] = n * 4  # a global row
        check_plan(counts, chunk)


def test_bigbird_global_row_is_cut_to_twice_the_mean():
    counts = [64] + [7] * 63
    items, splits, slots = check_plan(counts, 0)
    assert splits == [[0, 0, 4]] and slots == 4   # 2 ceil(mean) = 16 -> 4 pieces
    assert len(items) == 63 + 4 and all(ne <= 16 for _, _, ne, _ in items)
    assert [ne for _, _, ne, _ in items[:4]] == [16] * 4   # longest first


def test_empty_and_short_lists_keep_one_unsplit_item():
    items, splits, slots = check_plan([0, 0, 3], 0)
    assert slots == 0 and splits == [] and len(items) == 3
    items, splits, slots = check_plan([], 0)
    assert items == [] and splits == [] and slots == 0


def test_plan_argument_errors():
    lib = N.lib()
    sizes = (C.c_int32 * 3)()
    bad = torch.tensor([3, -1], dtype=torch.int32)
    assert lib.af_blockmask_plan(C.c_void_p(bad.data_ptr()), 2, 0, None, None, sizes) == N.AF_ERR_BAD_ARG
    assert "negative" in N.last_error()
    assert lib.af_blockmask_plan(None, 3, 0, None, None, sizes) == N.AF_ERR_BAD_ARG
    ok = torch.tensor([1], dtype=torch.int32)
    assert lib.af_blockmask_plan(C.c_void_p(ok.data_ptr()), 1, 0, None, None, None) == N.AF_ERR_BAD_ARG
