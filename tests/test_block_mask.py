"""BlockMask construction on the CPU against the oracle's per-tile loop and
the reference tests' known answers."""
import json
from pathlib import Path

import pytest
import torch

import attnfuse as af
import oracle as O
from attentionfuse_amd.runtime.block_mask import block_mask_from_blocks

PREDS = {
    "all": lambda q, k: torch.ones_like(q, dtype=torch.bool),
    "local": lambda q, k: ((q // 64) - (k // 64)).abs() <= 1,
    "bigbird": lambda q, k: ((q // 64) == 0) | ((k // 64) == 0) | (((q // 64) - (k // 64)).abs() <= 1),
    "strided": lambda q, k: ((q // 64) + (k // 64)) % 2 == 0,
    "causal_elem": lambda q, k: k <= q,
    "diag_point": lambda q, k: (q == k) & (q % 97 == 0),
}


def _check(bm, grid):
    rows, cols = O.block_lists(grid)
    fn, fi = bm.full_kv_num.tolist(), bm.full_kv_idx.tolist()
    assert bm.full_kv_idx.dtype == torch.int32
    assert bm.full_kv_idx.shape[1] == max(1, max(len(r) for r in rows))
    for r, want in enumerate(rows):
        assert fn[r] == len(want)
        assert fi[r][: len(want)] == want
        assert all(x == 0 for x in fi[r][len(want):])
    qn, qi = bm.q_num_blocks.tolist(), bm.q_indices.tolist()
    for c, want in enumerate(cols):
        assert qn[c] == len(want) and qi[c][: len(want)] == want
    assert bm.kv_num_blocks.sum() == 0
    assert bm.n_active == int(grid.sum()) == bm.n_full
    assert torch.equal(bm.dense_blocks(), grid)


@pytest.mark.parametrize("name", sorted(PREDS))
@pytest.mark.parametrize("shape", [(256, 256, 64, 64), (300, 200, 64, 64), (256, 512, 128, 64)])
def test_create_block_mask_matches_oracle(name, shape):
    q_len, kv_len, bm_, bn = shape
    bm = af.create_block_mask(PREDS[name], q_len, kv_len, bm_, bn, device="cpu")
    grid = O.block_grid(PREDS[name], q_len, kv_len, bm_, bn)
    assert (bm.n_q_blocks, bm.n_kv_blocks) == tuple(grid.shape)
    _check(bm, grid)


def test_reference_known_answers():
    N = 256
    assert af.create_block_mask(PREDS["all"], N, N, device="cpu").n_active == 16
    assert af.create_block_mask(PREDS["local"], N, N, device="cpu").n_active == 10
    assert af.create_block_mask(PREDS["strided"], N, N, device="cpu").n_active == 8


def test_bigbird_fixture_roundtrip():
    fx = json.loads((Path(__file__).parent / "golden" / "bigbird_c4_grid.json").read_text())
    n = fx["n_blocks"]
    grid = torch.zeros(n, n, dtype=torch.bool)
    for a, row in enumerate(fx["rows"]):
        grid[a, row] = True
    bm = block_mask_from_blocks(grid, 64, 64, device="cpu")
    _check(bm, grid)
    assert bm.n_active == fx["n_active"]


def test_block_mask_to_device_keeps_fields():
    bm = af.create_block_mask(PREDS["local"], 256, 256, device="cpu")
    bm2 = bm.to("cpu")
    assert bm2.n_active == bm.n_active and torch.equal(bm2.full_kv_idx, bm.full_kv_idx)


ELEM_PREDS = {
    "causal_elem": PREDS["causal_elem"],
    "diag_point": PREDS["diag_point"],
    "local": PREDS["local"],
    "window_elem": lambda q, k: (q - k).abs() < 70,
    "pattern": lambda q, k: ((q * 7 + k * 13) % 5 != 0) & ((q - k).abs() < 150),
}


def _unpack(words: torch.Tensor, nbits: int) -> torch.Tensor:
    """(..., w) int64 words -> (..., nbits) bool, bit k of word w = element
    64 w + k."""
    bits = (words[..., None] >> torch.arange(64)) & 1
    return bits.bool().reshape(*words.shape[:-1], -1)[..., :nbits]


@pytest.mark.parametrize("name", sorted(ELEM_PREDS))
@pytest.mark.parametrize("shape", [(256, 256, 64, 64), (300, 200, 64, 64), (256, 512, 128, 64),
                                   (200, 300, 32, 128), (320, 384, 128, 128)])
def test_exact_block_mask_lists_and_bits(name, shape):
    """create_block_mask(exact=True) against the reference's per-tile
    classification, and its bit words decoded back to the element mask."""
    q_len, kv_len, bm_, bn = shape
    pred = ELEM_PREDS[name]
    bm = af.create_block_mask(pred, q_len, kv_len, bm_, bn, device="cpu", exact=True)
    full, part = O.block_classes(pred, q_len, kv_len, bm_, bn)
    frows, _ = O.block_lists(full)
    prows, _ = O.block_lists(part)
    _, cols = O.block_lists(full | part)
    fn, fi = bm.full_kv_num.tolist(), bm.full_kv_idx.tolist()
    pn, pi = bm.kv_num_blocks.tolist(), bm.kv_indices.tolist()
    for r in range(bm.n_q_blocks):
        assert fi[r][: fn[r]] == frows[r]
        assert pi[r][: pn[r]] == prows[r]
    qn, qi = bm.q_num_blocks.tolist(), bm.q_indices.tolist()
    qp = bm.q_partial.tolist()
    for c, want in enumerate(cols):
        assert qi[c][: qn[c]] == want
        assert [qp[c][j] for j in range(qn[c])] == [int(part[a, c]) for a in want]
    assert bm.n_full == int(full.sum()) and bm.n_active == int((full | part).sum())
    # the element mask the kernels apply: full tiles whole, partial tiles
    # through their row bits (Q-major) and column bits (K-major)
    qi_ = torch.arange(q_len)[:, None].expand(q_len, kv_len)
    kj_ = torch.arange(kv_len)[None, :].expand(q_len, kv_len)
    elem = torch.as_tensor(pred(qi_, kj_), dtype=torch.bool).expand(q_len, kv_len)
    nqb, nkb = bm.n_q_blocks, bm.n_kv_blocks
    rows = torch.zeros(nqb * bm_, nkb * bn, dtype=torch.bool)
    colm = torch.zeros(nqb * bm_, nkb * bn, dtype=torch.bool)
    for a in range(nqb):
        for b in frows[a]:
            rows[a * bm_:(a + 1) * bm_, b * bn:(b + 1) * bn] = True
        for e, b in enumerate(prows[a]):
            rows[a * bm_:(a + 1) * bm_, b * bn:(b + 1) * bn] = _unpack(bm.part_row_bits[a, e], bn)
    for b, want in enumerate(cols):
        for j, a in enumerate(want):
            if qp[b][j]:
                colm[a * bm_:(a + 1) * bm_, b * bn:(b + 1) * bn] = _unpack(bm.q_col_bits[b, j], bm_).t()
            else:
                colm[a * bm_:(a + 1) * bm_, b * bn:(b + 1) * bn] = True
    assert torch.equal(rows[:q_len, :kv_len], elem)
    assert torch.equal(colm[:q_len, :kv_len], elem)


def test_exact_mask_of_block_aligned_predicate_has_no_partials():
    bm = af.create_block_mask(PREDS["bigbird"], 512, 512, device="cpu", exact=True)
    assert int(bm.kv_num_blocks.sum()) == 0 and int(bm.q_partial.sum()) == 0
    assert bm.n_active == af.create_block_mask(PREDS["bigbird"], 512, 512, device="cpu").n_active


def test_exact_mask_needs_whole_key_words():
    with pytest.raises(NotImplementedError):
        af.create_block_mask(PREDS["causal_elem"], 256, 256, 64, 32, device="cpu", exact=True)
