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
