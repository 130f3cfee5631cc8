"""Block-sparse walks with split rows and columns (af_blockmask_plan pieces
merged by the combine kernels) against the oracle: forward O and LSE, tile
coverage, dQ/dK/dV, with RoPE + ALiBi, GQA (with and without the head-group
split, which turns the K-major plan off), empty rows and 128-row blocks."""
import pytest
import torch

import oracle as O
from attnfuse.rope_utils import build_rope_cache
from attnfuse.runtime import backward as BW
from attnfuse.runtime.block_mask import (block_mask_from_blocks, run_block_sparse,
                                         run_block_sparse_backward)

pytestmark = pytest.mark.gpu
TOL = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}
LSE_TOL = {torch.float16: 5e-3, torch.bfloat16: 3e-2}
GRAD_REL = 1e-2


def rand(shape, dtype, g):
    return torch.randn(*shape, generator=g, device="cuda", dtype=dtype)


def grid_with_globals(n, seed, empty_rows=()):
    """Global row 0 and column 0, a +-1 band, two random blocks per row, and
    optionally some rows with no block at all."""
    g = torch.Generator().manual_seed(seed)
    grid = torch.zeros(n, n, dtype=torch.bool)
    grid[0, :] = True
    grid[:, 0] = True
    for i in range(n):
        grid[i, max(i - 1, 0): i + 2] = True
        grid[i, torch.randint(0, n, (2,), generator=g)] = True
    for r in empty_rows:
        grid[r, :] = False
    return grid


def check_forward(Q, K, V, grid, bmq, bnk, dtype, chunk, **kw):
    Nq, Nkv = Q.shape[2], K.shape[2]
    bm = block_mask_from_blocks(grid, bmq, bnk, device="cuda")
    plan = bm.plan_work(chunk)
    assert plan.q_splits.shape[0] > 0 and plan.kv_splits.shape[0] > 0
    lse = torch.empty(Q.shape[:3], device="cuda", dtype=torch.float32)
    cov = torch.zeros(Q.shape[0], Q.shape[1], -(-Nq // 32), -(-Nkv // 64), dtype=torch.int32, device="cuda")
    out = run_block_sparse(Q, K, V, bm, Q.shape[-1] ** -0.5, save_lse=lse, coverage=cov, **kw)
    torch.cuda.synchronize()
    em = O.element_mask_from_grid(grid, Nq, Nkv, bmq, bnk)
    return bm, out, lse, cov, em


@pytest.mark.parametrize("chunk", [1, 2, 3])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
def test_split_forward_lse_and_coverage(dtype, chunk):
    print(f"[bs-split] fwd {dtype} chunk={chunk}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(10 + chunk)
    n, D = 8, 64
    Q, K, V = (rand((2, 3, 64 * n, D), dtype, g) for _ in range(3))
    grid = grid_with_globals(n, seed=chunk, empty_rows=(5,))
    bm, out, lse, cov, em = check_forward(Q, K, V, grid, 64, 64, dtype, chunk)
    want, want_l = O.naive_attention(Q.cpu(), K.cpu(), V.cpu(), elem_mask=em, return_lse=True)
    assert (out.float().cpu() - want).abs().max().item() <= TOL[dtype]
    got_l = lse.cpu()
    fin = torch.isfinite(want_l)
    assert torch.equal(torch.isfinite(got_l), fin)          # empty row: -inf
    assert (got_l[fin] - want_l[fin]).abs().max().item() <= LSE_TOL[dtype]
    assert out[:, :, 5 * 64: 6 * 64].abs().max().item() == 0.0
    exp_cov = O.expected_coverage(64 * n, 64 * n, mask="block_sparse", grid=grid, bm=64, bn=64)
    assert torch.equal(cov.cpu(), exp_cov.expand(2, 3, *exp_cov.shape))


@pytest.mark.parametrize("chunk", [1, 3])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
def test_split_backward(dtype, chunk):
    print(f"[bs-split] bwd {dtype} chunk={chunk}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(20 + chunk)
    n, D = 8, 64
    Q, K, V, dO = (rand((2, 3, 64 * n, D), dtype, g) for _ in range(4))
    grid = grid_with_globals(n, seed=7 + chunk, empty_rows=(3,))
    bm = block_mask_from_blocks(grid, 64, 64, device="cuda")
    bm.plan_work(chunk)
    lse = torch.empty(Q.shape[:3], device="cuda", dtype=torch.float32)
    out = run_block_sparse(Q, K, V, bm, D ** -0.5, save_lse=lse)
    dq, dk, dv = run_block_sparse_backward(Q, K, V, out, lse, dO, bm, D ** -0.5)
    torch.cuda.synchronize()
    em = O.element_mask_from_grid(grid, 64 * n, 64 * n, 64, 64)
    o_ref, rq, rk, rv = O.attention_grads(Q.cpu(), K.cpu(), V.cpu(), dO.cpu(), dtype=torch.float32, elem_mask=em)
    assert (out.float().cpu() - o_ref).abs().max().item() <= TOL[dtype]
    for got, ref in ((dq, rq), (dk, rk), (dv, rv)):
        assert ((got.float().cpu() - ref).norm() / ref.norm()).item() <= GRAD_REL


@pytest.mark.parametrize("group_split", [0, 2])
def test_split_gqa_rope_alibi(group_split, monkeypatch):
    """Hq = 4 over Hkv = 2 with RoPE and ALiBi; group_split 0 keeps the
    heads together and walks the split columns, 2 turns the K-major plan
    off (the head-group partials take over)."""
    print(f"[bs-split] gqa rope alibi group_split={group_split}", flush=True)
    dtype = torch.float16
    monkeypatch.setitem(BW._BWD_TILE, "auto", group_split == 0)
    monkeypatch.setitem(BW._BWD_TILE, "group_split", group_split)
    g = torch.Generator(device="cuda").manual_seed(31)
    n, D = 6, 64
    Nn = 64 * n
    Q, dO = (rand((1, 4, Nn, D), dtype, g) for _ in range(2))
    K, V = (rand((1, 2, Nn, D), dtype, g) for _ in range(2))
    cos, sin = build_rope_cache(Nn, D, device="cuda", dtype=dtype)
    slopes = torch.tensor(O.alibi_slopes(4), dtype=torch.float32, device="cuda")
    grid = grid_with_globals(n, seed=5)
    bm = block_mask_from_blocks(grid, 64, 64, device="cuda")
    bm.plan_work(2)
    lse = torch.empty(Q.shape[:3], device="cuda", dtype=torch.float32)
    out = run_block_sparse(Q, K, V, bm, D ** -0.5, bias_kind=1, save_lse=lse, cos=cos, sin=sin,
                           alibi_slopes=slopes)
    dq, dk, dv = run_block_sparse_backward(Q, K, V, out, lse, dO, bm, D ** -0.5, bias_kind=1, cos=cos, sin=sin,
                                           alibi_slopes=slopes)
    torch.cuda.synchronize()
    em = O.element_mask_from_grid(grid, Nn, Nn, 64, 64)
    o_ref, rq, rk, rv = O.attention_grads(Q.cpu(), K.cpu(), V.cpu(), dO.cpu(), dtype=torch.float32, elem_mask=em,
                                          alibi_slopes=slopes.cpu(), rope=(cos[0, 0].cpu(), sin[0, 0].cpu()))
    assert (out.float().cpu() - o_ref).abs().max().item() <= TOL[dtype]
    for got, ref in ((dq, rq), (dk, rk), (dv, rv)):
        assert ((got.float().cpu() - ref).norm() / ref.norm()).item() <= GRAD_REL


@pytest.mark.parametrize("blocks", [(128, 64), (64, 128), (128, 128)])
def test_split_block_sizes(blocks):
    print(f"[bs-split] blocks {blocks}", flush=True)
    bmq, bnk = blocks
    dtype = torch.bfloat16
    g = torch.Generator(device="cuda").manual_seed(41)
    Nn, D = 768, 64
    Q, K, V, dO = (rand((1, 2, Nn, D), dtype, g) for _ in range(4))
    grid = grid_with_globals(Nn // max(bmq, bnk), seed=9)
    # the grid is square in blocks of max(bmq, bnk); re-cut to (bmq, bnk)
    em = O.element_mask_from_grid(grid, Nn, Nn, max(bmq, bnk), max(bmq, bnk))
    g2 = em.view(Nn // bmq, bmq, Nn // bnk, bnk).any(dim=3).any(dim=1)
    bm = block_mask_from_blocks(g2, bmq, bnk, device="cuda")
    bm.plan_work(1)
    lse = torch.empty(Q.shape[:3], device="cuda", dtype=torch.float32)
    out = run_block_sparse(Q, K, V, bm, D ** -0.5, save_lse=lse)
    dq, dk, dv = run_block_sparse_backward(Q, K, V, out, lse, dO, bm, D ** -0.5)
    torch.cuda.synchronize()
    o_ref, rq, rk, rv = O.attention_grads(Q.cpu(), K.cpu(), V.cpu(), dO.cpu(), dtype=torch.float32,
                                          elem_mask=O.element_mask_from_grid(g2, Nn, Nn, bmq, bnk))
    assert (out.float().cpu() - o_ref).abs().max().item() <= TOL[dtype]
    for got, ref in ((dq, rq), (dk, rk), (dv, rv)):
        assert ((got.float().cpu() - ref).norm() / ref.norm()).item() <= GRAD_REL


def test_split_head_dim_256_and_128():
    print("[bs-split] D=128/256", flush=True)
    dtype = torch.float16
    for D in (128, 256):
        g = torch.Generator(device="cuda").manual_seed(50 + D)
        n = 5
        Q, K, V, dO = (rand((1, 2, 64 * n, D), dtype, g) for _ in range(4))
        grid = grid_with_globals(n, seed=D)
        bm = block_mask_from_blocks(grid, 64, 64, device="cuda")
        bm.plan_work(1)
        lse = torch.empty(Q.shape[:3], device="cuda", dtype=torch.float32)
        out = run_block_sparse(Q, K, V, bm, D ** -0.5, save_lse=lse)
        dq, dk, dv = run_block_sparse_backward(Q, K, V, out, lse, dO, bm, D ** -0.5)
        torch.cuda.synchronize()
        em = O.element_mask_from_grid(grid, 64 * n, 64 * n, 64, 64)
        o_ref, rq, rk, rv = O.attention_grads(Q.cpu(), K.cpu(), V.cpu(), dO.cpu(), dtype=torch.float32,
                                              elem_mask=em)
        assert (out.float().cpu() - o_ref).abs().max().item() <= TOL[dtype], D
        for got, ref in ((dq, rq), (dk, rk), (dv, rv)):
            assert ((got.float().cpu() - ref).norm() / ref.norm()).item() <= GRAD_REL, D
