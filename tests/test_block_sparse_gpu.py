"""Block-sparse forward and backward on the GPU (the reference's
tests/test_block_sparse.py patterns at the tighter tolerances, the BigBird
benchmark mask fixture, tile coverage and RoPE/ALiBi with a block mask)."""
import json
from pathlib import Path

import pytest
import torch

import attnfuse as af
import oracle as O
from attnfuse.rope_utils import build_rope_cache
from attnfuse.runtime.block_mask import block_mask_from_blocks, run_block_sparse
from attnfuse.runtime.dispatch import _alibi_slopes

pytestmark = pytest.mark.gpu
TOL = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}
GRAD_REL = 1e-2
B, H, N, D = 2, 4, 256, 64

PATTERNS = {
    "all": lambda q, k: torch.ones_like(q, dtype=torch.bool),
    "local": lambda q, k: ((q // 64) - (k // 64)).abs() <= 1,
    "bigbird": lambda q, k: ((q // 64) == 0) | ((k // 64) == 0) | (((q // 64) - (k // 64)).abs() <= 1),
    "strided": lambda q, k: ((q // 64) + (k // 64)) % 2 == 0,
}


@af.attention
def bs_attn(Q, K, V):
    return af.softmax(af.block_sparse(af.scaled_dot_product(Q, K))) @ V


def make(Bn, Hn, Nn, Dn, dtype, seed=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return tuple(torch.randn(Bn, Hn, Nn, Dn, generator=g, device="cuda", dtype=dtype) for _ in range(4))


def elem_mask(grid, Nn, bm=64, bn=64):
    return O.element_mask_from_grid(grid, Nn, Nn, bm, bn)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("name", sorted(PATTERNS))
def test_forward_patterns(name, dtype):
    print(f"[bs] fwd {name} {dtype}", flush=True)
    Q, K, V, _ = make(B, H, N, D, dtype)
    bm = af.create_block_mask(PATTERNS[name], N, N, 64, 64)
    out = bs_attn(Q, K, V, block_mask=bm)
    torch.cuda.synchronize()
    grid = O.block_grid(PATTERNS[name], N, N, 64, 64)
    want = O.naive_attention(Q.cpu(), K.cpu(), V.cpu(), elem_mask=elem_mask(grid, N))
    assert (out.float().cpu() - want).abs().max().item() <= TOL[dtype]


def test_reference_known_answers_and_missing_mask():
    assert af.create_block_mask(PATTERNS["all"], N, N).n_active == 16
    assert af.create_block_mask(PATTERNS["local"], N, N).n_active == 10
    assert af.create_block_mask(PATTERNS["strided"], N, N).n_active == 8
    Q, K, V, _ = make(1, 2, N, D, torch.float16)
    with pytest.raises(RuntimeError, match="block_mask"):
        bs_attn(Q, K, V)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("name", ["local", "bigbird", "strided", "all"])
def test_backward_patterns(name, dtype):
    print(f"[bs] bwd {name} {dtype}", flush=True)
    Q, K, V, dO = make(B, H, N, D, dtype, seed=1)
    bm = af.create_block_mask(PATTERNS[name], N, N, 64, 64)
    q, k, v = (t.clone().requires_grad_(True) for t in (Q, K, V))
    out = bs_attn(q, k, v, block_mask=bm)
    out.backward(dO)
    torch.cuda.synchronize()
    grid = O.block_grid(PATTERNS[name], N, N, 64, 64)
    o_ref, dq, dk, dv = O.attention_grads(Q.cpu(), K.cpu(), V.cpu(), dO.cpu(), dtype=torch.float32,
                                          elem_mask=elem_mask(grid, N))
    assert (out.detach().float().cpu() - o_ref).abs().max().item() <= TOL[dtype]
    for got, ref in ((q.grad, dq), (k.grad, dk), (v.grad, dv)):
        assert ((got.float().cpu() - ref).norm() / ref.norm()).item() <= GRAD_REL


def test_reference_autograd_binding():
    """AttnFuseBlockSparseFunction.apply(Q, K, V, block_mask, bias_kind)."""
    from attnfuse.runtime.autograd import AttnFuseBlockSparseFunction
    Q, K, V, dO = make(1, 4, N, D, torch.float16, seed=2)
    bm = af.create_block_mask(PATTERNS["bigbird"], N, N)
    q, k, v = (t.clone().requires_grad_(True) for t in (Q, K, V))
    out = AttnFuseBlockSparseFunction.apply(q, k, v, bm, 1)
    out.backward(dO)
    torch.cuda.synchronize()
    grid = O.block_grid(PATTERNS["bigbird"], N, N, 64, 64)
    sl = _alibi_slopes(4, "cpu", "torch.float16").float()
    o_ref, dq, dk, dv = O.attention_grads(Q.cpu(), K.cpu(), V.cpu(), dO.cpu(), dtype=torch.float32,
                                          elem_mask=elem_mask(grid, N), alibi_slopes=sl)
    assert (out.detach().float().cpu() - o_ref).abs().max().item() <= TOL[torch.float16]
    for got, ref in ((q.grad, dq), (k.grad, dk), (v.grad, dv)):
        assert ((got.float().cpu() - ref).norm() / ref.norm()).item() <= GRAD_REL


def test_bigbird_benchmark_mask_fixture():
    """The config-4 mask (64x64 blocks of 64, BigBird + 3 random blocks per
    row) on one batch x two heads at full length 4096, forward + backward."""
    fx = json.loads((Path(__file__).parent / "golden" / "bigbird_c4_grid.json").read_text())
    n = fx["n_blocks"]
    grid = torch.zeros(n, n, dtype=torch.bool)
    for a, row in enumerate(fx["rows"]):
        grid[a, row] = True
    Nn = 64 * n
    bm = block_mask_from_blocks(grid, 64, 64, device="cuda")
    assert bm.n_active == fx["n_active"]
    Q, K, V, dO = make(1, 2, Nn, 64, torch.float16, seed=3)
    q, k, v = (t.clone().requires_grad_(True) for t in (Q, K, V))
    out = bs_attn(q, k, v, block_mask=bm)
    out.backward(dO)
    torch.cuda.synchronize()
    o_ref, dq, dk, dv = O.attention_grads(Q.cpu(), K.cpu(), V.cpu(), dO.cpu(), dtype=torch.float32,
                                          elem_mask=elem_mask(grid, Nn))
    assert (out.detach().float().cpu() - o_ref).abs().max().item() <= TOL[torch.float16]
    for got, ref in ((q.grad, dq), (k.grad, dk), (v.grad, dv)):
        assert ((got.float().cpu() - ref).norm() / ref.norm()).item() <= GRAD_REL


@pytest.mark.parametrize("blocks", [(64, 64), (128, 64), (64, 128), (128, 128)])
def test_block_sizes_and_coverage(blocks):
    bmq, bnk = blocks
    Nn = 384
    pred = lambda q, k: ((q // bmq) == (k // bnk)) | ((k // bnk) == 0)
    Q, K, V, _ = make(1, 2, Nn, D, torch.bfloat16, seed=4)
    bm = af.create_block_mask(pred, Nn, Nn, bmq, bnk)
    cov = torch.zeros(1, 2, Nn // 32, Nn // 64, dtype=torch.int32, device="cuda")
    out = run_block_sparse(Q, K, V, bm, D ** -0.5, coverage=cov)
    torch.cuda.synchronize()
    grid = O.block_grid(pred, Nn, Nn, bmq, bnk)
    want = O.naive_attention(Q.cpu(), K.cpu(), V.cpu(), elem_mask=O.element_mask_from_grid(grid, Nn, Nn, bmq, bnk))
    assert (out.float().cpu() - want).abs().max().item() <= TOL[torch.bfloat16]
    exp_cov = O.expected_coverage(Nn, Nn, mask="block_sparse", grid=grid, bm=bmq, bn=bnk)
    assert torch.equal(cov.cpu(), exp_cov.expand(1, 2, *exp_cov.shape))


def test_rope_and_alibi_with_block_mask():
    fn = af.attention(lambda Q, K, V: af.softmax(af.alibi(af.block_sparse(af.rope(Q, K)), 4)) @ V)
    Q, K, V, dO = make(1, 4, N, D, torch.float16, seed=5)
    cos, sin = build_rope_cache(N, D, device="cuda", dtype=torch.float16)
    bm = af.create_block_mask(PATTERNS["bigbird"], N, N)
    q, k, v = (t.clone().requires_grad_(True) for t in (Q, K, V))
    out = fn(q, k, v, block_mask=bm, cos=cos, sin=sin)
    out.backward(dO)
    torch.cuda.synchronize()
    grid = O.block_grid(PATTERNS["bigbird"], N, N, 64, 64)
    sl = _alibi_slopes(4, "cpu", "torch.float16").float()
    o_ref, dq, dk, dv = O.attention_grads(Q.cpu(), K.cpu(), V.cpu(), dO.cpu(), dtype=torch.float32,
                                          elem_mask=elem_mask(grid, N), alibi_slopes=sl,
                                          rope=(cos[0, 0].cpu(), sin[0, 0].cpu()))
    assert (out.detach().float().cpu() - o_ref).abs().max().item() <= TOL[torch.float16]
    for got, ref in ((q.grad, dq), (k.grad, dk), (v.grad, dv)):
        assert ((got.float().cpu() - ref).norm() / ref.norm()).item() <= GRAD_REL


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
def test_head_dim_256_forward_and_backward(dtype):
    """BigBird-style block mask at head dim 256, forward and backward."""
    print(f"[bs] D256 {dtype}", flush=True)
    Q, K, V, dO = make(1, 2, N, 256, dtype, seed=3)
    bm = af.create_block_mask(PATTERNS["bigbird"], N, N, 64, 64)
    q, k, v = (t.clone().requires_grad_(True) for t in (Q, K, V))
    out = bs_attn(q, k, v, block_mask=bm)
    out.backward(dO)
    torch.cuda.synchronize()
    grid = O.block_grid(PATTERNS["bigbird"], N, N, 64, 64)
    o_ref, dq, dk, dv = O.attention_grads(Q.cpu(), K.cpu(), V.cpu(), dO.cpu(), dtype=torch.float32,
                                          elem_mask=elem_mask(grid, N))
    assert (out.detach().float().cpu() - o_ref).abs().max().item() <= TOL[dtype]
    for got, ref in ((q.grad, dq), (k.grad, dk), (v.grad, dv)):
        assert ((got.float().cpu() - ref).norm() / ref.norm()).item() <= GRAD_REL


def test_lists_edited_in_place_between_launches():
    """A mask whose lists are rewritten in place on the device (as between
    graph replays) is walked to its new lengths without remaking the work
    plan: whole (unsplit) lists take their counts from the device.  Grid A
    has rows and columns of 2 or 3 tiles, grid B of 3 everywhere, with the
    same padded widths; B's lists are copied into A's tensors and the same
    BlockMask object is launched again."""
    from attnfuse.runtime.block_mask import run_block_sparse_backward
    print("[bs] lists edited in place", flush=True)
    Nn, nb = 512, 8
    r = torch.arange(nb)
    grid_a = (r[:, None] - r[None, :]).abs() <= 1
    grid_b = torch.zeros(nb, nb, dtype=torch.bool)
    for i in range(nb):
        grid_b[i, [i, (i + 2) % nb, (i + 5) % nb]] = True
    bm = block_mask_from_blocks(grid_a, 64, 64, device="cuda")
    bm_b = block_mask_from_blocks(grid_b, 64, 64, device="cuda")
    assert bm.plan.q_splits.shape[0] == 0 and bm.plan.kv_splits.shape[0] == 0
    fields = ("full_kv_num", "full_kv_idx", "q_num_blocks", "q_indices", "kv_num_blocks", "kv_indices")
    for f in fields:
        assert getattr(bm, f).shape == getattr(bm_b, f).shape, f
    Q, K, V, dO = make(1, 2, Nn, D, torch.float16, seed=5)
    for grid in (grid_a, grid_b):
        if grid is grid_b:
            for f in fields:
                getattr(bm, f).copy_(getattr(bm_b, f))
        lse = torch.empty(Q.shape[:3], device="cuda", dtype=torch.float32)
        out = run_block_sparse(Q, K, V, bm, D ** -0.5, save_lse=lse)
        dq, dk, dv = run_block_sparse_backward(Q, K, V, out, lse, dO, bm, D ** -0.5)
        torch.cuda.synchronize()
        em = elem_mask(grid, Nn)
        o_ref, rq, rk, rv = O.attention_grads(Q.cpu(), K.cpu(), V.cpu(), dO.cpu(), dtype=torch.float64,
                                              elem_mask=em)
        assert (out.double().cpu() - o_ref).abs().max().item() <= TOL[torch.float16]
        for got, ref in ((dq, rq), (dk, rk), (dv, rv)):
            assert ((got.double().cpu() - ref).norm() / ref.norm()).item() <= GRAD_REL


def test_one_head_per_xcd_group():
    """Sixteen heads of dimension 128 at length 4096 under the BigBird
    fixture mask: one head's K/V (2 MiB) fills an XCD's share of L2, so the
    forward, dQ and dK/dV grids all walk the heads one per XCD at a time
    (two groups of eight).  Every (head, tile) must be visited once (forward
    coverage counters) and every head must match the oracle."""
    from attnfuse.runtime.block_mask import run_block_sparse_backward
    print("[bs] one head per XCD group, 2x8 heads D=128 N=4096", flush=True)
    fx = json.loads((Path(__file__).parent / "golden" / "bigbird_c4_grid.json").read_text())
    n = fx["n_blocks"]
    grid = torch.zeros(n, n, dtype=torch.bool)
    for a, row in enumerate(fx["rows"]):
        grid[a, row] = True
    Nn, Dn, Bn, Hn = 64 * n, 128, 2, 8
    bm = block_mask_from_blocks(grid, 64, 64, device="cuda")
    Q, K, V, dO = make(Bn, Hn, Nn, Dn, torch.float16, seed=6)
    cov = torch.zeros(Bn, Hn, Nn // 32, Nn // 64, dtype=torch.int32, device="cuda")
    lse = torch.empty(Q.shape[:3], device="cuda", dtype=torch.float32)
    out = run_block_sparse(Q, K, V, bm, Dn ** -0.5, save_lse=lse, coverage=cov)
    dq, dk, dv = run_block_sparse_backward(Q, K, V, out, lse, dO, bm, Dn ** -0.5)
    torch.cuda.synchronize()
    exp_cov = O.expected_coverage(Nn, Nn, mask="block_sparse", grid=grid, bm=64, bn=64)
    assert torch.equal(cov.cpu(), exp_cov.expand(Bn, Hn, *exp_cov.shape))
    em = elem_mask(grid, Nn)
    for b in range(Bn):
        for h in range(Hn):
            sl = (slice(b, b + 1), slice(h, h + 1))
            o_ref, rq, rk, rv = O.attention_grads(Q[sl].cpu(), K[sl].cpu(), V[sl].cpu(), dO[sl].cpu(),
                                                  dtype=torch.float32, elem_mask=em)
            assert (out[sl].float().cpu() - o_ref).abs().max().item() <= TOL[torch.float16], (b, h)
            for got, ref in ((dq[sl], rq), (dk[sl], rk), (dv[sl], rv)):
                assert ((got.float().cpu() - ref).norm() / ref.norm()).item() <= GRAD_REL, (b, h)
