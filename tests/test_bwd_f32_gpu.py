"""fp32 backward (bwd_f32_kernel.hpp) against autograd of the oracle in fp64.

The reference runs fp32 backward in TF32 with dQ's product cast to bf16 and
tests it at 2e-2 (tests/test_backward.py:30-33,63-106).  Here every product
is fp32, so the bound is ||g - g_ref||_F / ||g_ref||_F <= 1e-4 per gradient
and 3e-5 max-abs on O.  Cases mirror the 16-bit backward tests: every mask,
ALiBi, fused RoPE, ragged lengths, head dims 32/64/128, GQA group sums,
an empty side, and block masks (64/128 blocks, the workgroup walking its
block's K-major or Q-major list).
"""
import pytest
import torch

import oracle as O
from attnfuse.rope_utils import build_rope_cache
from test_bwd_gpu import _fn, _oracle_kw, rel

pytestmark = pytest.mark.gpu
F32 = torch.float32
FWD_TOL = 3e-5
GRAD_REL = 1e-4


def run(name, B, Hq, Hkv, N, D, seed=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    Q, K, V = (torch.randn(B, H, N, D, generator=g, device="cuda", dtype=F32) for H in (Hq, Hkv, Hkv))
    dO = torch.randn(B, Hq, N, D, generator=g, device="cuda", dtype=F32)
    extra, rope = {}, None
    if name.startswith("rope"):
        cos, sin = build_rope_cache(N, D, device="cuda", dtype=F32)
        extra = {"cos": cos, "sin": sin}
        rope = (cos[0, 0].cpu(), sin[0, 0].cpu())
    q, k, v = (t.clone().requires_grad_(True) for t in (Q, K, V))
    out = _fn(name, Hq)(q, k, v, **extra)
    assert out.grad_fn is not None
    out.backward(dO)
    torch.cuda.synchronize()
    o_ref, dq, dk, dv = O.attention_grads(Q.cpu(), K.cpu(), V.cpu(), dO.cpu(), dtype=torch.float64,
                                          **_oracle_kw(name, Hq, F32, rope=rope))
    def err(got, want):
        # one visible key per row (N = 1) makes dS = P (dP - delta) = 0 in
        # closed form: there the bound is absolute
        if want.norm() == 0:
            return (got.double().cpu() - want).abs().max().item()
        return rel(got.double(), want)

    errs = {"O": (out.detach().double().cpu() - o_ref).abs().max().item(),
            "dQ": err(q.grad, dq), "dK": err(k.grad, dk), "dV": err(v.grad, dv)}
    assert errs["O"] <= FWD_TOL, errs
    for t in ("dQ", "dK", "dV"):
        assert errs[t] <= GRAD_REL, errs


@pytest.mark.parametrize("name", ["dense", "causal", "causal_alibi", "alibi", "sw", "sw_causal",
                                  "rope_causal", "rope_dense", "rope_causal_alibi", "scaled_causal"])
def test_backward_variants(name):
    print(f"[bwd f32] {name}", flush=True)
    run(name, 2, 4, 4, 256, 64)


@pytest.mark.parametrize("N", [1, 64, 200, 333])
@pytest.mark.parametrize("name", ["dense", "causal", "rope_causal"])
def test_backward_lengths(name, N):
    print(f"[bwd f32] {name} N={N}", flush=True)
    run(name, 1, 3, 3, N, 64, seed=N)


@pytest.mark.parametrize("D", [32, 128])
@pytest.mark.parametrize("name", ["causal", "rope_causal", "sw"])
def test_backward_head_dims(name, D):
    print(f"[bwd f32] {name} D={D}", flush=True)
    run(name, 1, 2, 2, 160, D)


@pytest.mark.parametrize("name", ["causal", "rope_causal_alibi", "dense"])
def test_backward_gqa_group_sum(name):
    print(f"[bwd f32] {name} GQA 8/2", flush=True)
    run(name, 2, 8, 2, 192, 64)


@pytest.mark.parametrize("D", [32, 128])
@pytest.mark.parametrize("name", ["causal", "rope_causal_alibi"])
def test_backward_gqa_split_head_dims(name, D):
    """GQA group of 4 at D=128 (config 5's ratio) and D=32: the group is
    split over several dK/dV workgroups whose partials the combine kernel
    adds, at every head dim."""
    print(f"[bwd f32] {name} GQA 8/2 D={D}", flush=True)
    run(name, 1, 8, 2, 384, D)


@pytest.mark.parametrize("Nq,Nkv", [(64, 0), (0, 64), (1, 0)])
def test_backward_with_an_empty_side(Nq, Nkv):
    """No keys: O = 0 and dQ = 0; no queries: dK = dV = 0."""
    g = torch.Generator(device="cuda").manual_seed(5)
    base = {n: torch.randn(1, 2, 64, 64, generator=g, device="cuda", dtype=F32) for n in ("q", "k", "v", "do")}
    q = base["q"][:, :, :Nq].clone().requires_grad_(True)
    k = base["k"][:, :, :Nkv].clone().requires_grad_(True)
    v = base["v"][:, :, :Nkv].clone().requires_grad_(True)
    out = _fn("dense", 2)(q, k, v)
    out.backward(base["do"][:, :, :Nq])
    torch.cuda.synchronize()
    assert out.shape == (1, 2, Nq, 64)
    for t in (q, k, v):
        assert t.grad is not None and t.grad.shape == t.shape
        assert torch.count_nonzero(t.grad) == 0


def test_backward_deterministic():
    """The GQA group is split over workgroups whose partial sums are added in
    split order: two runs give bit-identical gradients."""
    g = torch.Generator(device="cuda").manual_seed(11)
    Q = torch.randn(1, 8, 384, 64, generator=g, device="cuda", dtype=F32)
    K, V = (torch.randn(1, 2, 384, 64, generator=g, device="cuda", dtype=F32) for _ in range(2))
    dO = torch.randn(1, 8, 384, 64, generator=g, device="cuda", dtype=F32)
    grads = []
    for _ in range(2):
        q, k, v = (t.clone().requires_grad_(True) for t in (Q, K, V))
        _fn("causal", 8)(q, k, v).backward(dO)
        grads.append((q.grad, k.grad, v.grad))
    torch.cuda.synchronize()
    for a, b in zip(*grads):
        assert torch.equal(a, b)


BS_PATTERNS = {
    "bigbird": lambda q, k: ((q // 64) == 0) | ((k // 64) == 0) | (((q // 64) - (k // 64)).abs() <= 1),
    "strided": lambda q, k: ((q // 64) + (k // 64)) % 2 == 0,
    "local": lambda q, k: ((q // 64) - (k // 64)).abs() <= 1,
}


def run_bs(grid, bmq, bnk, B, Hq, Hkv, N, D, *, rope=False, alibi=False, seed=0):
    from attnfuse.runtime.block_mask import (block_mask_from_blocks, run_block_sparse,
                                             run_block_sparse_backward)
    g = torch.Generator(device="cuda").manual_seed(seed)
    Q, dO = (torch.randn(B, Hq, N, D, generator=g, device="cuda", dtype=F32) for _ in range(2))
    K, V = (torch.randn(B, Hkv, N, D, generator=g, device="cuda", dtype=F32) for _ in range(2))
    kw, okw = {}, {}
    if rope:
        cos, sin = build_rope_cache(N, D, device="cuda", dtype=F32)
        kw.update(cos=cos, sin=sin)
        okw["rope"] = (cos[0, 0].cpu(), sin[0, 0].cpu())
    if alibi:
        slopes = torch.tensor(O.alibi_slopes(Hq), dtype=F32, device="cuda")
        kw["alibi_slopes"] = slopes
        okw["alibi_slopes"] = slopes.cpu().double()
    bm = block_mask_from_blocks(grid, bmq, bnk, device="cuda")
    lse = torch.empty(B, Hq, N, device="cuda", dtype=F32)
    bias = 1 if alibi else 0
    out = run_block_sparse(Q, K, V, bm, D ** -0.5, bias_kind=bias, save_lse=lse, **kw)
    dq, dk, dv = run_block_sparse_backward(Q, K, V, out, lse, dO, bm, D ** -0.5, bias_kind=bias, **kw)
    torch.cuda.synchronize()
    em = O.element_mask_from_grid(grid, N, N, bmq, bnk)
    o_ref, rq, rk, rv = O.attention_grads(Q.cpu(), K.cpu(), V.cpu(), dO.cpu(), dtype=torch.float64, elem_mask=em,
                                          **okw)
    errs = {"O": (out.double().cpu() - o_ref).abs().max().item(),
            "dQ": rel(dq.double(), rq), "dK": rel(dk.double(), rk), "dV": rel(dv.double(), rv)}
    assert errs["O"] <= FWD_TOL, errs
    for t in ("dQ", "dK", "dV"):
        assert errs[t] <= GRAD_REL, errs


@pytest.mark.parametrize("blocks", [(64, 64), (128, 64), (64, 128), (128, 128)])
@pytest.mark.parametrize("name", sorted(BS_PATTERNS))
def test_block_sparse_backward(name, blocks):
    """fp32 gradients with a BlockMask: dK/dV workgroups of block_n / 32
    waves walk their key block's K-major list, dQ workgroups their query
    block's Q-major lists."""
    print(f"[bwd f32] block-sparse {name} {blocks}", flush=True)
    bmq, bnk = blocks
    N = 384
    grid = O.block_grid(BS_PATTERNS[name], N, N, bmq, bnk)
    run_bs(grid, bmq, bnk, 2, 4, 4, N, 64, seed=21)


@pytest.mark.parametrize("split", [0, 2])
def test_block_sparse_backward_gqa_rope_alibi(split, monkeypatch):
    """GQA (4 query heads on 2 KV heads) with RoPE and ALiBi and a block
    row with no block at all, under the library's and an explicit group
    split; head dims 32 and 128."""
    from attentionfuse_amd.runtime import backward as bwd
    monkeypatch.setitem(bwd._BWD_TILE, "auto", split == 0)
    monkeypatch.setitem(bwd._BWD_TILE, "group_split", split)
    for D in (32, 128):
        print(f"[bwd f32] block-sparse gqa split={split} D={D}", flush=True)
        N = 320
        grid = O.block_grid(BS_PATTERNS["bigbird"], N, N, 64, 64)
        grid[3, :] = False
        run_bs(grid, 64, 64, 1, 4, 2, N, D, rope=True, alibi=True, seed=22)
