"""Backward parity on the GPU against autograd of the CPU oracle.

Gradient error is ||g - g_ref||_F / ||g_ref||_F per tensor, bound 1e-2
(fp16 and bf16); the forward output keeps the forward tolerances.  Covers
the reference's tests/test_backward.py cases (dense / causal / ALiBi, GQA
with group-summed dK/dV) plus what the reference cannot do: fused RoPE,
sliding windows and the causal-window mask.
"""
import pytest
import torch

import attnfuse as af
import oracle as O
from attnfuse.rope_utils import build_rope_cache
from attnfuse.runtime.dispatch import _alibi_slopes

pytestmark = pytest.mark.gpu
FWD_TOL = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}
GRAD_REL = 1e-2


def _fn(name, H, W=48, base=10000.0):
    m = {
        "dense": lambda Q, K, V: af.softmax(af.scaled_dot_product(Q, K)) @ V,
        "causal": lambda Q, K, V: af.softmax(af.causal(af.scaled_dot_product(Q, K))) @ V,
        "causal_alibi": lambda Q, K, V: af.softmax(af.causal(af.alibi(af.scaled_dot_product(Q, K), H))) @ V,
        "alibi": lambda Q, K, V: af.softmax(af.alibi(af.scaled_dot_product(Q, K), H)) @ V,
        "sw": lambda Q, K, V: af.softmax(af.sliding_window(af.scaled_dot_product(Q, K), W)) @ V,
        "sw_causal": lambda Q, K, V: af.softmax(af.causal(af.sliding_window(af.scaled_dot_product(Q, K), W))) @ V,
        "rope_causal": lambda Q, K, V: af.softmax(af.causal(af.rope(Q, K))) @ V,
        "rope_dense": lambda Q, K, V: af.softmax(af.rope(Q, K)) @ V,
        "rope_causal_alibi": lambda Q, K, V: af.softmax(af.causal(af.alibi(af.rope(Q, K), H))) @ V,
        "scaled_causal": lambda Q, K, V: af.softmax(af.causal(af.scaled_dot_product(Q, K, 0.2))) @ V,
    }
    return af.attention(m[name])


def _oracle_kw(name, H, dtype, W=48, rope=None):
    kw = {}
    if "causal" in name:
        kw["causal"] = True
    if name.startswith("sw"):
        kw["window"] = W
    if "alibi" in name:
        kw["alibi_slopes"] = _alibi_slopes(H, "cpu", str(dtype)).float()
    if name.startswith("rope"):
        kw["rope"] = rope
    if name == "scaled_causal":
        kw["scale"] = 0.2
    return kw


def rel(a, b):
    return ((a.float().cpu() - b.float()).norm() / b.float().norm()).item()


def run(name, B, Hq, Hkv, N, D, dtype, base=10000.0, seed=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    Q = torch.randn(B, Hq, N, D, generator=g, device="cuda", dtype=dtype)
    K = torch.randn(B, Hkv, N, D, generator=g, device="cuda", dtype=dtype)
    V = torch.randn(B, Hkv, N, D, generator=g, device="cuda", dtype=dtype)
    dO = torch.randn(B, Hq, N, D, generator=g, device="cuda", dtype=dtype)
    extra, rope = {}, None
    if name.startswith("rope"):
        cos, sin = build_rope_cache(N, D, base=base, device="cuda", dtype=dtype)
        extra = {"cos": cos, "sin": sin}
        rope = (cos[0, 0].cpu(), sin[0, 0].cpu())
    q, k, v = (t.clone().requires_grad_(True) for t in (Q, K, V))
    out = _fn(name, Hq)(q, k, v, **extra)
    assert out.grad_fn is not None
    out.backward(dO)
    torch.cuda.synchronize()
    o_ref, dq, dk, dv = O.attention_grads(Q.cpu(), K.cpu(), V.cpu(), dO.cpu(), dtype=torch.float32,
                                          **_oracle_kw(name, Hq, dtype, rope=rope))
    return {"O": (out.detach().float().cpu() - o_ref).abs().max().item(),
            "dQ": rel(q.grad, dq), "dK": rel(k.grad, dk), "dV": rel(v.grad, dv)}


def check(errs, dtype):
    assert errs["O"] <= FWD_TOL[dtype], errs
    for t in ("dQ", "dK", "dV"):
        assert errs[t] <= GRAD_REL, errs


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("name", ["dense", "causal", "causal_alibi", "alibi", "sw", "sw_causal",
                                  "rope_causal", "rope_dense", "rope_causal_alibi", "scaled_causal"])
def test_backward_variants(name, dtype):
    print(f"[bwd] {name} {dtype}", flush=True)
    check(run(name, 2, 4, 4, 256, 64, dtype), dtype)


@pytest.mark.parametrize("N", [64, 200, 333, 512])
@pytest.mark.parametrize("name", ["dense", "causal", "rope_causal"])
def test_backward_lengths(name, N):
    print(f"[bwd] {name} N={N}", flush=True)
    check(run(name, 1, 4, 4, N, 64, torch.float16, seed=N), torch.float16)


@pytest.mark.parametrize("D", [32, 128])
@pytest.mark.parametrize("name", ["causal", "rope_causal_alibi", "dense"])
def test_backward_head_dims(name, D):
    print(f"[bwd] {name} D={D}", flush=True)
    check(run(name, 1, 4, 4, 192, D, torch.bfloat16), torch.bfloat16)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("name,N", [("dense", 333), ("causal", 700), ("sw", 600), ("sw_causal", 520),
                                    ("rope_causal", 777), ("rope_dense", 256)])
def test_backward_d128_masks_ragged(name, N, dtype):
    """Head dim 128 with GQA 4:1 at ragged lengths, every dense mask: key
    blocks that end past N_kv, waves with no keys, a 48-key window narrower
    than a workgroup's key block."""
    print(f"[bwd] D=128 {name} N={N} {dtype}", flush=True)
    check(run(name, 1, 8, 2, N, 128, dtype), dtype)


@pytest.mark.parametrize("heads", [(8, 2), (8, 1), (12, 4), (32, 8)])
@pytest.mark.parametrize("name", ["causal", "rope_causal"])
def test_backward_gqa_group_sum(name, heads):
    Hq, Hkv = heads
    print(f"[bwd] gqa {name} {heads}", flush=True)
    check(run(name, 1, Hq, Hkv, 256, 64, torch.float16), torch.float16)


def test_backward_llama3_geometry_small():
    """Config-5 geometry (H_q 32, H_kv 8, D 128, RoPE base 5e5, causal, bf16)
    at N=512."""
    check(run("rope_causal", 1, 32, 8, 512, 128, torch.bfloat16, base=500000.0), torch.bfloat16)


def test_backward_deterministic():
    g = torch.Generator(device="cuda").manual_seed(5)
    Q = torch.randn(1, 8, 300, 64, generator=g, device="cuda", dtype=torch.bfloat16)
    K = torch.randn(1, 2, 300, 64, generator=g, device="cuda", dtype=torch.bfloat16)
    V = torch.randn(1, 2, 300, 64, generator=g, device="cuda", dtype=torch.bfloat16)
    dO = torch.randn(1, 8, 300, 64, generator=g, device="cuda", dtype=torch.bfloat16)
    cos, sin = build_rope_cache(300, 64, device="cuda", dtype=torch.bfloat16)
    grads = []
    for _ in range(2):
        q, k, v = (t.clone().requires_grad_(True) for t in (Q, K, V))
        _fn("rope_causal", 8)(q, k, v, cos=cos, sin=sin).backward(dO)
        grads.append((q.grad, k.grad, v.grad))
    torch.cuda.synchronize()
    for a, b in zip(*grads):
        assert torch.equal(a, b)


@pytest.mark.parametrize("Nq,Nkv", [(64, 0), (0, 64), (1, 0)])
def test_backward_with_an_empty_side(Nq, Nkv):
    """No keys: O = 0 and dQ = 0; no queries: dK = dV = 0 (closed forms).
    The tensors are slices of real allocations, so the kernels see valid
    pointers with a zero length."""
    g = torch.Generator(device="cuda").manual_seed(5)
    base = {n: torch.randn(1, 2, 64, 64, generator=g, device="cuda", dtype=torch.float16)
            for n in ("q", "k", "v", "do")}
    q = base["q"][:, :, :Nq].clone().requires_grad_(True)
    k = base["k"][:, :, :Nkv].clone().requires_grad_(True)
    v = base["v"][:, :, :Nkv].clone().requires_grad_(True)
    out = _fn("dense", 2)(q, k, v)
    out.backward(base["do"][:, :, :Nq])
    torch.cuda.synchronize()
    assert out.shape == (1, 2, Nq, 64)
    if Nkv == 0:
        assert torch.count_nonzero(out) == 0
    for t in (q, k, v):
        assert t.grad is not None and t.grad.shape == t.shape
        assert torch.count_nonzero(t.grad) == 0


def test_explicit_alibi_slopes_reach_the_backward():
    """alibi_slopes= on a call that requires grad is used by the forward and
    the backward (config 2's slopes 2^(-8(h+1)/H), which differ from the
    default recipe at H=12)."""
    B, H, N, D = 1, 12, 256, 64
    dtype = torch.float16
    g = torch.Generator(device="cuda").manual_seed(11)
    Q, K, V, dO = (torch.randn(B, H, N, D, generator=g, device="cuda", dtype=dtype) for _ in range(4))
    slopes = torch.tensor([2.0 ** (-8.0 * (h + 1) / H) for h in range(H)])
    q, k, v = (t.clone().requires_grad_(True) for t in (Q, K, V))
    out = _fn("causal_alibi", H)(q, k, v, alibi_slopes=slopes.cuda())
    out.backward(dO)
    torch.cuda.synchronize()
    o_ref, dq, dk, dv = O.attention_grads(Q.cpu(), K.cpu(), V.cpu(), dO.cpu(), dtype=torch.float32,
                                          causal=True, alibi_slopes=slopes)
    check({"O": (out.detach().float().cpu() - o_ref).abs().max().item(),
           "dQ": rel(q.grad, dq), "dK": rel(k.grad, dk), "dV": rel(v.grad, dv)}, dtype)


@pytest.mark.parametrize("split", [1, 2, 4])
def test_backward_group_split_override(split):
    """_BWD_TILE's group split reaches the launch: every split of config 5's
    GQA group of 4 (the library picks 4 at N=512) gives oracle-exact
    gradients."""
    from attentionfuse_amd.runtime import backward as bwd
    print(f"[bwd] group_split={split}", flush=True)
    saved = dict(bwd._BWD_TILE)
    try:
        bwd._BWD_TILE.update({"auto": False, "group_split": split})
        check(run("rope_causal", 1, 8, 2, 512, 128, torch.bfloat16, base=500000.0), torch.bfloat16)
    finally:
        bwd._BWD_TILE.clear()
        bwd._BWD_TILE.update(saved)


@pytest.mark.parametrize("split,N,D", [(2, 1024, 128), (4, 1152, 64), (2, 1000, 64)])
def test_backward_split_heavy_blocks_only(split, N, D):
    """Under a causal mask only the heavy key blocks are split over the
    head group; the last n_kblocks / (2 g_split) run whole groups and store
    dK/dV directly (8, 9 and 8 key blocks: 2, 1 and 2 of them unsplit)."""
    from attentionfuse_amd.runtime import backward as bwd
    print(f"[bwd] heavy-only split={split} N={N} D={D}", flush=True)
    saved = dict(bwd._BWD_TILE)
    try:
        bwd._BWD_TILE.update({"auto": False, "group_split": split})
        check(run("rope_causal", 1, 8, 2, N, D, torch.bfloat16, base=500000.0), torch.bfloat16)
    finally:
        bwd._BWD_TILE.clear()
        bwd._BWD_TILE.update(saved)


@pytest.mark.parametrize("shape", [(2, 4, 1, 384, 64), (1, 8, 2, 640, 128), (1, 4, 4, 200, 64),
                                   (2, 6, 2, 1000, 128)])
def test_causal_block_counts(shape):
    """Causal backward at odd key-block counts, ragged lengths and GQA groups
    under the library's head-group split."""
    B, Hq, Hkv, N, D = shape
    print(f"[bwd] causal blocks {shape}", flush=True)
    check(run("rope_causal", B, Hq, Hkv, N, D, torch.bfloat16), torch.bfloat16)
    check(run("causal", B, Hq, Hkv, N, D, torch.float16), torch.float16)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("name", ["causal", "rope_causal", "rope_causal_alibi", "dense", "alibi", "sw"])
def test_backward_head_dim_256(name, dtype):
    """Head dim 256 with a GQA group of 2 (the ALiBi dK/dV kernels come from
    their own unit, bwd_d256_alt.hip)."""
    print(f"[bwd] D256 {name} {dtype}", flush=True)
    check(run(name, 1, 4, 2, 192, 256, dtype), dtype)
