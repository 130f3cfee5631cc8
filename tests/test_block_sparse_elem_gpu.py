"""Block-sparse walks with element masks inside partial tiles
(create_block_mask(..., exact=True)): forward O and LSE, dQ/dK/dV, in fp16,
bf16 and fp32, against the oracle on the element predicate itself (not its
block-rounded upper bound), with split work plans, 32/64/128 blocks, RoPE +
ALiBi and GQA.  A causal predicate through the block-sparse kernels is also
checked against the dense causal kernel."""
import pytest
import torch

import attnfuse as af
import oracle as O
from attnfuse.rope_utils import build_rope_cache
from attentionfuse_amd.runtime.block_mask import run_block_sparse, run_block_sparse_backward

pytestmark = pytest.mark.gpu
TOL = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2, torch.float32: 3e-5}
LSE_TOL = {torch.float16: 5e-3, torch.bfloat16: 3e-2, torch.float32: 1e-4}
GRAD_REL = {torch.float16: 1e-2, torch.bfloat16: 1e-2, torch.float32: 1e-4}
IDS = {torch.float16: "f16", torch.bfloat16: "bf16", torch.float32: "f32"}

PREDS = {
    "causal": lambda q, k: k <= q,
    "window": lambda q, k: (q - k).abs() < 70,
    # an irregular pattern that also leaves query rows 40..47 with no key
    "pattern": lambda q, k: ((q * 7 + k * 13) % 5 != 0) & ((q - k).abs() < 150) & ((q < 40) | (q >= 48)),
}


def elem_mask(pred, nq, nk):
    qi = torch.arange(nq)[:, None].expand(nq, nk)
    kj = torch.arange(nk)[None, :].expand(nq, nk)
    return torch.as_tensor(pred(qi, kj), dtype=torch.bool).expand(nq, nk)


def rand(shape, dtype, g):
    return torch.randn(*shape, generator=g, device="cuda", dtype=dtype)


def grads_ok(got3, ref3, dtype):
    for got, ref in zip(got3, ref3):
        assert ((got.double().cpu() - ref).norm() / ref.norm()).item() <= GRAD_REL[dtype]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32], ids=lambda d: IDS[d])
@pytest.mark.parametrize("name", sorted(PREDS))
def test_elem_forward(name, dtype):
    print(f"[bs-elem] fwd {name} {IDS[dtype]}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(3)
    N, D = 448, 64
    Q, K, V = (rand((2, 3, N, D), dtype, g) for _ in range(3))
    bm = af.create_block_mask(PREDS[name], N, N, 64, 64, device="cuda", exact=True)
    assert int(bm.kv_num_blocks.sum()) > 0
    lse = torch.empty(Q.shape[:3], device="cuda", dtype=torch.float32)
    out = run_block_sparse(Q, K, V, bm, D ** -0.5, save_lse=lse)
    torch.cuda.synchronize()
    em = elem_mask(PREDS[name], N, N)
    want, want_l = O.naive_attention(Q.cpu(), K.cpu(), V.cpu(), elem_mask=em, return_lse=True)
    assert (out.float().cpu() - want).abs().max().item() <= TOL[dtype]
    fin = torch.isfinite(want_l)
    assert torch.equal(torch.isfinite(lse.cpu()), fin)
    assert (lse.cpu()[fin] - want_l[fin]).abs().max().item() <= LSE_TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=lambda d: IDS[d])
@pytest.mark.parametrize("blocks", [(32, 64), (128, 64), (64, 128), (128, 128)])
def test_elem_forward_block_sizes(blocks, dtype):
    print(f"[bs-elem] fwd blocks {blocks} {IDS[dtype]}", flush=True)
    bmq, bnk = blocks
    g = torch.Generator(device="cuda").manual_seed(5)
    Nq, Nk, D = 400, 333, 64
    Q = rand((1, 2, Nq, D), dtype, g)
    K, V = (rand((1, 2, Nk, D), dtype, g) for _ in range(2))
    pred = PREDS["pattern"]
    bm = af.create_block_mask(pred, Nq, Nk, bmq, bnk, device="cuda", exact=True)
    out = run_block_sparse(Q, K, V, bm, D ** -0.5)
    torch.cuda.synchronize()
    want = O.naive_attention(Q.cpu(), K.cpu(), V.cpu(), elem_mask=elem_mask(pred, Nq, Nk))
    assert (out.float().cpu() - want).abs().max().item() <= TOL[dtype]


@pytest.mark.parametrize("chunk", [0, 1])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32], ids=lambda d: IDS[d])
@pytest.mark.parametrize("name", sorted(PREDS))
def test_elem_backward(name, dtype, chunk):
    print(f"[bs-elem] bwd {name} {IDS[dtype]} chunk={chunk}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(11)
    N, D = 384, 64
    Q, K, V, dO = (rand((2, 2, N, D), dtype, g) for _ in range(4))
    bm = af.create_block_mask(PREDS[name], N, N, 64, 64, device="cuda", exact=True)
    if chunk:
        bm.plan_work(chunk)
    lse = torch.empty(Q.shape[:3], device="cuda", dtype=torch.float32)
    out = run_block_sparse(Q, K, V, bm, D ** -0.5, save_lse=lse)
    dq, dk, dv = run_block_sparse_backward(Q, K, V, out, lse, dO, bm, D ** -0.5)
    torch.cuda.synchronize()
    o_ref, rq, rk, rv = O.attention_grads(Q.cpu(), K.cpu(), V.cpu(), dO.cpu(), dtype=torch.float64,
                                          elem_mask=elem_mask(PREDS[name], N, N))
    assert (out.double().cpu() - o_ref).abs().max().item() <= TOL[dtype]
    grads_ok((dq, dk, dv), (rq, rk, rv), dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=lambda d: IDS[d])
@pytest.mark.parametrize("blocks", [(128, 64), (64, 128), (128, 128)])
def test_elem_backward_block_sizes(blocks, dtype):
    print(f"[bs-elem] bwd blocks {blocks} {IDS[dtype]}", flush=True)
    bmq, bnk = blocks
    g = torch.Generator(device="cuda").manual_seed(13)
    N, D = 512, 64
    Q, K, V, dO = (rand((1, 2, N, D), dtype, g) for _ in range(4))
    pred = PREDS["window"]
    bm = af.create_block_mask(pred, N, N, bmq, bnk, device="cuda", exact=True)
    lse = torch.empty(Q.shape[:3], device="cuda", dtype=torch.float32)
    out = run_block_sparse(Q, K, V, bm, D ** -0.5, save_lse=lse)
    dq, dk, dv = run_block_sparse_backward(Q, K, V, out, lse, dO, bm, D ** -0.5)
    torch.cuda.synchronize()
    o_ref, rq, rk, rv = O.attention_grads(Q.cpu(), K.cpu(), V.cpu(), dO.cpu(), dtype=torch.float64,
                                          elem_mask=elem_mask(pred, N, N))
    assert (out.double().cpu() - o_ref).abs().max().item() <= TOL[dtype]
    grads_ok((dq, dk, dv), (rq, rk, rv), dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32], ids=lambda d: IDS[d])
def test_elem_gqa_rope_alibi(dtype):
    """Hq = 4 over Hkv = 2, fused RoPE and ALiBi, split plan."""
    print(f"[bs-elem] gqa rope alibi {IDS[dtype]}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(17)
    N, D = 320, 64
    Q, dO = (rand((1, 4, N, D), dtype, g) for _ in range(2))
    K, V = (rand((1, 2, N, D), dtype, g) for _ in range(2))
    cos, sin = build_rope_cache(N, D, device="cuda", dtype=dtype)
    slopes = torch.tensor(O.alibi_slopes(4), dtype=torch.float32, device="cuda")
    pred = PREDS["pattern"]
    bm = af.create_block_mask(pred, N, N, 64, 64, device="cuda", exact=True)
    bm.plan_work(1)
    lse = torch.empty(Q.shape[:3], device="cuda", dtype=torch.float32)
    kw = dict(bias_kind=1, cos=cos, sin=sin, alibi_slopes=slopes)
    out = run_block_sparse(Q, K, V, bm, D ** -0.5, save_lse=lse, **kw)
    dq, dk, dv = run_block_sparse_backward(Q, K, V, out, lse, dO, bm, D ** -0.5, **kw)
    torch.cuda.synchronize()
    o_ref, rq, rk, rv = O.attention_grads(Q.cpu(), K.cpu(), V.cpu(), dO.cpu(), dtype=torch.float64,
                                          elem_mask=elem_mask(pred, N, N), alibi_slopes=slopes.cpu(),
                                          rope=(cos[0, 0].cpu(), sin[0, 0].cpu()))
    assert (out.double().cpu() - o_ref).abs().max().item() <= TOL[dtype]
    grads_ok((dq, dk, dv), (rq, rk, rv), dtype)


def test_elem_causal_matches_dense_causal_kernel():
    """The causal predicate through the block-sparse walk (partial diagonal
    tiles) against the dense causal kernel on the same inputs."""
    print("[bs-elem] causal vs dense causal", flush=True)
    g = torch.Generator(device="cuda").manual_seed(19)
    N, D = 512, 64
    Q, K, V = (rand((2, 4, N, D), torch.float16, g) for _ in range(3))
    bm = af.create_block_mask(PREDS["causal"], N, N, 64, 64, device="cuda", exact=True)
    got = run_block_sparse(Q, K, V, bm, D ** -0.5)
    fn = af.attention(lambda Q, K, V: af.softmax(af.causal(af.scaled_dot_product(Q, K))) @ V)
    want = fn(Q, K, V)
    torch.cuda.synchronize()
    assert (got.float() - want.float()).abs().max().item() <= 1e-3


@pytest.mark.parametrize("name", ["causal", "mixed"])
def test_elem_walks_longer_than_64_tiles(name):
    """Lists of 72 entries (no plan split): tiles from 64 on are looked up in
    the lists rather than the per-lane table, partial-tile flags included
    (causal: the Q-major diagonal entry comes last; mixed: every tile is
    partial, so the K-major flags are read for entries past 64)."""
    print(f"[bs-elem] long walks {name}", flush=True)
    n, D, dtype = 72, 64, torch.float16
    N = 64 * n
    pred = PREDS["causal"] if name == "causal" else (lambda q, k: (q + k) % 3 != 0)
    g = torch.Generator(device="cuda").manual_seed(23)
    Q, K, V, dO = (rand((1, 1, N, D), dtype, g) for _ in range(4))
    bm = af.create_block_mask(pred, N, N, 64, 64, device="cuda", exact=True)
    assert int(bm.full_kv_num.max() + bm.kv_num_blocks.max()) >= 64
    assert bm.plan.q_splits.shape[0] == 0 and bm.plan.kv_splits.shape[0] == 0
    lse = torch.empty(Q.shape[:3], device="cuda", dtype=torch.float32)
    out = run_block_sparse(Q, K, V, bm, D ** -0.5, save_lse=lse)
    dq, dk, dv = run_block_sparse_backward(Q, K, V, out, lse, dO, bm, D ** -0.5)
    torch.cuda.synchronize()
    o_ref, rq, rk, rv = O.attention_grads(Q.cpu(), K.cpu(), V.cpu(), dO.cpu(), dtype=torch.float32,
                                          elem_mask=elem_mask(pred, N, N))
    assert (out.float().cpu() - o_ref).abs().max().item() <= TOL[dtype]
    grads_ok((dq, dk, dv), (rq, rk, rv), dtype)
