"""Prepared launches, eager and captured in a HIP graph (torch.cuda.CUDAGraph),
against the fp32 CPU oracle.

The kernels allocate nothing, take caller-owned workspaces and record no
memset, so a serving loop can capture a decode step or a prefill once and
replay it.  Each graph is replayed several times with other eager work and
synchronisations in between; every replay must equal the eager launch bit for
bit and the oracle within the forward tolerances (2e-3 fp16, 1.6e-2 bf16).
New input values written into the captured storage between replays must
give the oracle's answer for the new values."""
import pytest
import torch

import attnfuse as af
import oracle as O
from attnfuse.rope_utils import build_rope_cache
from attentionfuse_amd.runtime.prepared import prepare_attention, prepare_decode

pytestmark = pytest.mark.gpu


def _capture(launch):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        launch()                       # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch()
    torch.cuda.synchronize()
    return graph


def _replays_match(graph, out, want, scratch, oracle_out, tol):
    for i in range(4):
        out.zero_()
        scratch.mul_(1.5).add_(float(i))   # unrelated eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {i} differs from the eager launch"
        err = (out.float().cpu() - oracle_out).abs().max().item()
        assert err <= tol, f"replay {i}: max|err| vs oracle {err:.3e}"


@pytest.mark.parametrize("rope", [False, True], ids=["plain", "rope"])
def test_forward_graph_replays_match_eager(rope):
    B, H, N, D = 2, 4, 384, 64
    print(f"[graph fwd] rope={rope}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(3)
    Q, K, V = (torch.randn(B, H, N, D, generator=g, device="cuda", dtype=torch.float16) for _ in range(3))
    cos, sin = build_rope_cache(N, D, device="cuda", dtype=torch.float16)
    if rope:
        fn = af.attention(lambda Q, K, V: af.softmax(af.causal(af.rope(Q, K))) @ V)
    else:
        fn = af.attention(lambda Q, K, V: af.softmax(af.causal(af.scaled_dot_product(Q, K))) @ V)
    launch, out = prepare_attention(fn(Q, K, V, return_graph=True), Q, K, V, cos=cos, sin=sin)
    launch()
    torch.cuda.synchronize()
    want = out.clone()
    rope_t = (cos[0, 0].cpu(), sin[0, 0].cpu()) if rope else None
    ref = O.naive_attention(Q.cpu(), K.cpu(), V.cpu(), causal=True, rope=rope_t)
    assert (want.float().cpu() - ref).abs().max().item() <= 2e-3
    graph = _capture(launch)
    _replays_match(graph, out, want, torch.ones(1 << 16, device="cuda"), ref, 2e-3)
    # new values in the captured storage: the replay computes on them
    g2 = torch.Generator(device="cuda").manual_seed(4)
    for t in (Q, K, V):
        t.copy_(torch.randn(t.shape, generator=g2, device="cuda", dtype=t.dtype))
    graph.replay()
    torch.cuda.synchronize()
    ref2 = O.naive_attention(Q.cpu(), K.cpu(), V.cpu(), causal=True, rope=rope_t)
    assert (out.float().cpu() - ref2).abs().max().item() <= 2e-3


def test_decode_graph_replays_match_eager():
    B, Hq, Hkv, N, D = 2, 32, 8, 5000, 128
    print("[graph decode]", flush=True)
    g = torch.Generator(device="cuda").manual_seed(5)
    Q = torch.randn(B, Hq, 1, D, generator=g, device="cuda", dtype=torch.bfloat16)
    K = torch.randn(B, Hkv, N, D, generator=g, device="cuda", dtype=torch.bfloat16)
    V = torch.randn(B, Hkv, N, D, generator=g, device="cuda", dtype=torch.bfloat16)
    dense = af.attention(lambda Q, K, V: af.softmax(af.scaled_dot_product(Q, K)) @ V)
    launch, out = prepare_decode(dense(Q, K, V, return_graph=True), Q, K, V)
    launch()
    torch.cuda.synchronize()
    want = out.clone()
    ref = O.naive_attention(Q.cpu(), K.cpu(), V.cpu())
    assert (want.float().cpu() - ref).abs().max().item() <= 1.6e-2
    graph = _capture(launch)
    _replays_match(graph, out, want, torch.ones(1 << 16, device="cuda"), ref, 1.6e-2)
    # a new query token in the captured storage
    Q.copy_(torch.randn(Q.shape, generator=g, device="cuda", dtype=Q.dtype))
    graph.replay()
    torch.cuda.synchronize()
    ref2 = O.naive_attention(Q.cpu(), K.cpu(), V.cpu())
    assert (out.float().cpu() - ref2).abs().max().item() <= 1.6e-2


@pytest.mark.parametrize("kind", ["gqa_rope", "block_sparse"])
def test_training_step_graph_replays_match_eager(kind):
    """A whole training step -- forward (saving L) and backward, RoPE + GQA
    with the head-group split, or a block-sparse walk with a split plan --
    captured once: every replay equals the eager step bit for bit, and the
    gradients match the oracle."""
    from attentionfuse_amd.runtime.backward import run_backward
    from attentionfuse_amd.runtime.block_mask import (block_mask_from_blocks, run_block_sparse,
                                                      run_block_sparse_backward)
    print(f"[graph train] {kind}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(6)
    dtype = torch.bfloat16
    if kind == "gqa_rope":
        B, Hq, Hkv, N, D = 1, 8, 2, 1024, 128
    else:
        B, Hq, Hkv, N, D = 1, 2, 2, 1024, 64
    Q = torch.randn(B, Hq, N, D, generator=g, device="cuda", dtype=dtype)
    K, V = (torch.randn(B, Hkv, N, D, generator=g, device="cuda", dtype=dtype) for _ in range(2))
    dO = torch.randn(B, Hq, N, D, generator=g, device="cuda", dtype=dtype)
    L = torch.empty(B, Hq, N, dtype=torch.float32, device="cuda")
    res = {}
    if kind == "gqa_rope":
        cos, sin = build_rope_cache(N, D, base=500000.0, device="cuda", dtype=dtype)
        graph_ir = af.attention(lambda Q, K, V: af.softmax(af.causal(af.rope(Q, K))) @ V)(
            Q, K, V, return_graph=True)
        fwd, out = prepare_attention(graph_ir, Q, K, V, cos=cos, sin=sin, save_lse=L)

        def step():
            fwd()
            res["g"] = run_backward(graph_ir, Q, K, V, out, L, dO, D ** -0.5, cos=cos, sin=sin)
        kw = {"causal": True, "rope": (cos[0, 0].cpu(), sin[0, 0].cpu())}
    else:
        n = N // 64
        grid = torch.zeros(n, n, dtype=torch.bool)
        grid[0, :] = grid[:, 0] = True
        for i in range(n):
            grid[i, max(i - 1, 0): i + 2] = True
        bm = block_mask_from_blocks(grid, 64, 64, device="cuda")
        bm.plan_work(2)
        out = torch.empty_like(Q)

        def step():
            run_block_sparse(Q, K, V, bm, D ** -0.5, out=out, save_lse=L)
            res["g"] = run_block_sparse_backward(Q, K, V, out, L, dO, bm, D ** -0.5)
        kw = {"elem_mask": O.element_mask_from_grid(grid, N, N, 64, 64)}
    step()
    torch.cuda.synchronize()
    want = [t.clone() for t in (out, *res["g"])]
    graph = _capture(step)
    got = (out, *res["g"])                 # the graph's own output tensors
    scratch = torch.ones(1 << 16, device="cuda")
    for i in range(3):
        for t in got:
            t.zero_()
        scratch.mul_(1.5).add_(float(i))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(got, want):
            assert torch.equal(a, b), f"replay {i} differs from the eager step"
    o_ref, rq, rk, rv = O.attention_grads(Q.cpu(), K.cpu(), V.cpu(), dO.cpu(), dtype=torch.float32, **kw)
    assert (got[0].float().cpu() - o_ref).abs().max().item() <= 1.6e-2
    for t, r in zip(got[1:], (rq, rk, rv)):
        assert ((t.float().cpu() - r).norm() / r.norm()).item() <= 1e-2
