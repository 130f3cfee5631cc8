"""Prepared launches captured in a HIP graph (torch.cuda.CUDAGraph) give the
same bytes as eager launches on every replay.

The kernels allocate nothing, take caller-owned workspaces and record no
memset, so a serving loop can capture a decode step or a prefill once and
replay it.  Each graph is replayed several times with other eager work and
synchronisations in between, and every replay is compared with the eager
result of the same launch."""
import pytest
import torch

import attnfuse as af
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


def _replays_match(graph, out, want, scratch):
    for i in range(4):
        out.zero_()
        scratch.mul_(1.5).add_(float(i))   # unrelated eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {i} differs from the eager launch"


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
    graph = _capture(launch)
    _replays_match(graph, out, want, torch.ones(1 << 16, device="cuda"))


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
    graph = _capture(launch)
    _replays_match(graph, out, want, torch.ones(1 << 16, device="cuda"))
