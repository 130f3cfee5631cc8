"""Parity at the exact launch geometries bench.py times.

The bench lines time launches whose geometry depends on the full sizes: the
forward's grid and ALiBi offsets at N=4096 with 12 heads, the backward's
GQA head-group split at N=4096 (g_split 2, where N=512 gives 4), and the
decode split count at B=8 (8 splits x 64 groups, where B=1 gets 64 splits).
Each is run once here at that size and compared with the fp32 oracle:
max-abs 2e-3 (fp16) / 1.6e-2 (bf16) on outputs, ||g - g_ref||_F / ||g_ref||_F
<= 1e-2 per gradient.  The oracle runs on a sample where the full problem
would take minutes on the CPU (named in each test).
"""
import pytest
import torch

import attnfuse as af
import bench
import oracle as O
from attnfuse.rope_utils import build_rope_cache
from attentionfuse_amd.runtime import _native as native
from attentionfuse_amd.runtime.backward import run_backward
from attentionfuse_amd.runtime.prepared import prepare_attention, prepare_decode

pytestmark = pytest.mark.gpu
TOL = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}
GRAD_REL = 1e-2


def _rel(a, b):
    return ((a.float().cpu() - b.float()).norm() / b.float().norm()).item()


def test_config2_as_written_alibi_all_heads():
    """Causal + RoPE + ALiBi, fp16, B=4 H=12 N=4096 D=64, slopes 2^(-8(h+1)/H):
    every one of the 48 heads against the oracle."""
    B, H, N, D = (bench.C2[k] for k in ("B", "H", "N", "D"))
    print(f"[bench-launch] config 2 alibi B={B} H={H} N={N}", flush=True)
    _, (Q, K, V, cos, sin, out) = bench.bench_forward(1, 0, alibi=True)
    torch.cuda.synchronize()
    slopes = torch.tensor([2.0 ** (-8.0 * (h + 1) / H) for h in range(H)])
    rope = (cos[0, 0].cpu(), sin[0, 0].cpu())
    err = 0.0
    for b in range(B):
        for h in range(H):
            want = O.naive_attention(Q[b:b + 1, h:h + 1].cpu(), K[b:b + 1, h:h + 1].cpu(),
                                     V[b:b + 1, h:h + 1].cpu(), causal=True, rope=rope,
                                     alibi_slopes=slopes[h:h + 1])
            err = max(err, (out[b:b + 1, h:h + 1].float().cpu() - want).abs().max().item())
    print(f"[bench-launch] config 2 alibi max|err|={err:.3e}", flush=True)
    assert err <= TOL[torch.float16]


def test_config5_train_step_full_length():
    """Config 5 (causal GQA + RoPE base 5e5, bf16, B=1 N=4096 Hq=32 Hkv=8
    D=128) forward + backward at full length, the bench's g_split; oracle
    autograd (fp32) on KV heads 0 and 7 with their 4 query heads each."""
    B, Hq, Hkv, N, D = (bench.C5[k] for k in ("B", "Hq", "Hkv", "N", "D"))
    dt = torch.bfloat16
    print(f"[bench-launch] config 5 N={N}", flush=True)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    Q = torch.randn(B, Hq, N, D, generator=g, device=dev, dtype=dt)
    K = torch.randn(B, Hkv, N, D, generator=g, device=dev, dtype=dt)
    V = torch.randn(B, Hkv, N, D, generator=g, device=dev, dtype=dt)
    dO = torch.randn(B, Hq, N, D, generator=g, device=dev, dtype=dt)
    cos, sin = build_rope_cache(N, D, base=500000.0, device=dev, dtype=dt)
    fn = af.attention(lambda Q, K, V: af.softmax(af.causal(af.rope(Q, K))) @ V)
    graph = fn(Q, K, V, return_graph=True)
    L = torch.empty(B, Hq, N, dtype=torch.float32, device=dev)
    fwd, out = prepare_attention(graph, Q, K, V, cos=cos, sin=sin, save_lse=L)
    fwd()
    dQ, dK, dV = run_backward(graph, Q, K, V, out, L, dO, D ** -0.5, cos=cos, sin=sin)
    torch.cuda.synchronize()
    G = Hq // Hkv
    rope = (cos[0, 0].cpu(), sin[0, 0].cpu())
    for hk in (0, Hkv - 1):
        qs = slice(G * hk, G * (hk + 1))
        ks = slice(hk, hk + 1)
        o_ref, dq_ref, dk_ref, dv_ref = O.attention_grads(
            Q[:, qs].cpu(), K[:, ks].cpu(), V[:, ks].cpu(), dO[:, qs].cpu(),
            dtype=torch.float32, causal=True, rope=rope)
        err = (out[:, qs].float().cpu() - o_ref).abs().max().item()
        rels = (_rel(dQ[:, qs], dq_ref), _rel(dK[:, ks], dk_ref), _rel(dV[:, ks], dv_ref))
        print(f"[bench-launch] config 5 kv head {hk}: O {err:.3e} dQ/dK/dV {rels}", flush=True)
        assert err <= TOL[dt]
        assert max(rels) <= GRAD_REL


def test_config3_decode_batch8_default_splits():
    """Config 3 (GQA decode bf16, B=8 Hq=32 Hkv=8 D=128, cache 32768) with
    the library's default split count; oracle on batches 0, 3 and 7 (all 32
    query heads each)."""
    B, Hq, Hkv, N, D = (bench.C3[k] for k in ("B", "Hq", "Hkv", "N", "D"))
    S = int(native.lib().af_decode_num_splits(B, Hq, Hkv, N, D))
    print(f"[bench-launch] config 3 B={B} splits={S}", flush=True)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    Q = torch.randn(B, Hq, 1, D, generator=g, device=dev, dtype=torch.bfloat16)
    K = torch.randn(B, Hkv, N, D, generator=g, device=dev, dtype=torch.bfloat16)
    V = torch.randn(B, Hkv, N, D, generator=g, device=dev, dtype=torch.bfloat16)
    dense = af.attention(lambda Q, K, V: af.softmax(af.scaled_dot_product(Q, K)) @ V)
    launch, out = prepare_decode(dense(Q, K, V, return_graph=True), Q, K, V)
    launch()
    torch.cuda.synchronize()
    err = 0.0
    for b in (0, 3, B - 1):
        want = O.naive_attention(Q[b:b + 1].cpu(), K[b:b + 1].cpu(), V[b:b + 1].cpu())
        err = max(err, (out[b:b + 1].float().cpu() - want).abs().max().item())
    print(f"[bench-launch] config 3 max|err|={err:.3e}", flush=True)
    assert err <= TOL[torch.bfloat16]
