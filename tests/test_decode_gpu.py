"""Flash-decoding parity on the GPU (split-K + log-sum-exp combine) against
the fp32 CPU oracle, including ragged split boundaries (the reference
double-counts keys there) and the split-count invariance of the combine."""
import pytest
import torch

import attnfuse as af
import oracle as O
from attnfuse.runtime.dispatch import _alibi_slopes
from attnfuse.runtime.flash_decode import run_flash_decode

pytestmark = pytest.mark.gpu
TOL = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}


@af.attention
def dense(Q, K, V):
    return af.softmax(af.scaled_dot_product(Q, K)) @ V


def make(B, Hq, Hkv, N, D, dtype, seed=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    Q = torch.randn(B, Hq, 1, D, generator=g, device="cuda", dtype=dtype)
    K = torch.randn(B, Hkv, N, D, generator=g, device="cuda", dtype=dtype)
    V = torch.randn(B, Hkv, N, D, generator=g, device="cuda", dtype=dtype)
    return Q, K, V


def alibi_fn(H):
    return af.attention(lambda Q, K, V: af.softmax(af.alibi(af.scaled_dot_product(Q, K), H)) @ V)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("shape", [(2, 8, 2, 4096, 128), (1, 32, 8, 2048, 128), (2, 4, 4, 1000, 64),
                                   (1, 16, 1, 3000, 64), (1, 32, 1, 777, 128), (3, 6, 3, 513, 32),
                                   (2, 8, 4, 3000, 256), (1, 16, 8, 8192, 256)])
def test_decode_matches_oracle(shape, dtype):
    B, Hq, Hkv, N, D = shape
    print(f"[decode] {shape} {dtype}", flush=True)
    Q, K, V = make(B, Hq, Hkv, N, D, dtype)
    out = dense(Q, K, V)
    torch.cuda.synchronize()
    want = O.naive_attention(Q.cpu(), K.cpu(), V.cpu())
    err = (out.float().cpu() - want).abs().max().item()
    assert err <= TOL[dtype], f"max|err|={err:.3e}"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
def test_decode_alibi_uses_last_position(dtype):
    B, Hq, Hkv, N, D = 2, 8, 2, 2500, 128
    Q, K, V = make(B, Hq, Hkv, N, D, dtype, seed=4)
    out = alibi_fn(Hq)(Q, K, V)
    torch.cuda.synchronize()
    sl = _alibi_slopes(Hq, "cpu", str(dtype)).float()
    want = O.naive_attention(Q.cpu(), K.cpu(), V.cpu(), alibi_slopes=sl, query_offset=N - 1)
    assert (out.float().cpu() - want).abs().max().item() <= TOL[dtype]


@pytest.mark.parametrize("splits", [1, 2, 3, 7, 16, 40])
def test_ragged_splits_count_every_key_once(splits):
    B, Hq, Hkv, N, D = 2, 8, 2, 3001, 128
    Q, K, V = make(B, Hq, Hkv, N, D, torch.float16, seed=splits)
    g = dense(Q, K, V, return_graph=True)
    out = torch.empty_like(Q)
    run_flash_decode(g, Q, K, V, D ** -0.5, 0, Hkv, out, num_splits=splits)
    torch.cuda.synchronize()
    want = O.naive_attention(Q.cpu(), K.cpu(), V.cpu())
    assert (out.float().cpu() - want).abs().max().item() <= TOL[torch.float16]


def test_decode_deterministic_and_split_invariant():
    Q, K, V = make(2, 8, 2, 4096, 128, torch.bfloat16, seed=9)
    g = dense(Q, K, V, return_graph=True)
    outs = []
    for s in (4, 4, 13):
        o = torch.empty_like(Q)
        run_flash_decode(g, Q, K, V, 128 ** -0.5, 0, 2, o, num_splits=s)
        outs.append(o)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    assert (outs[0].float() - outs[2].float()).abs().max().item() <= TOL[torch.bfloat16]


def test_llama3_8b_geometry_small_batch():
    """Config-3 geometry (H_q 32, H_kv 8, D 128, cache 32768) at B=1."""
    Q, K, V = make(1, 32, 8, 32768, 128, torch.bfloat16, seed=1)
    out = dense(Q, K, V)
    torch.cuda.synchronize()
    want = O.naive_attention(Q.cpu(), K.cpu(), V.cpu())
    assert (out.float().cpu() - want).abs().max().item() <= TOL[torch.bfloat16]


def test_concurrent_decodes_on_two_streams():
    """Two decode calls in flight at once on two streams, each with its own
    split partials (the Python route allocates them per call from the
    stream's allocator pool); both match the oracle."""
    a = make(4, 32, 8, 16384, 128, torch.bfloat16, seed=21)
    b = make(2, 8, 2, 9000, 64, torch.float16, seed=22)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    for s in (s1, s2):
        s.wait_stream(torch.cuda.current_stream())
    outs = {}
    for _ in range(3):
        with torch.cuda.stream(s1):
            outs["a"] = dense(*a)
        with torch.cuda.stream(s2):
            outs["b"] = dense(*b)
    for s in (s1, s2):
        torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for name, (Q, K, V), dt in (("a", a, torch.bfloat16), ("b", b, torch.float16)):
        want = O.naive_attention(Q.cpu(), K.cpu(), V.cpu())
        err = (outs[name].float().cpu() - want).abs().max().item()
        assert err <= TOL[dt], (name, err)


@pytest.mark.parametrize("alibi", [False, True], ids=["plain", "alibi"])
def test_decode_long_cache(alibi):
    """A 262144-key cache (1 GiB of K/V, 64 splits of 4096 keys): every key
    counted once, against the oracle; with ALiBi the query sits at N - 1."""
    B, Hq, Hkv, N, D = 1, 32, 8, 262144, 128
    print(f"[decode] long cache N={N} alibi={alibi}", flush=True)
    Q, K, V = make(B, Hq, Hkv, N, D, torch.bfloat16, seed=9)
    out = (alibi_fn(Hq) if alibi else dense)(Q, K, V)
    torch.cuda.synchronize()
    kw = {}
    if alibi:
        kw = {"alibi_slopes": _alibi_slopes(Hq, "cpu", "torch.bfloat16").float(), "query_offset": N - 1}
    want = O.naive_attention(Q.cpu(), K.cpu(), V.cpu(), **kw)
    assert (out.float().cpu() - want).abs().max().item() <= TOL[torch.bfloat16]
