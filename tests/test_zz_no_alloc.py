"""af_decode_noalloc (flash decoding with library-owned split partials)
against af_decode on the same arguments, through the C ABI.

The two entry points launch the same kernels with the same split count, so
their outputs must agree bit for bit; both are also checked against the fp32
oracle.  Two calls run back to back, the second on a smaller problem, so the
shared device array is reused with a different layout.  The split-count
fitting and the size limit are checked too, and a call captured in a graph
(after the first, eager call on the GPU) replays bit-identically."""
import ctypes as C

import pytest
import torch

import oracle as O
from attentionfuse_amd.runtime import _native as N

pytestmark = pytest.mark.gpu
TOL = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}
LIMIT = 4 << 20   # AF_DECODE_NOALLOC_SCRATCH_BYTES


def _args(Q, K, V, out, num_splits=0, slopes=None):
    a = N.DecodeArgsC()
    dt = 0 if Q.dtype == torch.float16 else 1
    a.key = N.SpecKeyC(dt, Q.shape[-1], 0, 1 if slopes is not None else 0, 0, 0)
    a.q, a.k, a.v, a.o = Q.data_ptr(), K.data_ptr(), V.data_ptr(), out.data_ptr()
    a.alibi_slopes = N.ptr(slopes)
    a.q_stride[:] = Q.stride()
    a.k_stride[:] = K.stride()
    a.v_stride[:] = V.stride()
    a.o_stride[:] = out.stride()
    a.batch, a.heads_q, a.heads_kv, a.seqlen_kv = Q.shape[0], Q.shape[1], K.shape[1], K.shape[2]
    a.scale = Q.shape[-1] ** -0.5
    a.num_splits = num_splits
    return a


def _make(B, Hq, Hkv, N_kv, D, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    Q = torch.randn(B, Hq, 1, D, generator=g, device="cuda", dtype=dtype)
    K = torch.randn(B, Hkv, N_kv, D, generator=g, device="cuda", dtype=dtype)
    V = torch.randn(B, Hkv, N_kv, D, generator=g, device="cuda", dtype=dtype)
    return Q, K, V


def _both(Q, K, V, num_splits_ref, slopes=None):
    """(noalloc output, af_decode output at num_splits_ref)."""
    lib = N.lib()
    stream = torch.cuda.current_stream().cuda_stream
    o_na = torch.full_like(Q, float("nan"))
    o_ref = torch.full_like(Q, float("nan"))
    N.check(lib.af_decode_noalloc(_args(Q, K, V, o_na, 0, slopes), stream))
    a = _args(Q, K, V, o_ref, num_splits_ref, slopes)
    B, Hq, D = Q.shape[0], Q.shape[1], Q.shape[-1]
    nbytes = int(lib.af_decode_workspace_bytes(B, Hq, D, max(num_splits_ref, 1)))
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    N.check(lib.af_decode(a, ws.data_ptr(), nbytes, stream))
    torch.cuda.synchronize()
    return o_na, o_ref


def _default_splits(B, Hq, Hkv, N_kv, D):
    s = int(N.lib().af_decode_num_splits(B, Hq, Hkv, N_kv, D))
    per = int(N.lib().af_decode_workspace_bytes(B, Hq, D, 1))
    return min(s, LIMIT // per)


def test_two_calls_in_a_row_match_af_decode():
    cases = [
        # config-3 geometry at half the batch, then a smaller fp16 problem
        ((4, 32, 8, 32768, 128), torch.bfloat16, 1),
        ((2, 8, 2, 1000, 64), torch.float16, 2),
    ]
    for (B, Hq, Hkv, N_kv, D), dtype, seed in cases:
        print(f"[noalloc] B={B} Hq={Hq} Hkv={Hkv} N={N_kv} D={D} {dtype}", flush=True)
        Q, K, V = _make(B, Hq, Hkv, N_kv, D, dtype, seed)
        S = _default_splits(B, Hq, Hkv, N_kv, D)
        o_na, o_ref = _both(Q, K, V, S)
        assert torch.equal(o_na, o_ref), (o_na.float() - o_ref.float()).abs().max().item()
        want = O.naive_attention(Q.cpu(), K.cpu(), V.cpu())
        err = (o_na.float().cpu() - want).abs().max().item()
        assert err <= TOL[dtype], err


def test_split_count_is_lowered_to_fit():
    # 8 x 256 query rows at D=128: one split's partials are 1,064,960 bytes,
    # so the 4 MiB array holds 3 splits where the default asks for 4
    B, Hq, Hkv, N_kv, D = 8, 256, 16, 4096, 128
    per = int(N.lib().af_decode_workspace_bytes(B, Hq, D, 1))
    assert LIMIT // per == 3
    assert int(N.lib().af_decode_num_splits(B, Hq, Hkv, N_kv, D)) > 3
    print(f"[noalloc] fitted split count B={B}", flush=True)
    Q, K, V = _make(B, Hq, Hkv, N_kv, D, torch.bfloat16, 3)
    o_na, o_ref = _both(Q, K, V, 3)
    assert torch.equal(o_na, o_ref)
    sel = (slice(0, 1),)
    want = O.naive_attention(Q[sel].cpu(), K[sel].cpu(), V[sel].cpu())
    assert (o_na[sel].float().cpu() - want).abs().max().item() <= TOL[torch.bfloat16]


def test_alibi_after_a_larger_call():
    B, Hq, Hkv, N_kv, D = 2, 8, 2, 2500, 128
    print("[noalloc] alibi", flush=True)
    Q, K, V = _make(B, Hq, Hkv, N_kv, D, torch.float16, 5)
    slopes = torch.tensor([2.0 ** (-(h + 1)) for h in range(Hq)], device="cuda")
    S = _default_splits(B, Hq, Hkv, N_kv, D)
    o_na, o_ref = _both(Q, K, V, S, slopes)
    assert torch.equal(o_na, o_ref)
    want = O.naive_attention(Q.cpu(), K.cpu(), V.cpu(), alibi_slopes=slopes.cpu(),
                             query_offset=N_kv - 1)
    assert (o_na.float().cpu() - want).abs().max().item() <= TOL[torch.float16]


def test_sizes_beyond_the_limit_are_refused():
    lib = N.lib()
    per = int(lib.af_decode_workspace_bytes(1, 8, 128, 1))
    too_many = LIMIT // per + 1
    stream = torch.cuda.current_stream().cuda_stream
    # an explicit split count above the limit that the 32-key split rounding
    # trims to 128 non-empty splits is accepted, and matches af_decode
    print(f"[noalloc] {too_many} splits of 4096 keys", flush=True)
    Q, K, V = _make(1, 8, 2, 4096, 128, torch.bfloat16, 0)
    o_na = torch.full_like(Q, float("nan"))
    N.check(lib.af_decode_noalloc(_args(Q, K, V, o_na, too_many), stream))
    o_ref = torch.full_like(Q, float("nan"))
    nbytes = int(lib.af_decode_workspace_bytes(1, 8, 128, too_many))
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    N.check(lib.af_decode(_args(Q, K, V, o_ref, too_many), ws.data_ptr(), nbytes, stream))
    torch.cuda.synchronize()
    assert torch.equal(o_na, o_ref)
    # one whose non-empty splits still exceed the array is refused: 32-key
    # splits of a cache 32 * too_many keys long
    n_kv = 32 * too_many
    print(f"[noalloc] {too_many} splits of {n_kv} keys (refused)", flush=True)
    Q, K, V = _make(1, 8, 2, n_kv, 128, torch.bfloat16, 0)
    out = torch.empty_like(Q)
    assert lib.af_decode_noalloc(_args(Q, K, V, out, too_many), stream) == N.AF_ERR_WORKSPACE
    assert "limit" in N.last_error()
    # a batch whose single split does not fit
    a = _args(Q, K, V, out, 0)
    a.batch = LIMIT // (8 * 130 * 4) + 1
    a.q_stride[0] = a.o_stride[0] = 0
    a.k_stride[0] = a.v_stride[0] = 0
    assert lib.af_decode_noalloc(a, stream) == N.AF_ERR_WORKSPACE


def test_graph_capture_after_the_first_call():
    """After an eager call on the GPU, a captured af_decode_noalloc replays
    bit for bit like af_decode, with eager work between replays (the inputs
    are rewritten and the output cleared before each replay)."""
    B, Hq, Hkv, N_kv, D = 2, 16, 4, 3000, 128
    print(f"[noalloc] graph capture B={B} Hq={Hq} N={N_kv}", flush=True)
    lib = N.lib()
    Q, K, V = _make(B, Hq, Hkv, N_kv, D, torch.bfloat16, 7)
    S = _default_splits(B, Hq, Hkv, N_kv, D)
    o_first, _ = _both(Q, K, V, S)           # the first call, eager
    o_g = torch.full_like(Q, float("nan"))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        N.check(lib.af_decode_noalloc(_args(Q, K, V, o_g), torch.cuda.current_stream().cuda_stream))
    gen = torch.Generator(device="cuda").manual_seed(11)
    for rep in range(3):
        Q.copy_(torch.randn(Q.shape, generator=gen, device="cuda", dtype=Q.dtype))
        o_g.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        _, o_ref = _both(Q, K, V, S)
        assert torch.equal(o_g, o_ref), rep
    want = O.naive_attention(Q.cpu(), K.cpu(), V.cpu())
    assert (o_g.float().cpu() - want).abs().max().item() <= TOL[torch.bfloat16]
