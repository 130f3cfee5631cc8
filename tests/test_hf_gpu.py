"""HuggingFace hook on the GPU: the fused kernels behind
``attn_implementation="attnfuse"`` against the fp32 oracle, in transformers'
calling convention (strided (B, H, N, D) views in, (B, N, H, D) out)."""
import types

import pytest
import torch

transformers = pytest.importorskip("transformers")

import attnfuse.integrations.hf as hf  # noqa: E402
import oracle as O  # noqa: E402

pytestmark = pytest.mark.gpu
TOL = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}
GRAD_REL = 1e-2


@pytest.fixture
def no_sdpa(monkeypatch):
    """Fail the test if a call falls back to SDPA: the kernel must run."""
    def boom(*a, **k):
        raise AssertionError("routed to SDPA")
    monkeypatch.setattr(hf, "_sdpa", boom)


def hf_views(B, Hq, Hkv, Nq, Nkv, D, dtype, seed=0):
    """q/k/v as a Llama layer produces them: projections laid out
    (B, N, H, D) and viewed as (B, H, N, D)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(B, Nq, Hq, D, generator=g, device="cuda", dtype=dtype).transpose(1, 2)
    k = torch.randn(B, Nkv, Hkv, D, generator=g, device="cuda", dtype=dtype).transpose(1, 2)
    v = torch.randn(B, Nkv, Hkv, D, generator=g, device="cuda", dtype=dtype).transpose(1, 2)
    return q, k, v


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("case", [
    # (B, Hq, Hkv, Nq, Nkv, D, causal, scaling)
    (2, 8, 2, 256, 256, 64, True, None),
    (1, 8, 8, 200, 200, 128, True, 0.2),
    (2, 8, 2, 1, 1000, 128, True, None),       # decode step over a cache
    (2, 4, 4, 96, 96, 64, False, None),        # encoder (non-causal)
    (1, 4, 2, 48, 130, 64, False, 0.1),        # cross-attention
], ids=["prefill_gqa", "prefill_scaled", "decode", "encoder", "cross"])
def test_attention_function_matches_oracle(case, dtype, no_sdpa):
    B, Hq, Hkv, Nq, Nkv, D, causal, scaling = case
    q, k, v = hf_views(B, Hq, Hkv, Nq, Nkv, D, dtype)
    module = types.SimpleNamespace(is_causal=causal)
    out, w = hf.attnfuse_attention_forward(module, q, k, v, None, scaling=scaling)
    torch.cuda.synchronize()
    assert w is None and out.shape == (B, Nq, Hq, D) and out.is_contiguous()
    want = O.naive_attention(q.cpu(), k.cpu(), v.cpu(), causal=causal and Nq > 1,
                             scale=scaling)
    assert (out.float().cpu().transpose(1, 2) - want).abs().max().item() <= TOL[dtype]


def test_explicit_causal_mask_uses_kernel(no_sdpa):
    q, k, v = hf_views(1, 4, 2, 64, 64, 64, torch.float16, seed=1)
    mask = torch.ones(64, 64, dtype=torch.bool, device="cuda").tril()[None, None]
    out, _ = hf.attnfuse_attention_forward(types.SimpleNamespace(is_causal=True),
                                           q, k, v, mask, scaling=0.125)
    want = O.naive_attention(q.cpu(), k.cpu(), v.cpu(), causal=True, scale=0.125)
    assert (out.float().cpu().transpose(1, 2) - want).abs().max().item() <= TOL[torch.float16]


def test_padding_mask_matches_sdpa_exactly():
    from transformers.integrations.sdpa_attention import sdpa_attention_forward
    q, k, v = hf_views(2, 4, 2, 64, 64, 64, torch.float16, seed=2)
    mask = torch.ones(64, 64, dtype=torch.bool, device="cuda").tril().repeat(2, 1, 1, 1)
    mask[1, :, :, :5] = False
    module = types.SimpleNamespace(is_causal=True, num_key_value_groups=2)
    got, _ = hf.attnfuse_attention_forward(module, q, k, v, mask, scaling=0.125)
    want, _ = sdpa_attention_forward(module, q, k, v, mask, scaling=0.125)
    assert torch.equal(got, want)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
def test_training_route_gradients(dtype, no_sdpa):
    q, k, v = hf_views(1, 8, 2, 128, 128, 64, dtype, seed=3)
    q, k, v = (t.detach().requires_grad_(True) for t in (q, k, v))
    out, _ = hf.attnfuse_attention_forward(types.SimpleNamespace(is_causal=True),
                                           q, k, v, None, scaling=None)
    assert out.shape == (1, 128, 8, 64)
    g = torch.Generator(device="cuda").manual_seed(4)
    dO = torch.randn(out.shape, generator=g, device="cuda", dtype=dtype)
    out.backward(dO)
    o_ref, dq, dk, dv = O.attention_grads(q.detach().cpu(), k.detach().cpu(), v.detach().cpu(),
                                          dO.cpu().transpose(1, 2), dtype=torch.float32,
                                          causal=True)
    assert (out.detach().float().cpu().transpose(1, 2) - o_ref).abs().max().item() <= TOL[dtype]
    for got, ref in ((q.grad, dq), (k.grad, dk), (v.grad, dv)):
        assert ((got.float().cpu() - ref).norm() / ref.norm()).item() <= GRAD_REL


def test_tiny_llama_prefill_and_decode_against_sdpa():
    """A locally built 2-layer Llama (GQA 8/2, head_dim 64) in fp16: logits
    of a prefill and of one cached decode step, attnfuse vs sdpa."""
    from transformers import DynamicCache, LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(vocab_size=512, hidden_size=512, intermediate_size=1024,
                      num_hidden_layers=2, num_attention_heads=8,
                      num_key_value_heads=2, max_position_embeddings=1024)
    torch.manual_seed(0)
    model = LlamaForCausalLM(cfg).to("cuda", torch.float16).eval()
    ids = torch.randint(0, 512, (2, 200), device="cuda")
    nxt = torch.randint(0, 512, (2, 1), device="cuda")
    res = {}
    routes = []
    real = hf.plan

    def spy(*a, **k):
        routes.append(real(*a, **k))
        return routes[-1]
    hf.plan = spy
    try:
        for impl in ("sdpa", "attnfuse"):
            model.set_attn_implementation(impl)
            with torch.no_grad():
                cache = DynamicCache(config=cfg)
                pre = model(ids, past_key_values=cache, use_cache=True)
                dec = model(nxt, past_key_values=pre.past_key_values, use_cache=True)
            res[impl] = (pre.logits.float(), dec.logits.float())
    finally:
        hf.plan = real
    assert routes == ["causal", "causal", "dense", "dense"]
    for got, want in zip(res["attnfuse"], res["sdpa"]):
        assert ((got - want).norm() / want.norm()).item() <= 1e-2
