"""HuggingFace hook: registration, mask recognition and routing (CPU).

On the CPU every route ends in transformers' SDPA function, so a tiny
Llama run through ``attn_implementation="attnfuse"`` must reproduce
``"sdpa"`` exactly -- which also shows that the registered mask builder
keeps padding information.  The GPU kernels behind the routes are tested
in test_hf_gpu.py.
"""
import types

import pytest
import torch

transformers = pytest.importorskip("transformers")

import attnfuse.integrations.hf as hf  # noqa: E402


def _causal_bool(B, N):
    return torch.ones(N, N, dtype=torch.bool).tril().expand(B, 1, N, N)


def test_registered_under_reference_name():
    from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    assert ALL_ATTENTION_FUNCTIONS["attnfuse"] is hf.attnfuse_attention_forward
    assert "attnfuse" in ALL_MASK_ATTENTION_FUNCTIONS._global_mapping
    import attentionfuse_amd.integrations.hf as same
    assert same is hf


def test_causal_mask_recognition():
    N = 8
    assert hf._is_pure_causal_mask(None, N, N)
    assert hf._is_pure_causal_mask(_causal_bool(2, N).clone(), N, N)
    add = torch.zeros(1, 1, N, N).masked_fill(~_causal_bool(1, N), float("-inf"))
    assert hf._is_pure_causal_mask(add, N, N)
    add_min = torch.zeros(1, 1, N, N, dtype=torch.float16).masked_fill(
        ~_causal_bool(1, N), torch.finfo(torch.float16).min)
    assert hf._is_pure_causal_mask(add_min, N, N)
    # left padding in the second sequence
    pad = _causal_bool(2, N).clone()
    pad[1, :, :, :2] = False
    assert not hf._is_pure_causal_mask(pad, N, N)
    # the reference's corner test would accept this one (row 0 still blocks key 1)
    window = _causal_bool(1, N).clone()
    window[..., 5:, 0] = False
    assert not hf._is_pure_causal_mask(window, N, N)
    # a finite bias on the allowed positions is not a plain causal mask
    assert not hf._is_pure_causal_mask(add + 0.5 * _causal_bool(1, N), N, N)
    assert not hf._is_pure_causal_mask(_causal_bool(1, N), N, N + 1)
    assert not hf._is_pure_causal_mask(_causal_bool(1, N)[0], N, N)


def test_mask_answer_follows_in_place_edits():
    m = _causal_bool(1, 6).clone()
    assert hf._is_pure_causal_mask(m, 6, 6)
    m[0, 0, 4, 1] = False
    assert not hf._is_pure_causal_mask(m, 6, 6)


def test_routing_plan():
    dec = types.SimpleNamespace(is_causal=True)
    enc = types.SimpleNamespace(is_causal=False)
    q = torch.empty(1, 4, 16, 64)
    k16, k40 = torch.empty(1, 2, 16, 64), torch.empty(1, 2, 40, 64)
    assert hf.plan(dec, q, k16, None, 0.0, None) == "causal"
    assert hf.plan(dec, q, k16, _causal_bool(1, 16), 0.0, None) == "causal"
    assert hf.plan(dec, q, k16, None, 0.1, None) == "sdpa"
    assert hf.plan(enc, q, k16, None, 0.0, None) == "dense"
    assert hf.plan(dec, q, k16, None, 0.0, False) == "dense"
    # decode step over a cache: one query, full attention over the cache
    assert hf.plan(dec, q[:, :, :1], k40, None, 0.0, None) == "dense"
    # causal chunk with a cache offset: SDPA
    assert hf.plan(dec, q, k40, None, 0.0, None) == "sdpa"
    pad = _causal_bool(1, 16).clone()
    pad[..., :3] = False
    assert hf.plan(dec, q, k16, pad, 0.0, None) == "sdpa"
    # an explicit mask on a non-causal call is never dropped
    assert hf.plan(enc, q, k16, _causal_bool(1, 16), 0.0, None) == "sdpa"


def test_tiny_llama_matches_sdpa_on_cpu(monkeypatch):
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(vocab_size=128, hidden_size=128, intermediate_size=256,
                      num_hidden_layers=2, num_attention_heads=4,
                      num_key_value_heads=2, max_position_embeddings=256)
    torch.manual_seed(0)
    model = LlamaForCausalLM(cfg).eval()
    routes = []
    real = hf.plan
    monkeypatch.setattr(hf, "plan", lambda *a, **k: routes.append(real(*a, **k)) or routes[-1])
    ids = torch.randint(0, 128, (2, 16))
    am = torch.ones(2, 16, dtype=torch.long)
    am[1, :3] = 0
    with torch.no_grad():
        model.set_attn_implementation("sdpa")
        want_pad, want = model(ids, attention_mask=am).logits, model(ids).logits
        model.set_attn_implementation("attnfuse")
        got_pad, got = model(ids, attention_mask=am).logits, model(ids).logits
    assert routes == ["sdpa", "sdpa", "causal", "causal"]
    assert torch.equal(got_pad, want_pad) and torch.equal(got, want)
