"""fp32 backward (bwd_f32_kernel.hpp) against autograd of the oracle in fp64.

The reference runs fp32 backward in TF32 with dQ's product cast to bf16 and
tests it at 2e-2 (tests/test_backward.py:30-33,63-106).  Here every product
is fp32, so the bound is ||g - g_ref||_F / ||g_ref||_F <= 1e-4 per gradient
and 3e-5 max-abs on O.  Cases mirror the 16-bit backward tests: every mask,
ALiBi, fused RoPE, ragged lengths, head dims 32/64/128, GQA group sums and
an empty side.
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
