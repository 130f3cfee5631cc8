"""Long sequences (N = 65536): forward and backward of causal attention with
fused RoPE and a GQA group, checked against the oracle on row windows whose
exact values need only part of the problem.

* O and dQ of query rows [r0, r0 + R) depend on those rows alone (with all
  keys): the oracle runs on the window with query_offset r0.
* dK and dV of the last R keys get contributions only from the queries at or
  after them under the causal mask: the oracle runs on the last 2R queries
  and its gradients of those keys are exact.

This exercises 64-bit row offsets, the 4 GiB buffer-resource ranges per
(batch, head) slice and the group split at a size the full oracle could not
check.
"""
import pytest
import torch

import attnfuse as af
import oracle as O
from attnfuse.rope_utils import build_rope_cache

pytestmark = pytest.mark.gpu
TOL = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}
GRAD_REL = 1e-2


def rel(a, b):
    return ((a.double().cpu() - b.double()).norm() / b.double().norm()).item()


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 128), (torch.float16, 64)], ids=["bf16-d128", "f16-d64"])
def test_long_causal_rope_gqa(dtype, D):
    N, Hq, Hkv, R = 65536, 4, 1, 96
    print(f"[long] N={N} D={D} {dtype}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(5)
    Q = torch.randn(1, Hq, N, D, generator=g, device="cuda", dtype=dtype)
    K, V = (torch.randn(1, Hkv, N, D, generator=g, device="cuda", dtype=dtype) for _ in range(2))
    dO = torch.randn(1, Hq, N, D, generator=g, device="cuda", dtype=dtype)
    cos, sin = build_rope_cache(N, D, base=500000.0, device="cuda", dtype=dtype)
    fn = af.attention(lambda Q, K, V: af.softmax(af.causal(af.rope(Q, K))) @ V)
    q, k, v = (t.clone().requires_grad_(True) for t in (Q, K, V))
    out = fn(q, k, v, cos=cos, sin=sin)
    out.backward(dO)
    torch.cuda.synchronize()
    rope = (cos[0, 0].cpu(), sin[0, 0].cpu())
    Kc, Vc = K.cpu(), V.cpu()
    # a window of query rows in the middle of the sequence: O and dQ
    r0 = 40000
    o_ref, dq_ref, _, _ = O.attention_grads(Q[:, :, r0:r0 + R].cpu(), Kc, Vc, dO[:, :, r0:r0 + R].cpu(),
                                            dtype=torch.float32, causal=True, rope=rope, query_offset=r0)
    assert (out[:, :, r0:r0 + R].detach().float().cpu() - o_ref).abs().max().item() <= TOL[dtype]
    assert rel(q.grad[:, :, r0:r0 + R], dq_ref) <= GRAD_REL
    # the last 2R queries: exact dK / dV of the last R keys
    s0 = N - 2 * R
    o_ref, dq_ref, dk_ref, dv_ref = O.attention_grads(Q[:, :, s0:].cpu(), Kc, Vc, dO[:, :, s0:].cpu(),
                                                      dtype=torch.float32, causal=True, rope=rope,
                                                      query_offset=s0)
    assert (out[:, :, s0:].detach().float().cpu() - o_ref).abs().max().item() <= TOL[dtype]
    assert rel(q.grad[:, :, s0:], dq_ref) <= GRAD_REL
    assert rel(k.grad[:, :, N - R:], dk_ref[:, :, N - R:]) <= GRAD_REL
    assert rel(v.grad[:, :, N - R:], dv_ref[:, :, N - R:]) <= GRAD_REL
