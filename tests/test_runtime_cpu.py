"""Host logic that needs no GPU: routing predicates, slopes, RoPE tables,
layout helpers and the reference's error types."""
import math

import pytest
import torch

import attnfuse as af
import oracle as O
from attnfuse.rope_utils import apply_rope, build_rope_cache
from attnfuse.runtime.backward import can_backward
from attnfuse.runtime.dispatch import (_alibi_slopes, alibi_slope_values,
                                       kernel_layout, run_attention)
from attnfuse.runtime.flash_decode import can_use_flash_decode


def _graph(fn, D=64, H=4, N=16, dtype=torch.float16):
    z = torch.zeros(1, H, N, D, dtype=dtype)
    return fn(z, z, z, return_graph=True)


@af.attention
def dense(Q, K, V):
    return af.softmax(af.scaled_dot_product(Q, K)) @ V


@af.attention
def causal(Q, K, V):
    return af.softmax(af.causal(af.scaled_dot_product(Q, K))) @ V


@af.attention
def rope_causal(Q, K, V):
    return af.softmax(af.causal(af.rope(Q, K))) @ V


@af.attention
def relu(Q, K, V):
    return af.relu_attention(af.scaled_dot_product(Q, K)) @ V


@af.attention
def additive(Q, K, V):
    return af.softmax(af.additive_bias(af.scaled_dot_product(Q, K))) @ V


@af.attention
def bs(Q, K, V):
    return af.softmax(af.block_sparse(af.scaled_dot_product(Q, K))) @ V


@pytest.mark.parametrize("H", [1, 2, 3, 5, 8, 12, 16, 32])
def test_product_slopes_equal_oracle(H):
    assert alibi_slope_values(H) == pytest.approx(O.alibi_slopes(H), abs=1e-15)
    assert _alibi_slopes(H, "cpu", "torch.float16").dtype == torch.float16


@pytest.mark.parametrize("base", [10000.0, 500000.0])
def test_product_rope_tables_equal_oracle(base):
    c, s = build_rope_cache(33, 64, base=base, device="cpu", dtype=torch.float32)
    oc, os_ = O.rope_tables(33, 64, base)
    assert c.shape == (1, 1, 33, 64)
    assert torch.equal(c[0, 0], oc) and torch.equal(s[0, 0], os_)
    x = torch.randn(1, 2, 33, 64)
    assert torch.allclose(apply_rope(x, c, s), O.apply_rope(x, oc, os_))


def test_decode_and_backward_predicates():
    q1 = torch.zeros(1, 4, 1, 64, dtype=torch.float16)
    k = torch.zeros(1, 4, 512, 64, dtype=torch.float16)
    assert can_use_flash_decode(_graph(dense), q1, k)
    assert not can_use_flash_decode(_graph(causal), q1, k)
    assert not can_use_flash_decode(_graph(rope_causal), q1, k)
    assert not can_use_flash_decode(_graph(relu), q1, k)
    assert not can_use_flash_decode(_graph(dense), q1, k[:, :, :100])
    assert not can_use_flash_decode(_graph(dense), torch.zeros(1, 4, 2, 64, dtype=torch.float16), k)
    assert can_backward(_graph(causal)) and can_backward(_graph(rope_causal))
    assert can_backward(_graph(bs))
    assert not can_backward(_graph(relu)) and not can_backward(_graph(additive))


def test_kernel_layout_repairs_strides():
    t = torch.randn(2, 8, 16, 64)
    assert kernel_layout(t) is t
    tt = t.transpose(1, 2)              # still unit d-stride, rows aligned
    assert kernel_layout(tt) is tt
    odd = torch.randn(3, 5, 7, 12)[..., :10]
    fixed = kernel_layout(odd)
    assert torch.equal(fixed, odd) and fixed.stride(-1) == 1
    assert all(s % 8 == 0 for s in fixed.stride()[:-1])


def test_cpu_tensors_raise_runtime_error():
    q = torch.zeros(1, 2, 16, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError):
        run_attention(_graph(dense), q, q, q)
    with pytest.raises(RuntimeError):
        causal(q, q, q)


def test_block_sparse_mask_errors():
    q = torch.zeros(1, 2, 128, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="block_mask"):
        bs(q, q, q)
    with pytest.raises(TypeError):
        bs(q, q, q, block_mask=object())


def test_call_keywords_are_checked_before_any_launch():
    """Unknown call-time keywords raise TypeError; inference-only buffers
    (out=, save_lse=, coverage=) with an input that requires grad raise
    ValueError instead of being dropped by the autograd route."""
    z = torch.zeros(1, 2, 16, 64, dtype=torch.float16)
    with pytest.raises(TypeError):
        causal(z, z, z, bogus=1)
    zq = z.clone().requires_grad_(True)
    with pytest.raises(ValueError):
        causal(zq, z, z, out=torch.empty_like(z))


def test_missing_library_raises_runtime_error(monkeypatch, tmp_path):
    """Failure detection: a library that is not built, or is not a shared
    object, makes the first native call raise RuntimeError naming the path
    (there is no CPU fallback to drop into)."""
    from attentionfuse_amd.runtime import _native as N
    missing = tmp_path / "libattnfuse_hip.so"
    monkeypatch.setattr(N, "_lib", None)
    monkeypatch.setenv("ATTNFUSE_LIB", str(missing))
    with pytest.raises(RuntimeError, match="not built"):
        N.lib()
    with pytest.raises(RuntimeError, match="not built"):
        N.last_error()
    missing.write_bytes(b"not an ELF file")
    with pytest.raises(RuntimeError, match="cannot load"):
        N.lib()
    assert N._lib is None                  # nothing half-loaded is cached
