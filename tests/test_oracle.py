"""Pins the CPU oracle (oracle/attention.py) before anything is compared to
it: golden brute-force vectors, a library routine (SDPA in float64),
closed forms and invariants, the reference tests' known answers, and planted
mistakes that each check must catch."""
import json
import math
from pathlib import Path

import pytest
import torch
import torch.nn.functional as F

import oracle as O

GOLD = Path(__file__).resolve().parent / "golden"


def _t(x):
    return torch.tensor(x, dtype=torch.float64)


def _golden():
    return json.loads((GOLD / "tiny_attention.json").read_text())


def _run_case(case, **override):
    kw = dict(case["kwargs"])
    kw.update(override)
    Q, K, V = _t(case["Q"]), _t(case["K"]), _t(case["V"])
    args = {}
    if kw.get("causal"):
        args["causal"] = True
    if kw.get("window") is not None:
        args["window"] = kw["window"]
    if kw.get("slopes") is not None:
        args["alibi_slopes"] = kw["slopes"]
    if kw.get("bias") is not None:
        args["bias"] = _t(kw["bias"])
    if kw.get("norm"):
        args["norm"] = kw["norm"]
    if kw.get("scale") is not None:
        args["scale"] = kw["scale"]
    if kw.get("q_offset"):
        args["query_offset"] = kw["q_offset"]
    if kw.get("strict_causal"):
        # planted off-by-one: the diagonal key hidden from its own query
        args.pop("causal", None)
        i = torch.arange(Q.shape[2])[:, None]
        j = torch.arange(K.shape[2])[None, :]
        args["elem_mask"] = j < i
    if kw.get("rope_base") is not None:
        n = max(Q.shape[2] + kw.get("q_offset", 0), K.shape[2])
        args["rope"] = O.rope_tables(n, Q.shape[-1], kw["rope_base"], torch.float64)
    return O.naive_attention(Q, K, V, dtype=torch.float64, return_lse=True, **args)


@pytest.mark.parametrize("case", _golden(), ids=lambda c: c["name"])
def test_oracle_matches_bruteforce_golden(case):
    out, lse = _run_case(case)
    # RoPE tables are built in float32 (reference convention), the brute
    # force uses exact float64 angles
    tol = 1e-6 if case["kwargs"].get("rope_base") else 1e-10
    assert torch.allclose(out, _t(case["O"]), atol=tol, rtol=0)
    want = torch.tensor([[[float("-inf") if x is None else x for x in r]
                          for r in h] for h in case["L"]], dtype=torch.float64)
    assert torch.allclose(lse, want, atol=tol, rtol=0, equal_nan=False)


@pytest.mark.parametrize("mutation", ["scale", "swap_kv", "drop_mask", "alibi_sign",
                                      "causal_off_by_one", "drop_rope"])
def test_golden_catches_planted_mistakes(mutation):
    """A plausible oracle bug must make at least one golden case fail."""
    caught = False
    for case in _golden():
        kw = {}
        if mutation == "scale":
            kw["scale"] = 1.01 / math.sqrt(len(case["Q"][0][0][0]))
        elif mutation == "swap_kv":
            case = dict(case, K=case["V"], V=case["K"])
        elif mutation == "drop_mask":
            kw["causal"] = False
            kw["window"] = None
        elif mutation == "alibi_sign" and case["kwargs"].get("slopes"):
            kw["slopes"] = [-s for s in case["kwargs"]["slopes"]]
        elif mutation == "causal_off_by_one" and case["kwargs"].get("causal"):
            kw["strict_causal"] = True
        elif mutation == "drop_rope" and case["kwargs"].get("rope_base") is not None:
            kw["rope_base"] = None
        out, _ = _run_case(case, **kw)
        if not torch.allclose(out, _t(case["O"]), atol=1e-6, equal_nan=False):
            caught = True
    assert caught


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_oracle_matches_sdpa_float64(seed):
    g = torch.Generator().manual_seed(seed)
    B, H, Hk, N, D = 2, 4, 2, 37, 16
    Q = torch.randn(B, H, N, D, generator=g, dtype=torch.float64)
    K = torch.randn(B, Hk, N, D, generator=g, dtype=torch.float64)
    V = torch.randn(B, Hk, N, D, generator=g, dtype=torch.float64)
    bias = torch.randn(B, H, N, N, generator=g, dtype=torch.float64)
    slopes = O.alibi_slopes(H)
    i = torch.arange(N)
    keep = ((i[:, None] - i[None, :]).abs() < 9) & (i[None, :] <= i[:, None])
    add = bias - torch.tensor(slopes, dtype=torch.float64)[None, :, None, None] * \
        (i[:, None] - i[None, :]).abs().double()
    add = add.masked_fill(~keep, float("-inf"))
    want = F.scaled_dot_product_attention(Q, O.expand_kv(K, 2), O.expand_kv(V, 2),
                                          attn_mask=add, scale=0.3)
    got = O.naive_attention(Q, K, V, causal=True, window=9, alibi_slopes=slopes,
                            bias=bias, scale=0.3, dtype=torch.float64)
    assert torch.allclose(got, want, atol=1e-12)


def test_lse_is_logsumexp_of_scores():
    g = torch.Generator().manual_seed(3)
    Q, K, V = (torch.randn(1, 2, 9, 8, generator=g, dtype=torch.float64) for _ in range(3))
    _, L = O.naive_attention(Q, K, V, causal=True, dtype=torch.float64, return_lse=True)
    S = (Q @ K.transpose(-1, -2)) / math.sqrt(8)
    S = S.masked_fill(torch.ones(9, 9).triu(1).bool(), float("-inf"))
    assert torch.allclose(L, torch.logsumexp(S, dim=-1), atol=1e-12)


def test_rope_tables_closed_form_and_invariants():
    N, D, base = 50, 16, 10000.0
    cos, sin = O.rope_tables(N, D, base, torch.float64)
    t = torch.arange(N, dtype=torch.float64)[:, None]
    i = torch.arange(D // 2, dtype=torch.float64)[None, :]
    ang = t * base ** (-2 * i / D)
    assert torch.allclose(cos[:, : D // 2], torch.cos(ang).float().double(), atol=1e-6)
    assert torch.equal(cos[:, : D // 2], cos[:, D // 2:])
    assert torch.equal(sin[:, : D // 2], sin[:, D // 2:])
    x = torch.randn(1, 1, N, D, dtype=torch.float64)
    r = O.apply_rope(x, cos, sin)
    # position 0 is the identity; each (d, d + D/2) pair keeps its norm
    assert torch.allclose(r[..., 0, :], x[..., 0, :])
    n_in = x[..., : D // 2] ** 2 + x[..., D // 2:] ** 2
    n_out = r[..., : D // 2] ** 2 + r[..., D // 2:] ** 2
    assert torch.allclose(n_in, n_out, atol=1e-5)


def test_rope_relative_position_property():
    D, base = 8, 10000.0
    cos, sin = O.rope_tables(64, D, base, torch.float64)
    cos, sin = cos.double(), sin.double()
    q = torch.randn(D, dtype=torch.float64)
    k = torch.randn(D, dtype=torch.float64)

    def rot(v, p):
        return O.apply_rope(v[None, None, None], cos, sin, torch.tensor([p]))[0, 0, 0]
    a = torch.dot(rot(q, 20), rot(k, 13))
    b = torch.dot(rot(q, 37), rot(k, 30))
    # float32-built tables: agreement to the tables' precision
    assert abs(a - b) < 1e-5


def test_rope_gradient_is_the_transposed_rotation():
    """dx = g*cos + R^T(g*sin), R^T[y1; y2] = [y2; -y1] (the kernel's
    inverse rotation) equals autograd through apply_rope."""
    N, D = 7, 8
    cos, sin = O.rope_tables(N, D, 500000.0, torch.float64)
    x = torch.randn(1, 1, N, D, dtype=torch.float64, requires_grad=True)
    g = torch.randn(1, 1, N, D, dtype=torch.float64)
    O.apply_rope(x, cos, sin).backward(g)
    gs = g * sin
    rt = torch.cat([gs[..., D // 2:], -gs[..., : D // 2]], dim=-1)
    assert torch.allclose(x.grad, g * cos + rt, atol=1e-12)


def test_alibi_slopes_known_answers():
    assert O.alibi_slopes(8) == [2.0 ** -k for k in range(1, 9)]
    assert O.alibi_slopes(1) == [2.0 ** -8]
    h12 = [2.0 ** -k for k in range(1, 9)] + [2.0 ** -0.5, 2.0 ** -1.5, 2.0 ** -2.5, 2.0 ** -3.5]
    assert all(abs(a - b) < 1e-15 for a, b in zip(O.alibi_slopes(12), h12))
    assert all(abs(a - 2.0 ** (-0.5 * (k + 1))) < 1e-15
               for k, a in enumerate(O.alibi_slopes(16)))


def test_causal_alibi_equals_key_only_bias():
    """Under a causal mask -slope*|i-j| = slope*j - slope*i and the row term
    cancels in softmax: an independent closed form for causal ALiBi."""
    g = torch.Generator().manual_seed(5)
    Q, K, V = (torch.randn(1, 2, 11, 8, generator=g, dtype=torch.float64) for _ in range(3))
    sl = [0.3, 0.07]
    got = O.naive_attention(Q, K, V, causal=True, alibi_slopes=sl, dtype=torch.float64)
    j = torch.arange(11, dtype=torch.float64)
    bias = torch.tensor(sl, dtype=torch.float64)[None, :, None, None] * j[None, None, None, :]
    want = O.naive_attention(Q, K, V, causal=True, bias=bias.expand(1, 2, 11, 11),
                             dtype=torch.float64)
    assert torch.allclose(got, want, atol=1e-12)


@pytest.mark.parametrize("splits", [1, 2, 3, 7, 16])
def test_decode_combine_independent_of_split_count(splits):
    g = torch.Generator().manual_seed(11)
    Q = torch.randn(2, 8, 1, 16, generator=g, dtype=torch.float64)
    K = torch.randn(2, 2, 133, 16, generator=g, dtype=torch.float64)
    V = torch.randn(2, 2, 133, 16, generator=g, dtype=torch.float64)
    sl = O.alibi_slopes(8)
    want = O.naive_attention(Q, K, V, alibi_slopes=sl, query_offset=132, dtype=torch.float64)
    got = O.decode_split_combine(Q, K, V, splits, alibi_slopes=sl)
    assert torch.allclose(got, want, atol=1e-12)


def test_gradients_pass_gradcheck():
    g = torch.Generator().manual_seed(7)
    cos, sin = O.rope_tables(6, 4, 10000.0, torch.float64)
    Q = torch.randn(1, 4, 6, 4, generator=g, dtype=torch.float64, requires_grad=True)
    K = torch.randn(1, 2, 6, 4, generator=g, dtype=torch.float64, requires_grad=True)
    V = torch.randn(1, 2, 6, 4, generator=g, dtype=torch.float64, requires_grad=True)

    def f(q, k, v):
        return O.naive_attention(q, k, v, causal=True, alibi_slopes=[0.5, 0.25, 0.1, 0.05],
                                 rope=(cos, sin), dtype=torch.float64)
    assert torch.autograd.gradcheck(f, (Q, K, V))


def test_gqa_grads_are_group_sums():
    g = torch.Generator().manual_seed(9)
    Q = torch.randn(1, 6, 8, 4, generator=g, dtype=torch.float64)
    K = torch.randn(1, 2, 8, 4, generator=g, dtype=torch.float64)
    V = torch.randn(1, 2, 8, 4, generator=g, dtype=torch.float64)
    dO = torch.randn(1, 6, 8, 4, generator=g, dtype=torch.float64)
    _, dq, dk, dv = O.attention_grads(Q, K, V, dO, causal=True)
    _, dq2, dk2, dv2 = O.attention_grads(Q, O.expand_kv(K, 3), O.expand_kv(V, 3), dO, causal=True)
    assert torch.allclose(dq, dq2, atol=1e-12)
    assert torch.allclose(dk, dk2.view(1, 2, 3, 8, 4).sum(2), atol=1e-12)
    assert torch.allclose(dv, dv2.view(1, 2, 3, 8, 4).sum(2), atol=1e-12)


def test_block_grid_known_answers():
    N, Bk = 256, 64
    nb = N // Bk
    grid = O.block_grid(lambda q, k: torch.ones_like(q, dtype=torch.bool), N, N, Bk, Bk)
    assert int(grid.sum()) == 16
    grid = O.block_grid(lambda q, k: ((q // Bk) - (k // Bk)).abs() <= 1, N, N, Bk, Bk)
    assert int(grid.sum()) == 3 * nb - 2
    grid = O.block_grid(lambda q, k: ((q // Bk) + (k // Bk)) % 2 == 0, N, N, Bk, Bk)
    assert int(grid.sum()) == (nb * nb) // 2 + (nb % 2)
    # one element inside a tile is enough to make it active (rounded up)
    grid = O.block_grid(lambda q, k: (q == 70) & (k == 3), N, N, Bk, Bk)
    assert grid.sum() == 1 and grid[1, 0]
    rows, cols = O.block_lists(O.block_grid(lambda q, k: k <= q, N, N, Bk, Bk))
    assert rows == [[0], [0, 1], [0, 1, 2], [0, 1, 2, 3]]
    assert cols == [[0, 1, 2, 3], [1, 2, 3], [2, 3], [3]]


def test_bigbird_fixture_structure():
    fx = json.loads((GOLD / "bigbird_c4_grid.json").read_text())
    n = fx["n_blocks"]
    grid = torch.zeros(n, n, dtype=torch.bool)
    for a, row in enumerate(fx["rows"]):
        grid[a, row] = True
    assert grid[0].all() and grid[:, 0].all()
    for a in range(n):
        for b in range(max(0, a - 1), min(n, a + 2)):
            assert grid[a, b]
    assert int(grid.sum()) == fx["n_active"]
    # 3 random picks add at most 3 blocks to each row's base pattern
    for a in range(1, n):
        base = {0, *range(max(0, a - 1), min(n, a + 2))}
        assert 0 <= len(set(fx["rows"][a]) - base) <= 3
    # the oracle's generator reproduces the fixture on this torch build
    assert torch.equal(O.bigbird_grid(n, fx["n_random"], fx["seed"]), grid)


def test_expected_coverage_causal_staircase():
    cov = O.expected_coverage(256, 256, mask="causal")
    # 32-row block a sees 64-key block b iff 64 b <= 32 a + 31
    for a in range(8):
        for b in range(4):
            assert cov[a, b] == int(64 * b <= 32 * a + 31)


@pytest.mark.parametrize("Nq,Nkv,window", [(256, 256, 48), (333, 333, 7), (200, 200, 100),
                                           (64, 300, 1)])
def test_expected_coverage_is_any_visible_pair(Nq, Nkv, window):
    """Every tile formula against brute force: a 32x64 tile is visited iff
    some (i, j) pair inside it is visible under the element-level mask."""
    i = torch.arange(Nq)[:, None]
    j = torch.arange(Nkv)[None, :]
    preds = {"full": torch.ones(Nq, Nkv, dtype=torch.bool),
             "sliding_window": (i - j).abs() < window}
    if Nq == Nkv:
        preds["causal"] = j <= i
        preds["causal_sliding_window"] = (j <= i) & (i - j < window)
    g = torch.Generator().manual_seed(Nq)
    grid = torch.rand(-(-Nq // 64), -(-Nkv // 128), generator=g) < 0.4
    preds["block_sparse"] = O.element_mask_from_grid(grid, Nq, Nkv, 64, 128)
    nq, nk = -(-Nq // 32), -(-Nkv // 64)
    for mask, keep in preds.items():
        pad = torch.zeros(nq * 32, nk * 64, dtype=torch.bool)
        pad[:Nq, :Nkv] = keep
        brute = pad.view(nq, 32, nk, 64).any(3).any(1).to(torch.int32)
        got = O.expected_coverage(Nq, Nkv, mask=mask, window=window, grid=grid, bm=64, bn=128)
        assert torch.equal(got, brute), mask
