"""Generate the golden fixtures in this directory.

    python tests/golden/make_golden.py

* ``tiny_attention.json`` -- brute-force attention on tiny shapes written
  with plain Python floats and ``math.exp`` loops (no torch, no oracle code),
  so it pins the oracle independently: dense, causal, sliding window,
  causal+ALiBi, additive bias, ReLU normalisation, fused RoPE, GQA and a
  single-query decode with the N_kv-1 ALiBi position.  Inputs come from
  ``random.Random(seed)``.
* ``bigbird_c4_grid.json`` -- the 64x64 block grid of the BigBird benchmark
  configuration (block row 0, block column 0, the |qb-kb| <= 1 band, 3 random
  key blocks per row from ``torch.randperm(64, generator=g)[:3]`` in row
  order, g seeded with 0).  Committed because CPU ``randperm`` streams are
  not guaranteed stable across torch versions.
"""
from __future__ import annotations

import json
import math
import random
from pathlib import Path

HERE = Path(__file__).resolve().parent


def _rand(rng, *shape):
    if not shape:
        return rng.gauss(0.0, 1.0)
    return [_rand(rng, *shape[1:]) for _ in range(shape[0])]


def _rope_vec(x, pos, base):
    d = len(x)
    h = d // 2
    out = [0.0] * d
    for i in range(h):
        ang = pos * base ** (-2.0 * i / d)
        c, s = math.cos(ang), math.sin(ang)
        out[i] = x[i] * c - x[i + h] * s
        out[i + h] = x[i + h] * c + x[i] * s
    return out


def brute(Q, K, V, *, causal=False, window=None, slopes=None, bias=None,
          norm="softmax", rope_base=None, q_offset=0, scale=None):
    """Q[b][h][i][d], K/V[b][hk][j][d] -> O[b][h][i][d], L[b][h][i]."""
    B, H, Nq, D = len(Q), len(Q[0]), len(Q[0][0]), len(Q[0][0][0])
    Hk, Nk = len(K[0]), len(K[0][0])
    G = H // Hk
    sc = 1.0 / math.sqrt(D) if scale is None else scale
    O = [[[[0.0] * D for _ in range(Nq)] for _ in range(H)] for _ in range(B)]
    L = [[[0.0] * Nq for _ in range(H)] for _ in range(B)]
    for b in range(B):
        for h in range(H):
            hk = h // G
            for i in range(Nq):
                qpos = i + q_offset
                q = Q[b][h][i]
                if rope_base is not None:
                    q = _rope_vec(q, qpos, rope_base)
                logits = []
                for j in range(Nk):
                    k = K[b][hk][j]
                    if rope_base is not None:
                        k = _rope_vec(k, j, rope_base)
                    ok = True
                    if causal and j > qpos:
                        ok = False
                    if window is not None and abs(qpos - j) >= window:
                        ok = False
                    if not ok:
                        logits.append(None)
                        continue
                    s = sum(q[d] * k[d] for d in range(D)) * sc
                    if slopes is not None:
                        s -= slopes[h] * abs(qpos - j)
                    if bias is not None:
                        s += bias[b][h][i][j]
                    logits.append(s)
                live = [s for s in logits if s is not None]
                if norm == "softmax":
                    m = max(live)
                    w = [0.0 if s is None else math.exp(s - m) for s in logits]
                    l = sum(w)
                    L[b][h][i] = m + math.log(l)
                else:
                    w = [0.0 if s is None else max(s, 0.0) for s in logits]
                    l = sum(w) or 1.0
                    L[b][h][i] = float("-inf")
                for d in range(D):
                    O[b][h][i][d] = sum(w[j] * V[b][hk][j][d]
                                        for j in range(Nk)) / l
    return O, L


def tiny_cases():
    rng = random.Random(20261201)
    cases = []

    def add(name, B, H, Hk, Nq, Nk, D, **kw):
        Q = _rand(rng, B, H, Nq, D)
        K = _rand(rng, B, Hk, Nk, D)
        V = _rand(rng, B, Hk, Nk, D)
        bias = kw.pop("bias_shape", None)
        if bias:
            kw["bias"] = _rand(rng, B, H, Nq, Nk)
        O, L = brute(Q, K, V, **kw)
        L = [[[None if math.isinf(x) else x for x in r] for r in h] for h in L]
        cases.append({"name": name, "Q": Q, "K": K, "V": V,
                      "kwargs": {k: v for k, v in kw.items()}, "O": O, "L": L})

    add("dense", 1, 2, 2, 5, 5, 4)
    add("causal", 1, 2, 2, 5, 5, 4, causal=True)
    add("sliding_window_2", 1, 2, 2, 6, 6, 4, window=2)
    add("causal_alibi", 1, 2, 2, 5, 5, 4, causal=True, slopes=[2.0 ** -4, 2.0 ** -8])
    add("additive_bias", 1, 2, 2, 4, 4, 4, bias_shape=True)
    add("relu_causal", 1, 2, 2, 5, 5, 4, causal=True, norm="relu")
    add("rope_causal", 1, 2, 2, 6, 6, 4, causal=True, rope_base=10000.0)
    add("gqa_causal", 1, 4, 2, 5, 5, 4, causal=True)
    add("decode_alibi", 2, 2, 1, 1, 7, 4, slopes=[0.5, 0.25], q_offset=6)
    add("cross_dense", 1, 2, 2, 3, 6, 4, scale=0.3)
    return cases


def bigbird_grid_fixture(n_blocks=64, n_random=3, seed=0):
    import torch
    g = torch.Generator().manual_seed(seed)
    rows = []
    for a in range(n_blocks):
        act = {0, *range(max(0, a - 1), min(n_blocks, a + 2))}
        if a == 0:
            act = set(range(n_blocks))
        act |= set(torch.randperm(n_blocks, generator=g)[:n_random].tolist())
        rows.append(sorted(act))
    return {"n_blocks": n_blocks, "n_random": n_random, "seed": seed,
            "block": 64, "rows": rows,
            "n_active": sum(len(r) for r in rows)}


if __name__ == "__main__":
    (HERE / "tiny_attention.json").write_text(json.dumps(tiny_cases()))
    (HERE / "bigbird_c4_grid.json").write_text(json.dumps(bigbird_grid_fixture()))
    print("wrote", HERE / "tiny_attention.json", HERE / "bigbird_c4_grid.json")
