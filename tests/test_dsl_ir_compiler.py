"""DSL, IR and compiler behaviour on the CPU (the reference's
tests/test_dsl.py, test_ir.py, test_compiler.py and the CPU half of
test_smoke.py), through the drop-in import name ``attnfuse``."""
import math

import pytest
import torch

import attnfuse as af
from attnfuse.compiler.fusion import FusionError, fuse_score_softmax
from attnfuse.compiler.lowering import kernel_constexprs, lower_to_tiled
from attnfuse.compiler.tiling import choose_tile_config
from attnfuse.ir.high_level import (BiasKind, Graph, MaskKind, MatMulPV,
                                    NormKind, NormOp, ScoreKind, ScoreOp)
from attnfuse.ir.printer import format_graph, format_tiled


def _zeros(D=32, N=16, H=2, dtype=torch.float32):
    z = torch.zeros(1, H, N, D, dtype=dtype)
    return z, z.clone(), z.clone()


def _trace(fn, D=64, H=4, N=16, dtype=torch.float32):
    return fn(*_zeros(D, N, H, dtype), return_graph=True)


def test_import_and_version():
    assert af.__version__
    import attentionfuse_amd
    assert af.attention is attentionfuse_amd.attention


def test_dense_graph_shape():
    @af.attention
    def fn(Q, K, V):
        return af.softmax(af.scaled_dot_product(Q, K)) @ V
    g = fn(*_zeros(), return_graph=True)
    assert g.score().scale is None
    assert g.collect_masks() == []
    assert g.norm().kind == NormKind.SOFTMAX
    assert g.q.head_dim == 32 and len(g.signature()) == 16


def test_causal_alibi_graph():
    @af.attention
    def fn(Q, K, V):
        s = af.scaled_dot_product(Q, K)
        s = af.alibi(s, num_heads=2)
        s = af.causal(s)
        return af.softmax(s) @ V
    g = fn(*_zeros(), return_graph=True)
    assert [m.kind for m in g.collect_masks()] == [MaskKind.CAUSAL]
    assert [b.kind for b in g.collect_biases()] == [BiasKind.ALIBI]


def test_combinator_argument_checks():
    with pytest.raises(ValueError):
        @af.attention
        def fn(Q, K, V):
            return af.softmax(af.sliding_window(af.scaled_dot_product(Q, K), 0)) @ V
        fn(*_zeros(), return_graph=True)
    with pytest.raises(ValueError):
        @af.attention
        def fn2(Q, K, V):
            return af.softmax(af.alibi(af.scaled_dot_product(Q, K), num_heads=0)) @ V
        fn2(*_zeros(), return_graph=True)


def test_missing_value_projection_message():
    @af.attention
    def fn(Q, K, V):
        return af.softmax(af.scaled_dot_product(Q, K))
    with pytest.raises(TypeError, match="value projection"):
        fn(*_zeros(), return_graph=True)


def test_probs_must_be_normalised():
    @af.attention
    def fn(Q, K, V):
        return af.scaled_dot_product(Q, K) @ V
    with pytest.raises(TypeError):
        fn(*_zeros(), return_graph=True)


def test_tracer_rejects_bad_shapes():
    @af.attention
    def fn(Q, K, V):
        return af.softmax(af.scaled_dot_product(Q, K)) @ V
    with pytest.raises(ValueError):
        fn(torch.zeros(2, 16, 32), torch.zeros(2, 16, 32), torch.zeros(2, 16, 32),
           return_graph=True)
    with pytest.raises(ValueError):
        fn(torch.zeros(1, 2, 16, 32), torch.zeros(1, 2, 16, 64),
           torch.zeros(1, 2, 16, 64), return_graph=True)


def test_signature_stable_and_discriminating():
    def make(variant):
        @af.attention
        def fn(Q, K, V):
            s = af.scaled_dot_product(Q, K)
            if variant == "causal":
                s = af.causal(s)
            if variant == "rope":
                s = af.causal(af.rope(Q, K))
            return af.softmax(s) @ V
        return fn(*_zeros(), return_graph=True).signature()
    assert make("causal") == make("causal")
    assert len({make("causal"), make("dense"), make("rope")}) == 3
    # sizes do not enter the signature; dtype and head_dim do
    @af.attention
    def fn(Q, K, V):
        return af.softmax(af.scaled_dot_product(Q, K)) @ V
    a = fn(*_zeros(N=16), return_graph=True).signature()
    assert a == af.attention(fn.graph_fn)(*_zeros(N=99, H=5), return_graph=True).signature()
    z = torch.zeros(1, 2, 16, 32, dtype=torch.float16)
    assert a != af.attention(fn.graph_fn)(z, z, z, return_graph=True).signature()


def _g():
    @af.attention
    def fn(Q, K, V):
        s = af.scaled_dot_product(Q, K)
        s = af.alibi(s, num_heads=4)
        s = af.causal(s)
        return af.softmax(s) @ V
    Q = torch.zeros(1, 4, 16, 64)
    return fn(Q, Q.clone(), Q.clone(), return_graph=True)


def test_printers():
    s = format_graph(_g())
    assert "MatMulPV" in s and "ScoreOp" in s
    assert "BLOCK_M" in format_tiled(lower_to_tiled(_g()))


def test_lowering_collapses_to_key():
    k = lower_to_tiled(_g())
    assert k.head_dim == 64
    assert k.mask_kind is MaskKind.CAUSAL
    assert k.bias_kind is BiasKind.ALIBI
    assert k.norm_kind is NormKind.SOFTMAX
    assert abs(k.score_scale - 1.0 / 8.0) < 1e-9
    assert k.abi_tuple() == (2, 64, 1, 1, 0, 0)


def test_lowering_folds_and_rejects_masks():
    @af.attention
    def sw_causal(Q, K, V):
        return af.softmax(af.causal(af.sliding_window(af.scaled_dot_product(Q, K), 8))) @ V
    k = lower_to_tiled(_trace(sw_causal))
    # one-sided window: keys i-W < j <= i (the reference's fold to the
    # two-sided window changes the function)
    assert k.mask_kind is MaskKind.CAUSAL_SLIDING_WINDOW and k.mask_window == 8
    assert k.mask_code == 4

    @af.attention
    def two_bias(Q, K, V):
        s = af.additive_bias(af.alibi(af.scaled_dot_product(Q, K), 4))
        return af.softmax(s) @ V
    with pytest.raises(NotImplementedError):
        lower_to_tiled(_trace(two_bias))

    @af.attention
    def bs_causal(Q, K, V):
        return af.softmax(af.causal(af.block_sparse(af.scaled_dot_product(Q, K)))) @ V
    with pytest.raises(NotImplementedError):
        lower_to_tiled(_trace(bs_causal))


def test_custom_scale_and_rope_flag():
    @af.attention
    def fn(Q, K, V):
        return af.relu_attention(af.rope(Q, K, scale=0.5)) @ V
    k = lower_to_tiled(_trace(fn))
    assert k.score_scale == 0.5 and k.rope_kind == 1 and k.norm_kind is NormKind.RELU


def test_fusion_checks():
    @af.attention
    def fn(Q, K, V):
        return af.softmax(af.causal(af.scaled_dot_product(Q, K))) @ V
    g = _trace(fn)
    fuse_score_softmax(g)
    bad = Graph(q=g.q, k=g.k, v=g.v,
                root=MatMulPV(probs=NormOp(kind=NormKind.SOFTMAX, scores=g.q), v=g.v))
    with pytest.raises(FusionError):
        fuse_score_softmax(bad)


def test_tile_config_for_each_head_dim():
    """A tile for every instantiated head dim (the reference's
    tests/test_compiler.py:25-32 loop); a head dim with no kernels raises
    NotImplementedError instead of returning a table entry that no launch
    uses."""
    from attentionfuse_amd.compiler.tiling import SUPPORTED_HEAD_DIMS
    for D in (32, 64, 96, 128, 256):
        @af.attention
        def fn(Q, K, V):
            return af.softmax(af.scaled_dot_product(Q, K)) @ V
        if D not in SUPPORTED_HEAD_DIMS:
            with pytest.raises(NotImplementedError):
                choose_tile_config(_trace(fn, D=D, dtype=torch.float16))
            continue
        cfg = choose_tile_config(_trace(fn, D=D, dtype=torch.float16))
        assert cfg.BLOCK_M >= 32 and cfg.BLOCK_N >= 16
        assert cfg.BLOCK_M == 32 * cfg.waves


def test_key_config_is_the_librarys_tile_for_every_instantiated_key():
    """lower_to_key(...).config is what af_fwd_tile reports, for every
    (dtype, head dim, mask, bias, norm, rope) the library instantiates."""
    import ctypes as C
    import itertools

    from attentionfuse_amd.compiler.tiling import SUPPORTED_HEAD_DIMS, tile_for_key
    from attentionfuse_amd.runtime import _native as N
    lib = N.lib()
    variants = {
        "dense": lambda Q, K, V: af.softmax(af.scaled_dot_product(Q, K)) @ V,
        "causal": lambda Q, K, V: af.softmax(af.causal(af.scaled_dot_product(Q, K))) @ V,
        "sw": lambda Q, K, V: af.softmax(af.sliding_window(af.scaled_dot_product(Q, K), 64)) @ V,
        "csw": lambda Q, K, V: af.softmax(af.causal(af.sliding_window(af.scaled_dot_product(Q, K), 64))) @ V,
        "bs": lambda Q, K, V: af.softmax(af.block_sparse(af.scaled_dot_product(Q, K))) @ V,
        "alibi": lambda Q, K, V: af.softmax(af.causal(af.alibi(af.scaled_dot_product(Q, K), 4))) @ V,
        "add": lambda Q, K, V: af.softmax(af.additive_bias(af.scaled_dot_product(Q, K))) @ V,
        "relu": lambda Q, K, V: af.relu_attention(af.causal(af.scaled_dot_product(Q, K))) @ V,
        "rope": lambda Q, K, V: af.softmax(af.causal(af.rope(Q, K))) @ V,
    }
    checked = 0
    for dt, D, (name, fn) in itertools.product(
            (torch.float16, torch.bfloat16, torch.float32), SUPPORTED_HEAD_DIMS, variants.items()):
        g = _trace(af.attention(fn), D=D, dtype=dt)
        try:
            k = lower_to_tiled(g)
        except NotImplementedError:
            # lowering refuses exactly the keys the library does not have
            from attnfuse.ir.spec import DTYPE_CODES
            codes = {"dense": (0, 0, 0, 0), "causal": (1, 0, 0, 0), "sw": (2, 0, 0, 0), "csw": (4, 0, 0, 0),
                     "bs": (3, 0, 0, 0), "alibi": (1, 1, 0, 0), "add": (0, 2, 0, 0), "relu": (1, 0, 1, 0),
                     "rope": (1, 0, 0, 1)}[name]
            assert not lib.af_query(N.SpecKeyC(DTYPE_CODES[str(dt).replace("torch.", "")], D, *codes))
            continue
        assert lib.af_query(N.SpecKeyC(*k.abi_tuple()))
        bm, bn = C.c_int32(), C.c_int32()
        assert lib.af_fwd_tile(N.SpecKeyC(*k.abi_tuple()), C.byref(bm), C.byref(bn)) == 0
        assert (k.config.BLOCK_M, k.config.BLOCK_N) == (bm.value, bn.value), (name, dt, D)
        assert k.config.waves == bm.value // 32
        checked += 1
    assert checked >= 2 * 3 * 9 + 3 * 8
    # every key the library accepts, not only those a graph lowers to
    for key in itertools.product((0, 1, 2), SUPPORTED_HEAD_DIMS, range(5), range(3), range(2), range(2)):
        if lib.af_query(N.SpecKeyC(*key)):
            cfg = tile_for_key(key)
            assert cfg.BLOCK_M % 32 == 0 and cfg.BLOCK_N in (32, 64)


def test_backward_tile_override_reaches_the_library():
    """_BWD_TILE / _pick_backward_tile: the library's default group split,
    an explicit power-of-two override, and the refusal of a bad one."""
    from attentionfuse_amd.runtime import _native as N
    from attentionfuse_amd.runtime import backward as bwd
    a = N.BwdArgsC()
    a.key = N.SpecKeyC(1, 128, 1, 0, 0, 1)
    a.batch, a.heads_q, a.heads_kv, a.seqlen_q, a.seqlen_kv = 1, 32, 8, 4096, 4096
    auto = bwd._pick_backward_tile(a)
    assert (auto["BLOCK_M"], auto["BLOCK_N"]) == (128, 128)
    assert auto["group_split"] in (1, 2, 4)
    a.group_split = 4
    assert bwd._pick_backward_tile(a)["group_split"] == 4
    a.group_split = 3
    with pytest.raises(ValueError):
        bwd._pick_backward_tile(a)
    a.group_split = 8                       # does not divide the group of 4
    with pytest.raises(ValueError):
        bwd._pick_backward_tile(a)
    saved = dict(bwd._BWD_TILE)
    try:
        bwd._BWD_TILE.update({"auto": False, "group_split": 2})
        assert bwd._group_split_request() == 2
    finally:
        bwd._BWD_TILE.clear()
        bwd._BWD_TILE.update(saved)
    assert bwd._group_split_request() == 0


def test_backward_tile_reference_keys():
    """The reference's _BWD_TILE keys (attnfuse/runtime/backward.py:26-32)
    and its _pick_backward_tile(N_q) call form: a key that matches the
    launch's shape is accepted, any other value -- and any num_stages --
    raises ValueError instead of being ignored; with "auto" on the keys are
    not consulted, as in the reference."""
    from attentionfuse_amd.runtime import _native as N
    from attentionfuse_amd.runtime import backward as bwd
    ref = bwd._pick_backward_tile(4096)
    assert {"BLOCK_M", "BLOCK_N", "num_warps", "num_stages"} <= set(ref)
    assert (ref["BLOCK_M"], ref["BLOCK_N"], ref["num_warps"]) == (128, 128, 4)
    assert bwd._pick_backward_tile(256) == ref
    a = N.BwdArgsC()
    a.key = N.SpecKeyC(0, 64, 1, 0, 0, 0)
    a.batch, a.heads_q, a.heads_kv, a.seqlen_q, a.seqlen_kv = 1, 12, 12, 4096, 4096
    have = bwd._pick_backward_tile(a)
    assert (have["BLOCK_M"], have["BLOCK_N"], have["num_warps"]) == (128, 128, 4)
    saved = dict(bwd._BWD_TILE)
    try:
        # the reference sweep's form: update with a config, then auto off
        bwd._BWD_TILE.update({"BLOCK_M": 64, "BLOCK_N": 64, "num_warps": 4})
        bwd._check_tile_request(a)          # auto still on: not consulted
        bwd._BWD_TILE["auto"] = False
        with pytest.raises(ValueError, match="BLOCK_M=64"):
            bwd._check_tile_request(a)
        bwd._BWD_TILE.update({"BLOCK_M": 128, "BLOCK_N": 128, "num_warps": 4})
        bwd._check_tile_request(a)          # the launch's own shape
        bwd._BWD_TILE["num_warps"] = 8
        with pytest.raises(ValueError, match="num_warps=8"):
            bwd._check_tile_request(a)
        bwd._BWD_TILE.update({"num_warps": None, "num_stages": 2})
        with pytest.raises(ValueError, match="num_stages=2"):
            bwd._check_tile_request(a)
        bwd._BWD_TILE.update({"BLOCK_M": None, "BLOCK_N": None, "num_stages": None,
                              "group_split": 2})
        bwd._check_tile_request(a)
        assert bwd._group_split_request() == 2
    finally:
        bwd._BWD_TILE.clear()
        bwd._BWD_TILE.update(saved)


def test_constexprs_change_with_variant():
    @af.attention
    def dense(Q, K, V):
        return af.softmax(af.scaled_dot_product(Q, K)) @ V

    @af.attention
    def causal(Q, K, V):
        return af.softmax(af.causal(af.scaled_dot_product(Q, K))) @ V
    cd = kernel_constexprs(lower_to_tiled(_trace(dense)))
    cc = kernel_constexprs(lower_to_tiled(_trace(causal)))
    assert cd["MASK_KIND"] != cc["MASK_KIND"]


def test_debug_printing(capsys, monkeypatch):
    monkeypatch.setenv("ATTNFUSE_DEBUG", "1")

    @af.attention
    def fn(Q, K, V):
        return af.softmax(af.scaled_dot_product(Q, K)) @ V
    fn(*_zeros(), return_graph=True)
    assert "traced graph" in capsys.readouterr().out
