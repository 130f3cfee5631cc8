"""The C-ABI library: it loads, exports every symbol the header declares,
its structs have the layout the ctypes binding assumes, and its argument
checks answer without touching a GPU."""
import ctypes as C
import re
import subprocess
import textwrap
from pathlib import Path

import pytest

from attentionfuse_amd.runtime import _native as N

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "attnfuse_hip.h"


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(af_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_and_reports_abi():
    lib = N.lib()
    assert lib.af_abi_version() == 6


def test_every_declared_symbol_is_exported():
    names = _declared_functions()
    assert "af_fwd" in names and "af_decode" in names and "af_bwd" in names
    lib = C.CDLL(str(N.library_path()))
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(N.SIGNATURES)


def test_struct_layouts_match_header(tmp_path):
    structs = {"af_spec_key": N.SpecKeyC, "af_blockmask": N.BlockMaskC,
               "af_fwd_args": N.FwdArgsC, "af_decode_args": N.DecodeArgsC,
               "af_bwd_args": N.BwdArgsC}
    lines = []
    for cname, py in structs.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for f, _ in py._fields_:
            lines.append(f'printf("{cname} {f} %zu\\n", offsetof({cname}, {f}));')
    src = tmp_path / "layout.c"
    src.write_text(textwrap.dedent(f"""
        #include <stdio.h>
        #include <stddef.h>
        #include "attnfuse_hip.h"
        int main(void) {{ {' '.join(lines)} return 0; }}
    """))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)],
                   check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout
    for line in out.splitlines():
        cname, field, val = line.split()
        py = structs[cname]
        want = C.sizeof(py) if field == "size" else getattr(py, field).offset
        assert int(val) == want, (cname, field)


def test_query_and_tile():
    lib = N.lib()
    assert lib.af_query(N.SpecKeyC(0, 64, 1, 1, 0, 1)) == 1
    assert lib.af_query(N.SpecKeyC(1, 128, 3, 0, 0, 0)) == 1
    assert lib.af_query(N.SpecKeyC(2, 64, 1, 1, 1, 1)) == 1      # fp32 forward
    assert lib.af_query(N.SpecKeyC(2, 64, 3, 0, 0, 0)) == 1      # fp32 block-sparse
    assert lib.af_query(N.SpecKeyC(3, 64, 0, 0, 0, 0)) == 0      # dtype
    assert lib.af_query(N.SpecKeyC(0, 80, 0, 0, 0, 0)) == 0      # head_dim
    bm, bn = C.c_int32(), C.c_int32()
    assert lib.af_fwd_tile(N.SpecKeyC(0, 64, 1, 0, 0, 0), C.byref(bm), C.byref(bn)) == 0
    assert (bm.value, bn.value) == (128, 64)
    assert lib.af_fwd_tile(N.SpecKeyC(2, 64, 1, 0, 0, 0), C.byref(bm), C.byref(bn)) == 0
    assert (bm.value, bn.value) == (128, 32)


def test_fp32_coverage_of_the_entry_points():
    """fp32 has forward and backward (block-sparse included) and decode
    kernels; head dim 256 refuses it with a message, and decode without a
    workspace fails on the workspace, not the dtype."""
    lib = N.lib()
    assert lib.af_query(N.SpecKeyC(2, 64, 3, 0, 0, 0)) == 1      # fp32 block-sparse forward
    assert lib.af_query(N.SpecKeyC(2, 256, 0, 0, 0, 0)) == 0     # fp32 head dim 256
    a = N.DecodeArgsC()
    a.key = N.SpecKeyC(2, 64, 0, 0, 0, 0)
    a.batch, a.heads_q, a.heads_kv, a.seqlen_kv = 1, 4, 4, 64
    a.q, a.k, a.v, a.o = 256, 256, 256, 256
    for s in (a.q_stride, a.k_stride, a.v_stride, a.o_stride):
        s[:] = (64 * 4 * 64, 64 * 64, 64, 1)
    a.scale = 0.125
    assert lib.af_decode(a, None, 0, None) == N.AF_ERR_WORKSPACE
    a.key = N.SpecKeyC(2, 256, 0, 0, 0, 0)
    assert lib.af_decode(a, None, 0, None) == N.AF_ERR_UNSUPPORTED
    assert "256" in N.last_error()
    b = N.BwdArgsC()
    b.key = N.SpecKeyC(2, 256, 3, 0, 0, 0)
    assert lib.af_bwd(b, None, None, 0, None) == N.AF_ERR_UNSUPPORTED
    assert "32, 64 and 128" in N.last_error()
    b.key = N.SpecKeyC(2, 64, 3, 0, 0, 0)          # fp32 block-sparse: checked further on
    assert lib.af_bwd(b, None, None, 0, None) == N.AF_ERR_BAD_ARG


def test_argument_errors_need_no_gpu():
    lib = N.lib()
    a = N.FwdArgsC()
    a.key = N.SpecKeyC(0, 64, 1, 0, 0, 0)
    a.batch, a.heads_q, a.heads_kv, a.seqlen_q, a.seqlen_kv = 1, 4, 4, 64, 64
    for s in (a.q_stride, a.k_stride, a.v_stride, a.o_stride):
        s[:] = (64 * 4 * 64, 64 * 64, 64, 1)
    assert lib.af_fwd(a, None, 0, None) == N.AF_ERR_BAD_ARG
    assert "NULL" in N.last_error()
    # tensors with no rows are never touched and may be NULL: an empty
    # problem is accepted and returns before any launch
    a.seqlen_q = a.seqlen_kv = 0
    assert lib.af_fwd(a, None, 0, None) == N.AF_OK
    a.seqlen_q = a.seqlen_kv = 64
    assert lib.af_fwd(None, None, 0, None) == N.AF_ERR_BAD_ARG
    # misaligned / non-unit strides are refused before any launch
    a.q = a.k = a.v = a.o = 16
    for s in (a.q_stride, a.k_stride, a.v_stride, a.o_stride):
        s[:] = (64 * 4 * 64, 64 * 64, 64, 2)
    a.batch, a.heads_q, a.heads_kv, a.seqlen_q, a.seqlen_kv = 1, 4, 4, 64, 64
    assert lib.af_fwd(a, None, 0, None) == N.AF_ERR_BAD_ARG
    assert "stride" in N.last_error()
    for s in (a.q_stride, a.k_stride, a.v_stride, a.o_stride):
        s[:] = (64 * 4 * 64, 64 * 64, 64, 1)
    a.heads_kv = 3
    assert lib.af_fwd(a, None, 0, None) == N.AF_ERR_BAD_ARG
    assert "multiple" in N.last_error()
    a.heads_kv = 4
    a.seqlen_kv = 32
    assert lib.af_fwd(a, None, 0, None) == N.AF_ERR_BAD_ARG        # causal needs Nq == Nkv
    a.key = N.SpecKeyC(3, 64, 0, 0, 0, 0)
    assert lib.af_fwd(a, None, 0, None) == N.AF_ERR_UNSUPPORTED       # no such dtype
    a.key = N.SpecKeyC(2, 64, 0, 0, 0, 0)
    assert lib.af_fwd(a, None, 0, None) == N.AF_ERR_BAD_ARG           # fp32 taken; scale 0 refused
    assert "scale" in N.last_error()
    a.key = N.SpecKeyC(2, 64, 0, 0, 0, 1)                               # fp32 k~ is 4 bytes a value
    a.seqlen_kv = 64
    assert lib.af_fwd_workspace_bytes(a) == 1 * 4 * 64 * 64 * 4
    a.seqlen_kv = 32
    # fused RoPE needs the rotated-key workspace: B*Hkv*Nkv*D*2 bytes, rounded
    # up to 256; refused before any launch when it is missing or too small
    a.key = N.SpecKeyC(0, 64, 0, 0, 0, 1)
    a.seqlen_kv = 64
    a.cos = a.sin = 256
    a.rope_stride[:] = (64, 1)
    a.rope_len = 64
    a.scale = 0.125
    assert lib.af_fwd_workspace_bytes(a) == 1 * 4 * 64 * 64 * 2
    a.seqlen_kv = a.seqlen_q = 63
    assert lib.af_fwd_workspace_bytes(a) == (4 * 63 * 64 * 2 + 255) // 256 * 256
    assert lib.af_fwd(a, None, 0, None) == N.AF_ERR_WORKSPACE
    assert "workspace" in N.last_error()
    assert lib.af_fwd(a, 256, 100, None) == N.AF_ERR_WORKSPACE
    a.key = N.SpecKeyC(0, 64, 0, 0, 0, 0)
    assert lib.af_fwd_workspace_bytes(a) == 0
    assert lib.af_fwd_workspace_bytes(None) == 0
    with pytest.raises(NotImplementedError):
        N.check(N.AF_ERR_UNSUPPORTED)
    with pytest.raises(ValueError):
        N.check(N.AF_ERR_BAD_ARG)


def test_decode_split_and_workspace_arithmetic():
    lib = N.lib()
    s = lib.af_decode_num_splits(8, 32, 8, 32768, 128)
    assert 1 <= s <= 256
    assert lib.af_decode_num_splits(1, 1, 1, 300, 64) == 1
    assert lib.af_decode_workspace_bytes(8, 32, 128, 16) == 16 * 8 * 32 * 130 * 4
    a = N.DecodeArgsC()
    a.key = N.SpecKeyC(1, 128, 0, 0, 0, 0)
    a.q = a.k = a.v = a.o = 256
    for st in (a.q_stride, a.k_stride, a.v_stride, a.o_stride):
        st[:] = (8 * 128, 128, 128, 1)
    a.batch, a.heads_q, a.heads_kv, a.seqlen_kv = 1, 8, 2, 1024
    a.scale, a.num_splits = 0.1, 4
    assert lib.af_decode(a, None, 0, None) == N.AF_ERR_WORKSPACE
    a.key = N.SpecKeyC(1, 128, 1, 0, 0, 0)
    assert lib.af_decode(a, None, 0, None) == N.AF_ERR_UNSUPPORTED


def test_element_mask_arguments_are_checked_before_any_launch():
    """af_fwd_blocksparse / af_bwd refuse element masks given only in part
    and element masks at head dim 256, from the arguments alone."""
    lib = N.lib()
    D, Nn = 64, 128
    a = N.FwdArgsC()
    a.key = N.SpecKeyC(0, D, 3, 0, 0, 0)
    a.batch, a.heads_q, a.heads_kv, a.seqlen_q, a.seqlen_kv = 1, 2, 2, Nn, Nn
    a.q = a.k = a.v = a.o = 256
    for s in (a.q_stride, a.k_stride, a.v_stride, a.o_stride):
        s[:] = (2 * Nn * D, Nn * D, D, 1)
    a.scale = 0.125
    bm = N.BlockMaskC()
    bm.full_kv_num = bm.full_kv_idx = bm.kv_num_blocks = bm.kv_indices = 256
    bm.q_num_blocks = bm.q_indices = 256
    bm.full_kv_stride = bm.kv_stride = bm.q_stride = 2
    bm.block_m = bm.block_n = 64
    bm.n_q_blocks = bm.n_kv_blocks = 2
    bm.part_row_bits = 256                         # the other two missing
    assert lib.af_fwd_blocksparse(a, bm, None, 0, None) == N.AF_ERR_BAD_ARG
    assert "all NULL or all set" in N.last_error()
    bm.q_col_bits = bm.q_partial = 256
    a.key = N.SpecKeyC(0, 256, 3, 0, 0, 0)
    for s in (a.q_stride, a.k_stride, a.v_stride, a.o_stride):
        s[:] = (2 * Nn * 256, Nn * 256, 256, 1)
    assert lib.af_fwd_blocksparse(a, bm, None, 0, None) == N.AF_ERR_UNSUPPORTED
    assert "128" in N.last_error()
    b = N.BwdArgsC()
    b.key = N.SpecKeyC(0, D, 3, 0, 0, 0)
    b.q = b.k = b.v = b.o = b.dout = b.dq = b.dk = b.dv = b.lse = 256
    for s in (b.q_stride, b.k_stride, b.v_stride, b.o_stride, b.do_stride, b.dq_stride, b.dk_stride, b.dv_stride):
        s[:] = (2 * Nn * D, Nn * D, D, 1)
    b.lse_stride[:] = (2 * Nn, Nn, 1)
    b.batch, b.heads_q, b.heads_kv, b.seqlen_q, b.seqlen_kv = 1, 2, 2, Nn, Nn
    b.scale = 0.125
    bm.q_partial = None
    ws = int(lib.af_bwd_blocksparse_workspace_bytes(b, bm))
    assert lib.af_bwd(b, bm, 256, ws, None) == N.AF_ERR_BAD_ARG
    assert "all NULL or all set" in N.last_error()
    # a block-sparse key has no mask-free workspace size, and a bad block
    # size is reported as such before any workspace arithmetic uses it
    assert int(lib.af_bwd_workspace_bytes(b)) == 0
    bm.q_col_bits = bm.part_row_bits = None
    bm.block_m = 96
    assert lib.af_bwd(b, bm, None, 0, None) == N.AF_ERR_UNSUPPORTED
    assert "64 or 128 blocks" in N.last_error()
