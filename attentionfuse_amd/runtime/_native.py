"""ctypes binding of ``libattnfuse_hip.so`` (C ABI: include/attnfuse_hip.h).

This is the only place Python touches the HIP kernels.  The library is
loaded from the package directory; there is no fallback path: if it is
missing or cannot be loaded every kernel call raises ``RuntimeError``.

Structure layouts mirror the header field for field (a CPU test compiles the
header with gcc and compares ``sizeof``/``offsetof`` against these classes).
"""
from __future__ import annotations

import ctypes as C
import os
import threading
from pathlib import Path

LIB_NAME = "libattnfuse_hip.so"
LIB_PATH = Path(__file__).resolve().parent.parent / LIB_NAME

AF_OK = 0
AF_ERR_UNSUPPORTED = -1
AF_ERR_BAD_ARG = -2
AF_ERR_LAUNCH = -3
AF_ERR_WORKSPACE = -4

I64x4 = C.c_int64 * 4
I64x3 = C.c_int64 * 3
I64x2 = C.c_int64 * 2


class SpecKeyC(C.Structure):
    _fields_ = [("dtype", C.c_int32), ("head_dim", C.c_int32),
                ("mask", C.c_int32), ("bias", C.c_int32),
                ("norm", C.c_int32), ("rope", C.c_int32)]


class BlockMaskC(C.Structure):
    _fields_ = [("full_kv_num", C.c_void_p), ("full_kv_idx", C.c_void_p),
                ("kv_num_blocks", C.c_void_p), ("kv_indices", C.c_void_p),
                ("q_num_blocks", C.c_void_p), ("q_indices", C.c_void_p),
                ("full_kv_stride", C.c_int64), ("kv_stride", C.c_int64),
                ("q_stride", C.c_int64),
                ("block_m", C.c_int32), ("block_n", C.c_int32),
                ("n_q_blocks", C.c_int32), ("n_kv_blocks", C.c_int32),
                ("q_items", C.c_void_p), ("q_splits", C.c_void_p),
                ("kv_items", C.c_void_p), ("kv_splits", C.c_void_p),
                ("n_q_items", C.c_int32), ("n_q_splits", C.c_int32),
                ("n_q_slots", C.c_int32),
                ("n_kv_items", C.c_int32), ("n_kv_splits", C.c_int32),
                ("n_kv_slots", C.c_int32),
                ("part_row_bits", C.c_void_p), ("q_col_bits", C.c_void_p),
                ("q_partial", C.c_void_p)]


class FwdArgsC(C.Structure):
    _fields_ = [("key", SpecKeyC),
                ("q", C.c_void_p), ("k", C.c_void_p), ("v", C.c_void_p),
                ("o", C.c_void_p), ("lse", C.c_void_p),
                ("cos", C.c_void_p), ("sin", C.c_void_p),
                ("alibi_slopes", C.c_void_p), ("bias", C.c_void_p),
                ("coverage", C.c_void_p),
                ("q_stride", I64x4), ("k_stride", I64x4),
                ("v_stride", I64x4), ("o_stride", I64x4),
                ("lse_stride", I64x3), ("rope_stride", I64x2),
                ("bias_stride", I64x4),
                ("batch", C.c_int32), ("heads_q", C.c_int32),
                ("heads_kv", C.c_int32), ("seqlen_q", C.c_int32),
                ("seqlen_kv", C.c_int32), ("rope_len", C.c_int32),
                ("scale", C.c_float), ("window", C.c_int32)]


class DecodeArgsC(C.Structure):
    _fields_ = [("key", SpecKeyC),
                ("q", C.c_void_p), ("k", C.c_void_p), ("v", C.c_void_p),
                ("o", C.c_void_p), ("alibi_slopes", C.c_void_p),
                ("q_stride", I64x4), ("k_stride", I64x4),
                ("v_stride", I64x4), ("o_stride", I64x4),
                ("batch", C.c_int32), ("heads_q", C.c_int32),
                ("heads_kv", C.c_int32), ("seqlen_kv", C.c_int32),
                ("scale", C.c_float), ("num_splits", C.c_int32)]


class BwdArgsC(C.Structure):
    _fields_ = [("key", SpecKeyC),
                ("q", C.c_void_p), ("k", C.c_void_p), ("v", C.c_void_p),
                ("o", C.c_void_p), ("dout", C.c_void_p), ("lse", C.c_void_p),
                ("dq", C.c_void_p), ("dk", C.c_void_p), ("dv", C.c_void_p),
                ("cos", C.c_void_p), ("sin", C.c_void_p),
                ("alibi_slopes", C.c_void_p),
                ("q_stride", I64x4), ("k_stride", I64x4),
                ("v_stride", I64x4), ("o_stride", I64x4),
                ("do_stride", I64x4), ("dq_stride", I64x4),
                ("dk_stride", I64x4), ("dv_stride", I64x4),
                ("lse_stride", I64x3), ("rope_stride", I64x2),
                ("batch", C.c_int32), ("heads_q", C.c_int32),
                ("heads_kv", C.c_int32), ("seqlen_q", C.c_int32),
                ("seqlen_kv", C.c_int32), ("rope_len", C.c_int32),
                ("scale", C.c_float), ("window", C.c_int32),
                ("group_split", C.c_int32)]


# Every symbol the header declares, with its ctypes signature.
SIGNATURES = {
    "af_fwd_workspace_bytes": (C.c_size_t, [C.POINTER(FwdArgsC)]),
    "af_fwd": (C.c_int, [C.POINTER(FwdArgsC), C.c_void_p, C.c_size_t,
                         C.c_void_p]),
    "af_fwd_blocksparse": (C.c_int, [C.POINTER(FwdArgsC),
                                     C.POINTER(BlockMaskC), C.c_void_p,
                                     C.c_size_t, C.c_void_p]),
    "af_fwd_blocksparse_workspace_bytes": (C.c_size_t, [
        C.POINTER(FwdArgsC), C.POINTER(BlockMaskC)]),
    "af_blockmask_plan": (C.c_int, [C.c_void_p, C.c_int32, C.c_int32,
                                    C.c_void_p, C.c_void_p, C.c_void_p]),
    "af_decode_num_splits": (C.c_int32, [C.c_int32] * 5),
    "af_decode_workspace_bytes": (C.c_size_t, [C.c_int32] * 4),
    "af_decode": (C.c_int, [C.POINTER(DecodeArgsC), C.c_void_p, C.c_size_t,
                            C.c_void_p]),
    "af_decode_noalloc": (C.c_int, [C.POINTER(DecodeArgsC), C.c_void_p]),
    "af_bwd_workspace_bytes": (C.c_size_t, [C.POINTER(BwdArgsC)]),
    "af_bwd_blocksparse_workspace_bytes": (C.c_size_t, [
        C.POINTER(BwdArgsC), C.POINTER(BlockMaskC)]),
    "af_bwd": (C.c_int, [C.POINTER(BwdArgsC), C.POINTER(BlockMaskC),
                         C.c_void_p, C.c_size_t, C.c_void_p]),
    "af_bwd_tile": (C.c_int, [C.POINTER(BwdArgsC), C.POINTER(BlockMaskC),
                              C.POINTER(C.c_int32), C.POINTER(C.c_int32),
                              C.POINTER(C.c_int32)]),
    "af_query": (C.c_int, [C.POINTER(SpecKeyC)]),
    "af_fwd_tile": (C.c_int, [C.POINTER(SpecKeyC), C.POINTER(C.c_int32),
                              C.POINTER(C.c_int32)]),
    "af_last_error": (C.c_char_p, []),
    "af_abi_version": (C.c_int, []),
}

ABI_VERSION = 6

_lib = None
_lock = threading.Lock()


def library_path() -> Path:
    override = os.environ.get("ATTNFUSE_LIB")
    return Path(override) if override else LIB_PATH


def lib():
    """Load (once) and return the native library; raise if unavailable."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            path = library_path()
            if not path.exists():
                raise RuntimeError(
                    f"AttnFuse HIP library not built: {path} is missing. "
                    "Run `python -c 'import __graft_entry__ as g; g.build()'` "
                    "or `python attentionfuse_amd/csrc/build.py`.")
            try:
                handle = C.CDLL(str(path))
            except OSError as e:
                raise RuntimeError(f"cannot load {path}: {e}") from e
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            if handle.af_abi_version() != ABI_VERSION:
                raise RuntimeError(
                    f"{path} has ABI {handle.af_abi_version()}, "
                    f"expected {ABI_VERSION}")
            _lib = handle
    return _lib


def last_error() -> str:
    return lib().af_last_error().decode(errors="replace")


class NativeError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"attnfuse_hip error {code}: {msg}")
        self.code = code


def check(rc: int) -> None:
    """Map a C status to the reference's exception types."""
    if rc == AF_OK:
        return
    msg = last_error()
    if rc == AF_ERR_UNSUPPORTED:
        raise NotImplementedError(f"attnfuse_hip: {msg}")
    if rc == AF_ERR_BAD_ARG:
        raise ValueError(f"attnfuse_hip: {msg}")
    raise NativeError(rc, msg)


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def strides(t, n: int):
    if t is None:
        return (0,) * n
    s = tuple(t.stride())
    return s + (0,) * (n - len(s))


def stream_handle(device) -> int:
    import torch
    return torch.cuda.current_stream(device).cuda_stream
