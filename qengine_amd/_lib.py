"""ctypes binding of libqkv.so (the C ABI declared in include/qkv.h).

The library is built in-tree (qengine_amd/libqkv.so) by __graft_entry__.build().
There is no fallback: if the library is missing or fails to load, every call
raises QKVError.
"""
from __future__ import annotations

import ctypes
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libqkv.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "qkv.h")
# the benchmark's measurement helper lives in a library of its own
BENCH_LIB_PATH = os.path.join(_HERE, "libqkv_bench.so")
BENCH_HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "qkv_bench.h")

QKV_OK = 0
STATUS_NAMES = {
    0: "QKV_OK", -1: "QKV_ERR_INVALID", -2: "QKV_ERR_NULL", -3: "QKV_ERR_UNSUPPORTED",
    -4: "QKV_ERR_ALIGN", -5: "QKV_ERR_DEVICE", -6: "QKV_ERR_LAUNCH", -7: "QKV_ERR_WORKSPACE",
    -8: "QKV_ERR_TIMEOUT",
}


class QKVError(RuntimeError):
    def __init__(self, status: int, where: str = ""):
        self.status = status
        super().__init__(f"{where}: {STATUS_NAMES.get(status, status)} ({status})")


_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t

# name -> (restype, argtypes); must cover every function declared in include/qkv.h
SIGNATURES = {
    "qkv_version": (_I, []),
    "qkv_status_string": (ctypes.c_char_p, [_I]),
    "qkv_tq3_init": (_I, [_I]),
    "qkv_tq3_append": (_I, [_P, _P, _I, _P]),
    "qkv_tq3_append_kv": (_I, [_P, _P, _P, _P, _I, _P]),
    "qkv_tq3_dequant": (_I, [_P, _P, _I, _P]),
    "qkv_q8_append": (_I, [_P, _P, _I, _P]),
    "qkv_q8_append_kv": (_I, [_P, _P, _P, _P, _I, _P]),
    "qkv_q8_dequant": (_I, [_P, _P, _I, _P]),
    "qkv_kv_move_tokens": (_I, [_P, _P, _SZ, _SZ, ctypes.c_long, ctypes.c_long, _P, _I, _P]),
    "qkv_kv_gather_rows": (_I, [_P, _P, _P, _P, _SZ, _SZ, ctypes.c_long, _P, _I, _I, _I, _P]),
    "qkv_kv_scatter_rows": (_I, [_P, _P, _P, _P, _SZ, _SZ, ctypes.c_long, _P, _I, _I, _I, _P]),
    "qkv_dfk2_dequant": (_I, [_P, _P, _P, ctypes.c_longlong, _I, _P]),
    "qkv_tq3_append_dfk2": (_I, [_P, _P, _P, _I, _P]),
    "qkv_q8_append_dfk2": (_I, [_P, _P, _P, _I, _P]),
    "qkv_attn_split_tq3": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _I, _I,
                               _I, _P, _P]),
    "qkv_attn_split_q8": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _I, _P]),
    "qkv_attn_split_merge": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P]),
    "qkv_tq3_kpool_update": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _P]),
    "qkv_block_index_ms_workspace_bytes": (_SZ, [_I, _I, _I]),
    "qkv_block_index_ms": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _F, _P, _SZ,
                               _P]),
    "qkv_attn_block_sparse_split_tq3": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I,
                                            _F, _I, _I, _I, _P, _P]),
    "qkv_decode_attn_tq3_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "qkv_decode_attn_tq3": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _I, _I, _P, _P, _SZ,
                                _P]),
    "qkv_decode_attn_tq3_noalloc": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _I, _I, _P,
                                        _P]),
    "qkv_decode_attn_q8_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "qkv_decode_attn_q8": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _P, _SZ, _P]),
    "qkv_decode_attn_q8_append": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P, _SZ, _P]),
    "qkv_decode_attn_tq3_append": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _I, _I, _P, _P,
                                        _SZ, _P]),
    "qkv_decode_attn_q8k_tq3v_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "qkv_decode_attn_q8k_tq3v": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _P, _SZ, _P]),
    "qkv_tq3_append_kv_paged": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P, _I, _I, _I, _P, _P]),
    "qkv_decode_attn_tq3_paged_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "qkv_decode_attn_tq3_paged": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P, _I, _I, _I, _P, _I,
                                      _F, _P, _SZ, _P]),
    "qkv_decode_workspace_status": (_I, [_P, _P]),
    "qkv_decode_workspace_reset": (_I, [_P, _SZ, _P]),
    "qkv_decode_workspace_status_async": (_I, [_P, _P, _P]),
    "qkv_decode_noalloc_status": (_I, [_I, _P]),
    "qkv_decode_noalloc_reset": (_I, [_I, _P]),
    "qkv_decode_noalloc_status_async": (_I, [_I, _P, _P]),
    "qkv_debug_set_merge_spin_limit": (_I, [_I]),
    "qkv_prefill_attn_tq3_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "qkv_prefill_attn_tq3": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _P, _SZ, _P]),
}

BENCH_SIGNATURES = {
    "qkv_hbm_read_bench": (_I, [_P, _SZ, _P, _P]),
    "qkv_mfma_rate_bench": (_I, [_I, _I, _P, _P]),
}

_lib = None
_bench_lib = None


def header_functions(path: str = HEADER_PATH) -> list[str]:
    """Names of the functions declared in a header (include/qkv.h by default)."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qkv_[a-z0-9_]+)\s*\(", text)))


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise QKVError(-5, f"{LIB_PATH} is not built (run __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def bench_lib() -> ctypes.CDLL:
    """libqkv_bench.so (include/qkv_bench.h): the benchmark's streaming read and MFMA loop."""
    global _bench_lib
    if _bench_lib is None:
        if not os.path.exists(BENCH_LIB_PATH):
            raise QKVError(-5, f"{BENCH_LIB_PATH} is not built (run __graft_entry__.build())")
        L = ctypes.CDLL(BENCH_LIB_PATH)
        for name, (res, args) in BENCH_SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _bench_lib = L
    return _bench_lib


def check(status: int, where: str) -> None:
    if status != QKV_OK:
        raise QKVError(status, where)
