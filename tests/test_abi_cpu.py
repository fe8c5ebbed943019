"""CPU-side checks of the C ABI: libqkv.so loads, exports every function that
include/qkv.h declares, and rejects bad arguments before touching a GPU."""
import ctypes

import pytest

from qengine_amd import _lib


@pytest.fixture(scope="module")
def L():
    return _lib.lib()


def test_exports_every_declared_function(L):
    names = _lib.header_functions()
    assert names, "no declarations parsed from include/qkv.h"
    for n in names:
        assert hasattr(L, n), f"libqkv.so does not export {n}"
        assert n in _lib.SIGNATURES, f"ctypes binding lacks {n}"


def test_version_and_status_strings(L):
    assert L.qkv_version() >= 100
    for code in _lib.STATUS_NAMES:
        assert L.qkv_status_string(code)
    assert L.qkv_status_string(0) == b"ok"


def test_argument_errors_without_gpu(L):
    buf = ctypes.create_string_buffer(4096)
    p = ctypes.addressof(buf)
    p16 = (p + 15) & ~15
    assert L.qkv_tq3_append(p16, p16, -1, None) == -1
    assert L.qkv_tq3_append(p16, p16, 0, None) == 0          # empty append is a no-op
    assert L.qkv_tq3_append(None, p16, 4, None) == -2
    assert L.qkv_tq3_append(p16 + 2, p16, 4, None) == -4     # fp16 input must be 16-B aligned
    assert L.qkv_tq3_append(p16, p16 + 2, 4, None) == -4     # blocks are 4-B aligned
    assert L.qkv_tq3_append_kv(p16, None, p16, p16, 4, None) == -2
    assert L.qkv_tq3_dequant(p16, p16 + 8, 4, None) == -4
    assert L.qkv_q8_append(p16, p16, -5, None) == -1
    assert L.qkv_q8_dequant(None, p16, 1, None) == -2
    assert L.qkv_tq3_init(-1) == -1
