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


def test_bench_library_exports_its_header():
    """The benchmark's streaming read and MFMA loop live in libqkv_bench.so
    (include/qkv_bench.h), not in the product library."""
    B = _lib.bench_lib()
    names = _lib.header_functions(_lib.BENCH_HEADER_PATH)
    assert names == ["qkv_hbm_read_bench", "qkv_mfma_rate_bench"]
    for n in names:
        assert hasattr(B, n) and n in _lib.BENCH_SIGNATURES
        assert not hasattr(_lib.lib(), n), f"libqkv.so still exports {n}"
    buf = ctypes.create_string_buffer(256)
    p = (ctypes.addressof(buf) + 63) & ~63
    assert B.qkv_hbm_read_bench(p, 0, p, None) == 0          # nothing to read
    assert B.qkv_hbm_read_bench(p, 48, p, None) == -1        # multiples of 64 bytes
    assert B.qkv_hbm_read_bench(None, 64, p, None) == -2
    assert B.qkv_hbm_read_bench(p + 4, 64, p, None) == -4
    assert B.qkv_mfma_rate_bench(0, 1, p, None) == -1        # no workgroup: refused, nothing launched
    assert B.qkv_mfma_rate_bench(1, 0, p, None) == -1
    assert B.qkv_mfma_rate_bench(1, 1, None, None) == -2
    assert B.qkv_mfma_rate_bench(1, 1, p + 2, None) == -4


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


def test_paged_argument_errors_without_gpu(L):
    buf = ctypes.create_string_buffer(1 << 16)
    p = (ctypes.addressof(buf) + 255) & ~255
    ws_n = L.qkv_decode_attn_tq3_paged_workspace_bytes(16, 4, 2, 1000)
    assert ws_n > 0
    assert L.qkv_decode_attn_tq3_paged_workspace_bytes(16, 4, 0, 1000) == 0

    def dec(**kw):
        a = dict(q=p, k=p, v=p, out=p, num_q=16, num_kv=4, hd=256, n_slots=2, bt=p, max_blocks=4,
                 block_tokens=256, pool_rows=1024, ctx=p, max_ctx=1000, scale=0.0625, ws=p,
                 ws_bytes=ws_n)
        a.update(kw)
        return L.qkv_decode_attn_tq3_paged(a["q"], a["k"], a["v"], a["out"], a["num_q"],
                                           a["num_kv"], a["hd"], a["n_slots"], a["bt"],
                                           a["max_blocks"], a["block_tokens"], a["pool_rows"],
                                           a["ctx"], a["max_ctx"], a["scale"], a["ws"],
                                           a["ws_bytes"], None)
    assert dec(block_tokens=100) == -3          # block size must be a multiple of 64
    assert dec(block_tokens=32) == -3
    assert dec(max_ctx=2000) == -1              # max_ctx beyond max_blocks * block_tokens
    assert dec(n_slots=0) == -1
    assert dec(hd=128) == -3
    assert dec(num_q=40) == -3                  # GQA 10 is not instantiated
    assert dec(bt=None) == -2
    assert dec(ctx=None) == -2
    assert dec(ws_bytes=ws_n - 1) == -7
    assert dec(q=p + 2) == -4
    assert dec(ws=p + 4) == -4

    def app(**kw):
        a = dict(k=p, v=p, kp=p, vp=p, n_slots=2, n_tok=1, num_kv=4, hd=256, bt=p, max_blocks=4,
                 block_tokens=256, pool_rows=1024, pos=p)
        a.update(kw)
        return L.qkv_tq3_append_kv_paged(a["k"], a["v"], a["kp"], a["vp"], a["n_slots"],
                                         a["n_tok"], a["num_kv"], a["hd"], a["bt"],
                                         a["max_blocks"], a["block_tokens"], a["pool_rows"],
                                         a["pos"], None)
    assert app(n_slots=0) == 0                  # nothing to append
    assert app(n_tok=-1) == -1
    assert app(hd=64) == -3
    assert app(pos=None) == -2
    assert app(k=p + 8) == -4


def test_kv_move_tokens_argument_errors_without_gpu(L):
    buf = ctypes.create_string_buffer(4096)
    p = (ctypes.addressof(buf) + 15) & ~15
    pairs = (ctypes.c_int32 * 4)(0, 1, 2, 3)
    pp = ctypes.cast(pairs, ctypes.c_void_p)
    assert L.qkv_kv_move_tokens(p, p, 416, 416, 0, 8, pp, 0, None) == 0       # empty list
    assert L.qkv_kv_move_tokens(p, p, 416, 416, 0, 8, pp, -1, None) == -1
    assert L.qkv_kv_move_tokens(p, p, 416, 416, 0, 8, pp, 65, None) == -1     # more than 64 moves
    assert L.qkv_kv_move_tokens(None, p, 416, 416, 0, 8, pp, 2, None) == -2
    assert L.qkv_kv_move_tokens(p, p, 416, 416, 0, 8, None, 2, None) == -2
    assert L.qkv_kv_move_tokens(p, p, 418, 416, 0, 8, pp, 2, None) == -1      # rows of whole dwords
    assert L.qkv_kv_move_tokens(p, p, 416, 416, 0, 3, pp, 2, None) == -1      # row 3 outside 3 rows
    assert L.qkv_kv_move_tokens(p, p, 416, 416, -1, 8, pp, 2, None) == -1
    assert L.qkv_kv_move_tokens(p + 2, p, 416, 416, 0, 8, pp, 2, None) == -4


def test_decode_workspace_for_the_longest_call_covers_shorter_ones(L):
    """The fast path's chunk size grows with the key count (one round of
    workgroups), so its record area is not monotone in the length (16,384 Q8
    keys take 128 chunks, 16,385 take 65; one TQ3 query over 65,536 keys takes
    64, over 65,537 keys 43; a 16-query TQ3 verify over 32,768 keys 64, over
    32,833 keys 33); a workspace sized for the longest call must still cover
    every shorter one.  The chunk count moves only at whole 64-key tiles, so
    every tile boundary and the key after it are checked."""
    queries = [L.qkv_decode_attn_tq3_workspace_bytes, L.qkv_decode_attn_q8_workspace_bytes]
    for num_q, num_kv in [(16, 4), (24, 4), (16, 16), (8, 4)]:
        for sub_n in (1, 16):
            for query in queries:
                for n_max in (16385, 32833, 40000, 65537):
                    top = query(num_q, num_kv, sub_n, n_max)
                    assert top > 0
                    for n in range(64, n_max, 64):
                        for m in (n, n + 1):
                            if sub_n <= m <= n_max:
                                assert query(num_q, num_kv, sub_n, m) <= top, \
                                    (query.__name__, num_q, num_kv, sub_n, m, n_max)
    # the sizes themselves: header 256 B, 16 B per record row rounded to
    # 256 B, 1 KiB of fp32 output per record row; rows = queries x slots
    def size(num_q, sub_n, slots):
        rows = num_q * sub_n * slots
        return 256 + ((rows * 16 + 255) & ~255) + rows * 1024
    # one query over 65,536 keys: 64 chunks of 1,024; 65,537 keys take 43
    # chunks of 1,536, but a workspace for them still holds 64
    assert L.qkv_decode_attn_tq3_workspace_bytes(16, 4, 1, 65536) == size(16, 1, 64)
    assert L.qkv_decode_attn_tq3_workspace_bytes(16, 4, 1, 65537) == size(16, 1, 64)
    # 16-token verify (64 query-head columns, one workgroup per chunk): 32,768
    # keys and 32,784 (a last 16-key tile joined) take 64 chunks of 512 keys;
    # 32,833 keys take 33 chunks of 1,024, and a workspace for them holds 64
    for n in (32768, 32784, 32833):
        assert L.qkv_decode_attn_tq3_workspace_bytes(16, 4, 16, n) == size(16, 16, 64)
    assert L.qkv_decode_attn_q8_workspace_bytes(16, 4, 1, 16384) == size(16, 1, 128)
    assert L.qkv_decode_attn_q8_workspace_bytes(16, 4, 1, 16385) == size(16, 1, 128)


def test_mixed_decode_argument_errors_without_gpu(L):
    """Q8_0-key / TQ3-value decode: the Q8 decode's workspace size and error
    order (shape, then pointers, alignment, workspace); no call reaches a launch."""
    buf = ctypes.create_string_buffer(4096)
    p = (ctypes.addressof(buf) + 255) & ~255
    n = L.qkv_decode_attn_q8k_tq3v_workspace_bytes(16, 4, 1, 4097)
    assert n == L.qkv_decode_attn_q8_workspace_bytes(16, 4, 1, 4097) > 0

    def call(q=p, hd=256, ws=p, wsb=n - 1, num_q=16):
        return L.qkv_decode_attn_q8k_tq3v(q, p, p, p, num_q, 4, hd, 4096, 1, 1 / 16, ws, wsb, None)
    assert call(q=None) == -2
    assert call(hd=128) in (-1, -3)
    assert call(num_q=18) in (-1, -3)          # 18 q heads over 4 kv heads
    assert call(q=p + 2) == -4
    assert call(ws=None) == -7
    assert call() == -7                        # one byte short


def test_workspace_health_argument_errors(L):
    buf = ctypes.create_string_buffer(4096)
    p = (ctypes.addressof(buf) + 255) & ~255
    assert L.qkv_decode_workspace_status(None, None) == -2
    assert L.qkv_decode_workspace_status(p + 4, None) == -4
    assert L.qkv_decode_workspace_reset(None, 256, None) == -2
    assert L.qkv_decode_workspace_reset(p + 4, 256, None) == -4
    assert L.qkv_decode_workspace_reset(p, 6, None) == -4      # whole words only
    assert L.qkv_decode_workspace_reset(p, 0, None) == 0       # nothing to clear
    assert L.qkv_decode_workspace_status_async(None, p, None) == -2
    assert L.qkv_decode_workspace_status_async(p, None, None) == -2
    assert L.qkv_decode_workspace_status_async(p + 4, p, None) == -4
    assert L.qkv_decode_workspace_status_async(p, p + 2, None) == -4
    assert L.qkv_debug_set_merge_spin_limit(-1) == 0
    assert L.qkv_status_string(-8) == b"in-kernel merge timed out; reset the workspace"


def test_inject_and_page_copy_argument_errors_without_gpu(L):
    """DFK2 re-quantizing appends and paged snapshot copies: shape, pointer
    and alignment errors before any launch."""
    buf = ctypes.create_string_buffer(8192)
    p = (ctypes.addressof(buf) + 255) & ~255
    assert L.qkv_dfk2_dequant(p, p, p, 0, 1024, None) == 0
    assert L.qkv_dfk2_dequant(p, p, p, -8, 1024, None) == -1
    assert L.qkv_dfk2_dequant(p, p, p, 1024, 1000, None) == -3     # kv_dim not a multiple of 128
    assert L.qkv_dfk2_dequant(p, p, p, 1020, 1024, None) == -3
    assert L.qkv_dfk2_dequant(None, p, p, 1024, 1024, None) == -2
    assert L.qkv_dfk2_dequant(p + 4, p, p, 1024, 1024, None) == -4
    assert L.qkv_tq3_append_dfk2(p, p, p, 0, None) == 0
    assert L.qkv_tq3_append_dfk2(p, p, p, -1, None) == -1
    assert L.qkv_tq3_append_dfk2(p, None, p, 8, None) == -2
    assert L.qkv_tq3_append_dfk2(p + 8, p, p, 8, None) == -4
    assert L.qkv_q8_append_dfk2(p, p, p, 6, None) == -3            # 32-element blocks in fours
    assert L.qkv_q8_append_dfk2(p, p, None, 8, None) == -2
    assert L.qkv_q8_append_dfk2(p + 4, p, p, 8, None) == -4
    g = L.qkv_kv_gather_rows
    assert g(p, p, p, p, 416, 416, 100, p, 4, 16, 0, None) == 0
    assert g(p, p, p, p, 416, 416, 100, p, 4, 16, -1, None) == -1
    assert g(p, p, p, p, 418, 416, 100, p, 4, 16, 8, None) == -1     # rows of whole dwords
    assert g(p, p, p, p, 416, 416, 100, p, 4, 16, 65, None) == -1    # past the table's 4 blocks
    assert g(p, p, p, p, 416, 416, 100, p, 4, 0, 8, None) == -1
    assert g(p, None, p, p, 416, 416, 100, p, 4, 16, 8, None) == -2  # V pool without V buffer
    assert g(p, p, p, p, 416, 416, 100, None, 4, 16, 8, None) == -2
    assert g(p + 2, p, p, p, 416, 416, 100, p, 4, 16, 8, None) == -4
    assert L.qkv_kv_scatter_rows(p, p, None, p, 416, 416, 100, p, 4, 16, 8, None) == -2


def test_block_sparse_argument_errors_without_gpu(L):
    buf = ctypes.create_string_buffer(8192)
    p = (ctypes.addressof(buf) + 255) & ~255
    kp = L.qkv_tq3_kpool_update
    assert kp(p, p, p, 4, 256, 0, 0, 8, 64, None) == 0            # nothing to build
    assert kp(p, p, p, 4, 128, 100, 0, 8, 64, None) == -3
    assert kp(p, p, p, 4, 256, 100, 0, 8, 65, None) == -3          # blocks of at most 64 rows
    assert kp(p, p, p, 4, 256, 64 * 9, 0, 8, 64, None) == -1        # 9 blocks in a stride of 8
    assert kp(None, p, p, 4, 256, 100, 0, 8, 64, None) == -2
    assert kp(p, p + 1, p, 4, 256, 100, 0, 8, 64, None) == -4
    bi = L.qkv_block_index_ms
    wsb = L.qkv_block_index_ms_workspace_bytes(4, 1, 2)
    assert wsb == 256
    assert bi(p, p, p, p, 16, 4, 256, 2, 1, 100, 8, 64, 2, 2, 0.5, p, wsb, None) == -1   # sub_n > sub_n_max
    assert bi(p, p, p, p, 16, 4, 256, 1, 1, 100, 0, 64, 2, 2, 0.5, p, wsb, None) == -1   # top_k 0
    assert bi(p, p, p, p, 16, 4, 256, 1, 1, 100, 8, 64, 3, 2, 0.5, p, wsb, None) == -1   # n_blocks > stride
    assert bi(p, None, p, p, 16, 4, 256, 1, 1, 100, 8, 64, 2, 2, 0.5, p, wsb, None) == -2
    assert bi(p, p, p, p, 16, 4, 256, 1, 1, 100, 8, 64, 2, 2, 0.5, None, wsb, None) == -7
    # no cap on n_blocks beyond the workspace (the selection keeps nothing per block in LDS)
    assert bi(p, p, p, p, 16, 4, 256, 1, 1, 100, 8, 64, 40000, 40000, 0.5, p, wsb, None) == -7
    assert bi(p, p, p, p, 16, 4, 256, 1, 1, 100, 8, 64, 2, 2, 0.5, p, wsb - 1, None) == -7
    sp = L.qkv_attn_block_sparse_split_tq3
    assert sp(p, p, p, p, p, p, p, 16, 4, 256, 100, 1, 1, 1.0, 8, 32, 8, None, None) == -3
    assert sp(p, p, p, p, p, p, p, 16, 4, 256, 100, 1, 1, 1.0, 600, 64, 8, None, None) == -3
    assert sp(p, p, p, p, p, p, p, 16, 4, 256, 100, 1, 1, 1.0, 0, 64, 8, None, None) == -1
    assert sp(p, p, p, None, p, p, p, 16, 4, 256, 100, 1, 1, 1.0, 8, 64, 8, None, None) == -2
    assert sp(p + 8, p, p, p, p, p, p, 16, 4, 256, 100, 1, 1, 1.0, 8, 64, 8, None, None) == -4


def test_noalloc_health_argument_errors(L):
    # device numbers outside 0..63 are rejected before any HIP call
    buf = ctypes.create_string_buffer(64)
    st = (ctypes.addressof(buf) + 15) & ~15
    for dev in (-1, 64):
        assert L.qkv_decode_noalloc_status(dev, None) == -1
        assert L.qkv_decode_noalloc_reset(dev, None) == -1
        assert L.qkv_decode_noalloc_status_async(dev, st, None) == -1
    assert L.qkv_decode_noalloc_status_async(0, None, None) == -2
    assert L.qkv_decode_noalloc_status_async(0, st + 2, None) == -4


@pytest.mark.parametrize("lang,compiler,std", [("c", "gcc", "-std=c11"), ("c++", "g++", "-std=c++17")])
def test_header_compiles_as_c_and_cxx(lang, compiler, std):
    """include/qkv.h (through the compiled caller tests/c_caller/qkv_caller.c)
    is valid C11 and C++17 with warnings as errors."""
    import os
    import shutil
    import subprocess
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    rocm_inc = "/opt/rocm/include"
    if shutil.which(compiler) is None or not os.path.isdir(rocm_inc):
        pytest.skip(f"{compiler} or the HIP headers are not installed")
    cmd = [compiler, std, "-fsyntax-only", "-Wall", "-Wextra", "-Werror",
           "-I", os.path.join(root, "include"), "-isystem", rocm_inc, "-D__HIP_PLATFORM_AMD__",
           "-x", lang, os.path.join(root, "tests", "c_caller", "qkv_caller.c")]
    if lang == "c":
        cmd.insert(2, "-pedantic")
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
