"""ctypes wrapper of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker.  The product path
(qengine_amd) never imports this module.

Arrays are numpy; fp16 data travels as uint16 bit patterns (or numpy float16
viewed as uint16).  Block arrays use the structured dtypes BLOCK_TQ3 (52 B)
and BLOCK_Q8 (36 B), identical to the reference's block_tq3
(turboquant.cuh:73-77) and block_q8_0_aligned (quant_gemv.cuh:19).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

BLOCK_TQ3 = np.dtype([("norm", "<f4"), ("qs", "u1", (48,))])
BLOCK_Q8 = np.dtype([("qs", "i1", (32,)), ("pad", "<u2"), ("d", "<u2")])
assert BLOCK_TQ3.itemsize == 52 and BLOCK_Q8.itemsize == 36

KV_TQ3, KV_Q8, KV_F16 = 0, 1, 2

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float


def _declare(L):
    L.or_f16_to_f32.restype = _F
    L.or_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.or_f32_to_f16.restype = ctypes.c_uint16
    L.or_f32_to_f16.argtypes = [_F]
    L.or_f16_to_f32_n.argtypes = [_P, _P, _I64]
    L.or_f32_to_f16_n.argtypes = [_P, _P, _I64]
    L.or_tq3_signs.argtypes = [_P]
    L.or_tq3_centroids.argtypes = [_P]
    L.or_tq3_bounds.argtypes = [_P]
    L.or_tq3_wht_scale.restype = _F
    L.or_wht128.argtypes = [_P]
    L.or_tq3_find_bin.restype = ctypes.c_uint8
    L.or_tq3_find_bin.argtypes = [_F]
    L.or_tq3_prescale_threshold_mismatches.restype = _I64
    L.or_tq3_prescale_threshold_mismatches.argtypes = [_P, _I64, _I64, _I, _I]
    L.or_tq3_fold_mismatches.restype = _I64
    L.or_tq3_fold_mismatches.argtypes = [ctypes.c_uint32, _P, _I64, _I64, _I, _I]
    L.or_pack_3bit_8.argtypes = [_P, _P]
    L.or_unpack_3bit_8.argtypes = [_P, _P]
    L.or_tq3_encode.argtypes = [_P, _P, _I64, _I]
    L.or_tq3_encode_rotated.argtypes = [_P, _P, _P, _I64]
    L.or_tq3_decode.argtypes = [_P, _P, _I64, _I]
    L.or_tq3_decode_f32.argtypes = [_P, _P, _I64]
    L.or_q8_encode.argtypes = [_P, _P, _I64, _I]
    L.or_q8_decode.argtypes = [_P, _P, _I64, _I]
    L.or_attn_split.argtypes = [_I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I,
                                _F, _I, _I, _I, _P, _I]
    L.or_attn_split_merge.argtypes = [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I]
    L.or_attn_ref_f64.argtypes = [_P, _P, _P, _P, _I, _I, _I, _I, _I, ctypes.c_double,
                                  _I, _I, _P]
    L.or_attn_ref_f64_f32kv.argtypes = [_P, _P, _P, _P, _I, _I, _I, _I, _I, ctypes.c_double,
                                  _I, _I, _P]
    L.or_key_visible.restype = _I
    L.or_key_visible.argtypes = [_I, _I, _I, _I, _I, _P]
    L.or_dfk2_dequant.argtypes = [_P, _P, _P, _I64, _I]
    L.or_tq3_kpool_update.argtypes = [_P, _P, _P, _I, _I, _I, _I, _I, _I]
    L.or_block_index_ms.argtypes = [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _F]
    L.or_block_scores_ms.argtypes = [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _F]
    L.or_attn_block_sparse_split.argtypes = [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I,
                                             _F, _I, _I, _I, _P]
    L.or_legacy_decode.restype = _I
    L.or_legacy_decode.argtypes = [_I, _I, _I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F]


def _ptr(a):
    return None if a is None else a.ctypes.data


def _u16(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.float16:
        a = a.view(np.uint16)
    assert a.dtype == np.uint16, a.dtype
    return a


# ---- scalar / constants -------------------------------------------------

def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = _u16(h)
    out = np.empty(h.shape, np.float32)
    lib().or_f16_to_f32_n(_ptr(h), _ptr(out), h.size)
    return out


def f32_to_f16(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().or_f32_to_f16_n(_ptr(f), _ptr(out), f.size)
    return out


def tq3_signs() -> np.ndarray:
    out = np.empty(128, np.float32)
    lib().or_tq3_signs(_ptr(out))
    return out


def tq3_centroids() -> np.ndarray:
    out = np.empty(8, np.float32)
    lib().or_tq3_centroids(_ptr(out))
    return out


def tq3_bounds() -> np.ndarray:
    out = np.empty(7, np.float32)
    lib().or_tq3_bounds(_ptr(out))
    return out


def wht_scale() -> float:
    return float(np.float32(lib().or_tq3_wht_scale()))


def wht128(x: np.ndarray) -> np.ndarray:
    x = np.array(x, dtype=np.float32, copy=True).reshape(-1, 128)
    for row in x:
        lib().or_wht128(row.ctypes.data)
    return x


def find_bin(v: np.ndarray) -> np.ndarray:
    v = np.asarray(v, np.float32).ravel()
    return np.array([lib().or_tq3_find_bin(float(x)) for x in v], np.uint8)


def fold_mismatches(a_bits: int, q_bits, lo: int = 0, hi: int = 0xFFFFFFFF,
                    negated: bool = False, nthreads: int = 0) -> int:
    """Number of reachable fp32 patterns w in [lo, hi] (w = +-0 or
    2^-67 <= |w| < 2^100) where the sign-folded binning (y = fl(-A w + |w|),
    bin = 4 + m or 3 - m by the sign of y, m = #{j: |y| > q_j}) differs from
    binning fl(w * rs); `negated` checks a lane holding -w."""
    q = np.ascontiguousarray(q_bits, np.uint32)
    assert q.size == 3 and 0 <= lo <= hi <= 0xFFFFFFFF
    return int(lib().or_tq3_fold_mismatches(a_bits, _ptr(q), lo, hi, int(negated), nthreads))


def prescale_threshold_mismatches(thr_bits, lo: int = 0, hi: int = 0xFFFFFFFF,
                                  negated: bool = False, nthreads: int = 0) -> int:
    """Number of fp32 bit patterns w in [lo, hi] (default: all 2^32) where
    binning fl(w * rs) per the reference differs from counting the thresholds
    below w; with `negated` the pattern holds -w and the bin is 7 minus the
    count (NaN patterns skipped)."""
    t = np.ascontiguousarray(thr_bits, np.uint32)
    assert t.size == 7 and 0 <= lo <= hi <= 0xFFFFFFFF
    return int(lib().or_tq3_prescale_threshold_mismatches(_ptr(t), lo, hi, int(negated),
                                                          nthreads))


def pack_3bit_8(idx8: np.ndarray) -> np.ndarray:
    idx8 = np.ascontiguousarray(idx8, np.uint8)
    out = np.zeros(3, np.uint8)
    lib().or_pack_3bit_8(_ptr(out), _ptr(idx8))
    return out


def unpack_3bit_8(b3: np.ndarray) -> np.ndarray:
    b3 = np.ascontiguousarray(b3, np.uint8)
    out = np.zeros(8, np.uint8)
    lib().or_unpack_3bit_8(_ptr(b3), _ptr(out))
    return out


# ---- codecs --------------------------------------------------------------

def tq3_encode(x_f16: np.ndarray, nthreads: int = 0) -> np.ndarray:
    x = _u16(x_f16).reshape(-1)
    assert x.size % 128 == 0
    n = x.size // 128
    out = np.zeros(n, BLOCK_TQ3)
    lib().or_tq3_encode(_ptr(x), _ptr(out), n, nthreads)
    return out


def tq3_encode_rotated(x_f16: np.ndarray):
    x = _u16(x_f16).reshape(-1)
    n = x.size // 128
    out = np.zeros(n, BLOCK_TQ3)
    rot = np.zeros((n, 128), np.float32)
    lib().or_tq3_encode_rotated(_ptr(x), _ptr(out), _ptr(rot), n)
    return out, rot


def tq3_decode(blocks: np.ndarray, nthreads: int = 0) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks).view(BLOCK_TQ3).reshape(-1)
    out = np.empty(blocks.size * 128, np.uint16)
    lib().or_tq3_decode(_ptr(blocks), _ptr(out), blocks.size, nthreads)
    return out


def tq3_decode_f32(blocks: np.ndarray) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks).view(BLOCK_TQ3).reshape(-1)
    out = np.empty(blocks.size * 128, np.float32)
    lib().or_tq3_decode_f32(_ptr(blocks), _ptr(out), blocks.size)
    return out


def q8_encode(x_f16: np.ndarray, nthreads: int = 0) -> np.ndarray:
    x = _u16(x_f16).reshape(-1)
    assert x.size % 32 == 0
    n = x.size // 32
    out = np.zeros(n, BLOCK_Q8)
    lib().or_q8_encode(_ptr(x), _ptr(out), n, nthreads)
    return out


def q8_decode(blocks: np.ndarray, nthreads: int = 0) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks).view(BLOCK_Q8).reshape(-1)
    out = np.empty(blocks.size * 32, np.uint16)
    lib().or_q8_decode(_ptr(blocks), _ptr(out), blocks.size, nthreads)
    return out


# ---- attention -------------------------------------------------------------

def attn_split(kind, q, k, v, *, num_q, num_kv, hd, start_pos, sub_n, sub_n_max,
               active_end_max, scale, k_splits, sink_tok=0, window_tok=0,
               tree_mask=None, nthreads=0):
    """attention.cuh:1905-2177 / 2633-2801.  Returns (part_m, part_l, part_o)."""
    q = _u16(q)
    k = np.ascontiguousarray(k)
    v = np.ascontiguousarray(v)
    pm = np.full((num_q, sub_n_max, k_splits), np.nan, np.float32)
    pl = np.full((num_q, sub_n_max, k_splits), np.nan, np.float32)
    po = np.full((num_q, sub_n_max, k_splits, hd), np.nan, np.float32)
    tm = None if tree_mask is None else np.ascontiguousarray(tree_mask, np.uint32)
    lib().or_attn_split(kind, _ptr(q), _ptr(k), _ptr(v), _ptr(pm), _ptr(pl), _ptr(po),
                        num_q, num_kv, hd, start_pos, sub_n, sub_n_max, active_end_max,
                        float(scale), k_splits, sink_tok, window_tok, _ptr(tm), nthreads)
    return pm, pl, po


def attn_split_merge(pm, pl, po, *, num_q, num_kv, hd, sub_n, sub_n_max, k_splits):
    """attention.cuh:1837-1891.  Returns fp16 bits [sub_n][num_q][hd]."""
    pm = np.ascontiguousarray(pm, np.float32)
    pl = np.ascontiguousarray(pl, np.float32)
    po = np.ascontiguousarray(po, np.float32)
    out = np.zeros((sub_n, num_q, hd), np.uint16)
    lib().or_attn_split_merge(_ptr(pm), _ptr(pl), _ptr(po), _ptr(out), num_q, num_kv, hd,
                              sub_n, sub_n_max, k_splits)
    return out


def attn_ref_f64(q, k_f16, v_f16, *, num_q, num_kv, hd, start_pos, sub_n, scale,
                 sink_tok=0, window_tok=0, tree_mask=None):
    q = _u16(q)
    k_f16 = _u16(k_f16)
    v_f16 = _u16(v_f16)
    out = np.zeros((sub_n, num_q, hd), np.float64)
    tm = None if tree_mask is None else np.ascontiguousarray(tree_mask, np.uint32)
    lib().or_attn_ref_f64(_ptr(q), _ptr(k_f16), _ptr(v_f16), _ptr(out), num_q, num_kv, hd,
                          start_pos, sub_n, float(scale), sink_tok, window_tok, _ptr(tm))
    return out


def attn_exact_tq3(q, k_tq3, v_tq3, *, num_q, num_kv, hd, start_pos, sub_n, scale,
                   sink_tok=0, window_tok=0, tree_mask=None):
    """fp64 attention over the EXACT dequantization of TQ3 caches
    (norm * rs * sign * (H c), turboquant.cuh:169-200 without its final fp16
    rounding; tq3_decode_f32), same visibility rules as attn_ref_f64.  The
    reference's own numerics round every dequantized element to fp16; this is
    the mathematical value both approximate.  Returns [sub_n][num_q][hd]."""
    return attn_ref_f64_f32kv(q, tq3_decode_f32(k_tq3), tq3_decode_f32(v_tq3), num_q=num_q,
                              num_kv=num_kv, hd=hd, start_pos=start_pos, sub_n=sub_n,
                              scale=scale, sink_tok=sink_tok, window_tok=window_tok,
                              tree_mask=tree_mask)


def attn_ref_f64_f32kv(q, k_f32, v_f32, *, num_q, num_kv, hd, start_pos, sub_n, scale,
                       sink_tok=0, window_tok=0, tree_mask=None):
    """attn_ref_f64 over float K/V rows [n][num_kv][hd] (same core)."""
    q = _u16(q)
    k = np.ascontiguousarray(k_f32, np.float32)
    v = np.ascontiguousarray(v_f32, np.float32)
    out = np.zeros((sub_n, num_q, hd), np.float64)
    tm = None if tree_mask is None else np.ascontiguousarray(tree_mask, np.uint32)
    lib().or_attn_ref_f64_f32kv(_ptr(q), _ptr(k), _ptr(v), _ptr(out), num_q, num_kv, hd,
                                start_pos, sub_n, float(scale), sink_tok, window_tok, _ptr(tm))
    return out


def attn_q8k_tq3v_f64(q, k_q8, v_tq3, *, num_q, num_kv, hd, start_pos, sub_n, scale):
    """V-only TurboQuant decode (TQ_KEYS_Q8, model.cuh:2574-2588): keys
    dequantized from Q8_0 to fp16 (dequantize_kv_q8_0_kern,
    attention.cuh:2614-2626) for attn_score_kernel_h, values decoded from TQ3
    in fp32 as attn_value_kernel_tq3 does (attention.cuh:920-989); query t
    attends keys 0 .. start_pos + t; softmax and sums in float64.
    Returns [sub_n][num_q][hd] float64."""
    k = f16_to_f32(q8_decode(k_q8)).astype(np.float64).reshape(-1, num_kv, hd)
    v = tq3_decode_f32(v_tq3).astype(np.float64).reshape(-1, num_kv, hd)
    qf = f16_to_f32(_u16(q)).astype(np.float64).reshape(sub_n, num_q, hd)
    gqa = num_q // num_kv
    out = np.zeros((sub_n, num_q, hd))
    for t in range(sub_n):
        n = start_pos + t + 1
        for h in range(num_kv):
            s = qf[t, h * gqa:(h + 1) * gqa] @ k[:n, h].T * scale     # [gqa][n]
            w = np.exp(s - s.max(axis=1, keepdims=True))
            out[t, h * gqa:(h + 1) * gqa] = (w @ v[:n, h]) / w.sum(axis=1, keepdims=True)
    return out


def legacy_decode(k_kind, v_kind, q, k, v, *, num_q, num_kv, hd, seq_len, scale,
                  tq_fused=False, return_probs=False):
    """The reference's short-context decode (model.cuh:2544-2664) of one query
    token over cache rows 0 .. seq_len-1: K and V dequantized to an fp16
    scratch, attn_score_kernel_h, softmax_kernel (sum + 1e-10),
    attn_value_kernel_h (attention.cuh:277-316, 531-575, 885-907); with
    tq_fused, TQ3 operands go through attn_score_kernel_tq3 /
    attn_value_kernel_tq3 (attention.cuh:400-483, 920-989).  q [1][num_q][hd]
    or [num_q][hd] fp16; k / v in the layout of their kind (KV_TQ3 blocks,
    KV_Q8 blocks, KV_F16 fp16 rows).  Returns fp16 bits [num_q][hd] (and the
    softmax rows [num_q][seq_len] float32 when return_probs)."""
    qq = _u16(q).reshape(num_q, hd)
    kk = np.ascontiguousarray(k)
    vv = np.ascontiguousarray(v)
    out = np.zeros((num_q, hd), np.uint16)
    probs = np.zeros((num_q, seq_len), np.float32)
    rc = lib().or_legacy_decode(k_kind, v_kind, int(bool(tq_fused)), _ptr(qq), _ptr(kk), _ptr(vv),
                                _ptr(out), _ptr(probs), num_q, num_kv, hd, seq_len, float(scale))
    if rc != 0:
        raise ValueError("legacy_decode: unsupported shape")
    return (out, probs) if return_probs else out


def dfk2_dequant(q_i8, scales_f16, kv_dim):
    """dfki2_dequant_kernel (model.cuh:149-159): int8 rows [n_rows][kv_dim]
    with fp16 scales [n_rows][kv_dim / 128] to fp16 bits of the same shape."""
    q = np.ascontiguousarray(q_i8, np.int8)
    s = _u16(scales_f16)
    out = np.zeros(q.shape, np.uint16)
    lib().or_dfk2_dequant(_ptr(q), _ptr(s), _ptr(out), q.size, kv_dim)
    return out


def tq3_kpool_update(k_tq3, k_pool, k_pool_max, *, num_kv, hd, total_kv, blk_lo,
                     block_size_n=64):
    """tq3_kpool_ms_update_kern (attention.cuh:2445-2533), in place on the fp16
    pools [num_kv][n_blocks_stride][hd] (uint16 bits): blocks blk_lo ..
    ceil(total_kv / block_size_n) - 1 get the mean / signed max-abs of their
    dequantized K rows."""
    assert k_pool.dtype == np.uint16 and k_pool_max.dtype == np.uint16
    assert k_pool.flags.c_contiguous and k_pool_max.flags.c_contiguous
    stride = k_pool.shape[1]
    lib().or_tq3_kpool_update(_ptr(np.ascontiguousarray(k_tq3)), _ptr(k_pool), _ptr(k_pool_max),
                              num_kv, hd, total_kv, blk_lo, stride, block_size_n)


def block_index_ms(q, k_pool, k_pool_max, *, num_q, num_kv, hd, sub_n, sub_n_max, start_pos,
                   top_k, n_blocks, block_size_n=64, beta=0.5):
    """build_block_index_ms_kern (sparse_attn/sparse_index.cuh:214-330):
    int32 [num_kv][sub_n_max][top_k], rows sorted ascending, -1 padded."""
    qq = _u16(q)
    out = np.full((num_kv, sub_n_max, top_k), -1, np.int32)
    lib().or_block_index_ms(_ptr(qq), _ptr(_u16(k_pool)), _ptr(_u16(k_pool_max)), _ptr(out),
                            num_q, num_kv, hd, sub_n, sub_n_max, start_pos, top_k, block_size_n,
                            n_blocks, k_pool.shape[1], float(beta))
    return out


def block_scores_ms(q, k_pool, k_pool_max, *, num_q, num_kv, hd, sub_n, start_pos, n_blocks,
                    block_size_n=64, beta=0.5):
    """The block scores build_block_index_ms_kern selects from
    (sparse_attn/sparse_index.cuh:243-290): float32 [num_kv][sub_n][n_blocks],
    -inf past each query's causal block."""
    out = np.zeros((num_kv, sub_n, n_blocks), np.float32)
    lib().or_block_scores_ms(_ptr(_u16(q)), _ptr(_u16(k_pool)), _ptr(_u16(k_pool_max)), _ptr(out),
                             num_q, num_kv, hd, sub_n, start_pos, block_size_n, n_blocks,
                             k_pool.shape[1], float(beta))
    return out


def attn_block_sparse_split(q, k_tq3, v_tq3, block_index, *, num_q, num_kv, hd, start_pos, sub_n,
                            sub_n_max, scale, top_k, k_splits, block_size_n=64, tree_mask=None):
    """flash_attn_chunk_block_sparse_split_tq3 (attention.cuh:2193-2433):
    partials (m, l, o) in the split layout; merge with attn_split_merge."""
    qq = _u16(q)
    pm = np.zeros((num_q, sub_n_max, k_splits), np.float32)
    pl = np.zeros_like(pm)
    po = np.zeros((num_q, sub_n_max, k_splits, hd), np.float32)
    tm = None if tree_mask is None else np.ascontiguousarray(tree_mask, np.uint32)
    bi = np.ascontiguousarray(block_index, np.int32)
    lib().or_attn_block_sparse_split(_ptr(qq), _ptr(np.ascontiguousarray(k_tq3)),
                                     _ptr(np.ascontiguousarray(v_tq3)), _ptr(bi), _ptr(pm),
                                     _ptr(pl), _ptr(po), num_q, num_kv, hd, start_pos, sub_n,
                                     sub_n_max, float(scale), top_k, block_size_n, k_splits,
                                     _ptr(tm))
    return pm, pl, po


def key_visible(key, start_pos, t_idx, sink_tok=0, window_tok=0, tree_mask=None):
    tm = None if tree_mask is None else np.ascontiguousarray(tree_mask, np.uint32)
    return bool(lib().or_key_visible(key, start_pos, t_idx, sink_tok, window_tok, _ptr(tm)))


# ---- paged caches ------------------------------------------------------------
# The reference keeps each slot contiguous from kv_slot_offset(slot)
# (model.cuh:1708-1715) and hands attention a slot-base pointer
# (model.cuh:2466-2468).  A per-slot block table generalises that offset per
# block_tokens keys; gathering a slot's rows and running the contiguous
# reference decode on them is the paged decode's definition.

def move_token_rows(cache_rows: np.ndarray, moves, slot_row0: int = 0) -> np.ndarray:
    """kv_move_token (model.cuh:7430-7471) applied per move in list order, as
    the reference's sequence of device copies: row slot_row0 + to := row
    slot_row0 + from.  cache_rows: [rows][row_bytes] uint8 (K or V of one
    layer).  Returns a new array."""
    out = np.array(cache_rows, copy=True)
    for f, t in moves:
        if f != t:
            out[slot_row0 + t] = out[slot_row0 + f]
    return out


def paged_rows(block_table, n_keys, block_tokens):
    """Cache rows of keys 0..n_keys-1 of one slot."""
    k = np.arange(n_keys, dtype=np.int64)
    bt = np.asarray(block_table, np.int64)
    return bt[k // block_tokens] * block_tokens + k % block_tokens


def gather_rows(pool_blocks, rows, blocks_per_row):
    """Blocks of the given token rows, in row order ([len(rows)*blocks_per_row])."""
    idx = np.asarray(rows, np.int64)[:, None] * blocks_per_row + np.arange(blocks_per_row)
    return np.ascontiguousarray(pool_blocks[idx.reshape(-1)])


def decode_paged(kind, q, k_pool, v_pool, block_tables, ctx_lens, *, num_q, num_kv, hd,
                 block_tokens, scale, k_splits=8):
    """One decode query per slot (q [n_slots][num_q][hd]) over its gathered rows:
    the reference split decode + merge with start_pos = ctx - 1, sub_n = 1.
    A slot without keys gives a zero row.  Returns fp16 bits."""
    q = _u16(q)
    bpr = num_kv * hd // 128
    out = np.zeros((q.shape[0], num_q, hd), np.uint16)
    for s, ctx in enumerate(ctx_lens):
        ctx = int(ctx)
        if ctx <= 0:
            continue
        rows = paged_rows(block_tables[s], ctx, block_tokens)
        kb = gather_rows(k_pool, rows, bpr)
        vb = gather_rows(v_pool, rows, bpr)
        ks = min(k_splits, ctx)
        pm, pl, po = attn_split(kind, q[s:s + 1], kb, vb, num_q=num_q, num_kv=num_kv, hd=hd,
                                start_pos=ctx - 1, sub_n=1, sub_n_max=1, active_end_max=ctx,
                                scale=scale, k_splits=ks)
        out[s] = attn_split_merge(pm, pl, po, num_q=num_q, num_kv=num_kv, hd=hd, sub_n=1,
                                  sub_n_max=1, k_splits=ks)[0]
    return out
