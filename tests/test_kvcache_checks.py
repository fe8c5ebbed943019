"""Host-side buffer checks of qengine_amd.kvcache (CPU only).

The kernels trust the sizes implied by the shape arguments (a write path such
as decode_attn_q8_append stores the new token into row start_pos of the
caches), so the torch wrappers reject undersized or mistyped buffers with
ValueError before anything is launched.  The checks run ahead of the device
checks, so CPU tensors exercise them here without a GPU."""
import pytest
import torch

from qengine_amd import kvcache as K

NQ, NKV, HD = 16, 4, 256


def _f16(n):
    return torch.zeros(n, dtype=torch.float16)


def _u8(n):
    return torch.zeros(n, dtype=torch.uint8)


def _q8_cache(rows):
    return _u8(rows * NKV * K.Q8_ROW)


def _tq3_cache(rows):
    return _u8(rows * NKV * K.TQ3_ROW)


def test_q8_append_rejects_cache_without_the_new_row():
    start = 100
    q, out = _f16(NQ * HD), _f16(NQ * HD)
    knew, vnew = _f16(NKV * HD), _f16(NKV * HD)
    ws = _u8(1 << 16)
    # caches sized to the tokens already cached: row start_pos is missing
    with pytest.raises(ValueError, match="k holds"):
        K.decode_attn_q8_append(q, knew, vnew, _q8_cache(start), _q8_cache(start + 1), out, ws,
                                num_q=NQ, num_kv=NKV, start_pos=start, scale=0.0625)
    with pytest.raises(ValueError, match="v holds"):
        K.decode_attn_q8_append(q, knew, vnew, _q8_cache(start + 1), _q8_cache(start), out, ws,
                                num_q=NQ, num_kv=NKV, start_pos=start, scale=0.0625)
    with pytest.raises(ValueError, match="k_new"):
        K.decode_attn_q8_append(q, _f16(NKV * HD - 1), vnew, _q8_cache(start + 1),
                                _q8_cache(start + 1), out, ws, num_q=NQ, num_kv=NKV,
                                start_pos=start, scale=0.0625)
    with pytest.raises(ValueError, match="v_new must be"):
        K.decode_attn_q8_append(q, knew, vnew.float(), _q8_cache(start + 1), _q8_cache(start + 1),
                                out, ws, num_q=NQ, num_kv=NKV, start_pos=start, scale=0.0625)


@pytest.mark.parametrize("fn,kc,vc", [
    (K.decode_attn_tq3, _tq3_cache, _tq3_cache),
    (K.decode_attn_q8, _q8_cache, _q8_cache),
    (K.decode_attn_q8k_tq3v, _q8_cache, _tq3_cache),
])
def test_decode_rejects_short_caches_and_outputs(fn, kc, vc):
    start, sub_n = 500, 4
    n = start + sub_n
    q, out = _f16(sub_n * NQ * HD), _f16(sub_n * NQ * HD)
    ws = _u8(1 << 16)
    kw = dict(num_q=NQ, num_kv=NKV, start_pos=start, sub_n=sub_n, scale=0.0625)
    with pytest.raises(ValueError, match="k holds"):
        fn(q, kc(n - 1), vc(n), out, ws, **kw)
    with pytest.raises(ValueError, match="v holds"):
        fn(q, kc(n), vc(n - 1), out, ws, **kw)
    with pytest.raises(ValueError, match="out holds"):
        fn(q, kc(n), vc(n), _f16(sub_n * NQ * HD - 8), ws, **kw)
    with pytest.raises(ValueError, match="q must be"):
        fn(q.float(), kc(n), vc(n), out, ws, **kw)


def test_noalloc_decode_rejects_short_cache():
    q, out = _f16(NQ * HD), _f16(NQ * HD)
    with pytest.raises(ValueError, match="k holds"):
        K.decode_attn_tq3_noalloc(q, _tq3_cache(63), _tq3_cache(64), out, num_q=NQ, num_kv=NKV,
                                  start_pos=63, sub_n=1, scale=0.0625)


@pytest.mark.parametrize("fn", [K.kv_gather_rows, K.kv_scatter_rows])
def test_row_copies_reject_short_flat_buffers(fn):
    rows, bt, kr, vr = 300, 256, 416, 416
    pool_k, pool_v = _u8(1024 * kr), _u8(1024 * vr)
    table = torch.zeros(2, dtype=torch.int32)
    kw = dict(n_rows=rows, block_tokens=bt, k_row_bytes=kr, v_row_bytes=vr)
    with pytest.raises(ValueError, match="k_flat holds"):
        fn(pool_k, pool_v, _u8(rows * kr - 1), _u8(rows * vr), table, **kw)
    with pytest.raises(ValueError, match="v_flat holds"):
        fn(pool_k, pool_v, _u8(rows * kr), _u8(rows * vr - 16), table, **kw)
    with pytest.raises(ValueError, match="v_flat is required"):
        fn(pool_k, pool_v, _u8(rows * kr), None, table, **kw)
    with pytest.raises(ValueError, match="block_table holds"):
        fn(pool_k, pool_v, _u8(rows * kr), _u8(rows * vr), table[:1], **kw)
    with pytest.raises(ValueError, match="block_table must be"):
        fn(pool_k, pool_v, _u8(rows * kr), _u8(rows * vr), table.to(torch.int64), **kw)
