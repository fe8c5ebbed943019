"""A verify block, or a decode step's token, appended inside the decode call
(qkv_decode_attn_tq3_append).
The reference encodes the block's K and V into the cache with
tq3_quantize_kernel and then runs the split attention and its merge
(model.cuh:4566-4571, 4663-4687).  Checked on identical seeded inputs: the
cache rows the call writes equal the oracle's encoding byte for byte, caches
and output equal those of qkv_tq3_append_kv followed by qkv_decode_attn_tq3
bit for bit, and the output meets the decode bar against the oracle."""
import numpy as np
import pytest

from oracle import oracle as O
from tests._data import assert_tq3_attn, kv_f16, q_f16

pytestmark = pytest.mark.gpu


def _dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


# (start_pos, num_q, sub_n, tree); num_kv 4, so sub_n * num_q / 4 (query, head) columns
SHAPES = [
    (32768, 16, 16, False),   # config 5(ii)'s block over 32K keys: 64 columns, one launch
    (3000, 16, 16, True),     # tree mask
    (2500, 24, 16, False),    # 96 columns: two query groups; the last group stores the rows
    (2500, 32, 16, True),     # GQA 8, 128 columns: two query groups of 8 queries, tree mask
    (4600, 4, 80, False),     # GQA 1, 80 rows: more than 64, so the append's own launch first
    (1800, 8, 33, False),     # 66 columns
    (0, 16, 16, False),       # no history: every key is new
    (900, 16, 3, False),      # 12 columns: the append's own launch, then the decode
    # one query (a decode step): the wave whose tile holds the new key encodes it
    (32767, 16, 1, False),    # config 3's step: the new key is the last of 32,768
    (4100, 24, 1, False),     # GQA 6, the new key inside a partial last tile
    (1000, 16, 1, False),
    (0, 16, 1, False),        # the new key is the only key
]


@pytest.mark.parametrize("start,num_q,sub_n,tree", SHAPES)
def test_decode_append_matches_append_then_decode(dev, start, num_q, sub_n, tree):
    import torch
    from qengine_amd import kvcache
    num_kv, n = 4, start + sub_n
    rng = np.random.default_rng(4242 + start + sub_n)
    k16, v16 = kv_f16(rng, n, num_kv, 256), kv_f16(rng, n, num_kv, 256)
    kb, vb = O.tq3_encode(k16), O.tq3_encode(v16)   # the caches once the block is appended
    q = q_f16(rng, sub_n, num_q, 256)
    tm = None
    if tree:
        tm = np.array([(1 << t) | (int(rng.integers(0, 1 << max(t, 1))) & ((1 << t) - 1))
                       for t in range(sub_n)], np.uint32)
    # the caches before the append: the history, then stale blocks (another
    # encoding) where the block's rows go
    row0 = start * num_kv * 104
    k_pre, v_pre = kb.view(np.uint8).reshape(-1).copy(), vb.view(np.uint8).reshape(-1).copy()
    k_pre[row0:] = O.tq3_encode(kv_f16(rng, sub_n, num_kv, 256)).view(np.uint8).reshape(-1)
    v_pre[row0:] = O.tq3_encode(kv_f16(rng, sub_n, num_kv, 256)).view(np.uint8).reshape(-1)
    k_new, v_new = _dev(k16[start:], dev), _dev(v16[start:], dev)
    qd = _dev(q.view(np.uint16), dev)
    tmd = None if tm is None else _dev(tm, dev)
    kw = dict(num_q=num_q, num_kv=num_kv, start_pos=start, sub_n=sub_n, scale=1 / 16,
              tree_mask=tmd)

    ka, va = _dev(k_pre, dev), _dev(v_pre, dev)
    out_a = torch.zeros((sub_n, num_q, 256), dtype=torch.float16, device=dev)
    ws_a = kvcache.decode_attn_tq3_workspace(num_q, num_kv, sub_n, n, dev)
    kvcache.tq3_append_kv(k_new, v_new, ka[row0:], va[row0:])
    kvcache.decode_attn_tq3(qd, ka, va, out_a, ws_a, **kw)

    kf, vf = _dev(k_pre, dev), _dev(v_pre, dev)
    out_f = torch.zeros((sub_n, num_q, 256), dtype=torch.float16, device=dev)
    ws_f = kvcache.decode_attn_tq3_workspace(num_q, num_kv, sub_n, n, dev)
    kvcache.decode_attn_tq3_append(qd, k_new, v_new, kf, vf, out_f, ws_f, **kw)
    # twice in a row on the same workspace: the second call sees the rows it
    # wrote and leaves the same caches and output
    out_f2 = torch.zeros_like(out_f)
    kvcache.decode_attn_tq3_append(qd, k_new, v_new, kf, vf, out_f2, ws_f, **kw)
    torch.cuda.synchronize()

    assert np.array_equal(kf.cpu().numpy(), kb.view(np.uint8).reshape(-1)), "K rows differ from the oracle"
    assert np.array_equal(vf.cpu().numpy(), vb.view(np.uint8).reshape(-1)), "V rows differ from the oracle"
    assert torch.equal(kf, ka) and torch.equal(vf, va)
    assert torch.equal(out_f, out_a), "output differs from append + decode"
    assert torch.equal(out_f2, out_a)
    em, el, eo = O.attn_split(O.KV_TQ3, q, kb, vb, num_q=num_q, num_kv=num_kv, hd=256,
                              start_pos=start, sub_n=sub_n, sub_n_max=sub_n, active_end_max=n,
                              scale=1 / 16, k_splits=8, tree_mask=tm)
    exp = O.attn_split_merge(em, el, eo, num_q=num_q, num_kv=num_kv, hd=256, sub_n=sub_n,
                             sub_n_max=sub_n, k_splits=8)
    exact = O.attn_exact_tq3(q, kb, vb, num_q=num_q, num_kv=num_kv, hd=256, start_pos=start,
                             sub_n=sub_n, scale=1 / 16, tree_mask=tm)
    assert_tq3_attn(out_f.cpu().numpy(), exp.view(np.float16), exact,
                    what=f"decode_append start={start} num_q={num_q} sub_n={sub_n}")


def test_decode_append_rejects_null_rows(dev):
    import torch
    from qengine_amd import kvcache
    from qengine_amd._lib import lib
    k = kvcache.tq3_blocks(16 * 8, dev)
    v = kvcache.tq3_blocks(16 * 8, dev)
    q = torch.zeros((16, 16, 256), dtype=torch.float16, device=dev)
    out = torch.zeros_like(q)
    ws = kvcache.decode_attn_tq3_workspace(16, 4, 16, 16, dev)
    rc = lib().qkv_decode_attn_tq3_append(q.data_ptr(), None, None, k.data_ptr(), v.data_ptr(),
                                          out.data_ptr(), 16, 4, 256, 0, 16, 1 / 16, 0, 0, None,
                                          ws.data_ptr(), ws.numel(), None)
    assert rc != 0   # QKV_ERR_NULL, before any launch
    with pytest.raises(ValueError):   # rows smaller than the block: refused by the wrapper
        kvcache.decode_attn_tq3_append(q, q[:0], q[:0], k, v, out, ws, num_q=16, num_kv=4,
                                       start_pos=0, sub_n=16, scale=1 / 16)
