"""The allocation-free decode entry point qkv_decode_attn_tq3_noalloc, called
through the C ABI, against the workspace entry point qkv_decode_attn_tq3 on
the same inputs: two calls in a row, the second with a smaller input (the
scratch keeps the first call's contents).  Both run the same kernels with the
same geometry, so the outputs must be bit-identical (and meet the decode's
own bar, tests/_data.assert_tq3_attn)."""
import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from tests._data import assert_tq3_attn, kv_f16, q_f16

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _case(dev, seed, n_keys, sub_n, num_q, num_kv):
    import torch
    from qengine_amd import _lib
    L = _lib.lib()
    rng = np.random.default_rng(seed)
    k16, v16 = kv_f16(rng, n_keys, num_kv, 256), kv_f16(rng, n_keys, num_kv, 256)
    kb, vb = O.tq3_encode(k16), O.tq3_encode(v16)
    q = q_f16(rng, sub_n, num_q, 256)
    start = n_keys - sub_n
    qd, kd, vd = _dev(q.view(np.uint16), dev), _dev(kb.view(np.uint8), dev), _dev(vb.view(np.uint8), dev)
    st = torch.cuda.current_stream().cuda_stream
    ws_n = L.qkv_decode_attn_tq3_workspace_bytes(num_q, num_kv, sub_n, n_keys)
    ws = torch.zeros(ws_n, dtype=torch.uint8, device=dev)
    out_ws = torch.zeros((sub_n, num_q, 256), dtype=torch.float16, device=dev)
    out_na = torch.full((sub_n, num_q, 256), float("nan"), dtype=torch.float16, device=dev)
    assert L.qkv_decode_attn_tq3(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), out_ws.data_ptr(),
                                 num_q, num_kv, 256, start, sub_n, ctypes.c_float(1 / 16), 0, 0,
                                 None, ws.data_ptr(), ws_n, st) == 0
    assert L.qkv_decode_attn_tq3_noalloc(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(),
                                         out_na.data_ptr(), num_q, num_kv, 256, start, sub_n,
                                         ctypes.c_float(1 / 16), 0, 0, None, st) == 0
    torch.cuda.synchronize()
    a, b = out_ws.cpu().numpy(), out_na.cpu().numpy()
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))
    ks = 8
    pm, pl, po = O.attn_split(O.KV_TQ3, q, kb, vb, num_q=num_q, num_kv=num_kv, hd=256,
                              start_pos=start, sub_n=sub_n, sub_n_max=sub_n, active_end_max=n_keys,
                              scale=1 / 16, k_splits=ks)
    ref = O.attn_split_merge(pm, pl, po, num_q=num_q, num_kv=num_kv, hd=256, sub_n=sub_n,
                             sub_n_max=sub_n, k_splits=ks).view(np.float16)
    exact = O.attn_exact_tq3(q, kb, vb, num_q=num_q, num_kv=num_kv, hd=256, start_pos=start,
                             sub_n=sub_n, scale=1 / 16)
    assert_tq3_attn(b, ref, exact)


def test_noalloc_matches_workspace_entry_point(dev):
    _case(dev, 301, 9000, 1, 16, 4)      # 18 key chunks of 512
    _case(dev, 302, 700, 1, 16, 4)       # smaller: 2 chunks, the scratch keeps call 1's rows
    _case(dev, 303, 2500, 4, 24, 4)      # multi-query, GQA 6


def test_noalloc_rejects_oversized_shape(dev):
    from qengine_amd import _lib
    L = _lib.lib()
    # 64 q heads x 256 queries over one chunk: 16384 record rows (> 8 MiB of scratch)
    need = L.qkv_decode_attn_tq3_workspace_bytes(64, 8, 256, 4096)
    assert need > 8 << 20
    import torch
    buf = torch.zeros(1 << 20, dtype=torch.uint8, device=dev)
    p = buf.data_ptr()
    assert L.qkv_decode_attn_tq3_noalloc(p, p, p, p, 64, 8, 256, 4096 - 256, 256,
                                         ctypes.c_float(1 / 16), 0, 0, None, None) == -7
