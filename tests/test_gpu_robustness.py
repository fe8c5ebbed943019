"""Failure handling of the single-launch decode paths, forced from the host.

The in-kernel merge waits for the records of its launch with a bounded poll.
qkv_debug_set_merge_spin_limit(0) makes every merger run out of polls at once
(no wait, every kernel exits normally), which must yield NaN rows, a sticky
QKV_ERR_TIMEOUT from qkv_decode_workspace_status, NaN rows on later calls with
the normal limit, and correct results again after qkv_decode_workspace_reset."""
import numpy as np
import pytest

from oracle import oracle as O
from tests._data import assert_tq3_attn, kv_f16, q_f16, rel_err

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _oracle(kind, q, kb, vb, nq, nkv, n):
    """Reference-order split decode + merge (attention.cuh:1905-2177, 1837-1891)."""
    pm, pl, po = O.attn_split(kind, q, kb, vb, num_q=nq, num_kv=nkv, hd=256, start_pos=n - 1,
                              sub_n=1, sub_n_max=1, active_end_max=n, scale=1 / 16, k_splits=8)
    return O.attn_split_merge(pm, pl, po, num_q=nq, num_kv=nkv, hd=256, sub_n=1, sub_n_max=1,
                              k_splits=8).view(np.float16).astype(np.float64)


def _async_status(ws):
    """qkv_decode_workspace_status_async into a device int, read after a sync."""
    import torch
    from qengine_amd import kvcache
    st = torch.full((1,), 12345, dtype=torch.int32, device=ws.device)
    kvcache.decode_workspace_status_async(ws, st)
    torch.cuda.synchronize()
    return int(st.item())


def _timeout_cycle(dev, call, ws, ref, exact=None):
    from qengine_amd import kvcache
    import torch
    assert kvcache.decode_workspace_status(ws) == 0
    assert _async_status(ws) == 0
    try:
        kvcache.debug_set_merge_spin_limit(0)
        out = call()
        assert kvcache.decode_workspace_status(ws) == -8
        assert _async_status(ws) == -8
        assert np.all(np.isnan(out)), "timed-out merge must write NaN rows"
        kvcache.debug_set_merge_spin_limit(-1)
        out = call()   # the error is sticky until the workspace is reset
        assert np.all(np.isnan(out))
        assert kvcache.decode_workspace_status(ws) == -8
    finally:
        kvcache.debug_set_merge_spin_limit(-1)
    kvcache.decode_workspace_reset(ws)
    assert kvcache.decode_workspace_status(ws) == 0
    assert _async_status(ws) == 0
    out = call()
    torch.cuda.synchronize()
    assert not np.any(np.isnan(out))
    if exact is None:
        assert rel_err(out, ref) < TOL
    else:
        assert_tq3_attn(out, ref, exact)
    assert kvcache.decode_workspace_status(ws) == 0


def test_tq3_decode_merge_timeout(dev):
    import torch
    from qengine_amd import kvcache
    rng = np.random.default_rng(71)
    n, nq, nkv = 3000, 16, 4
    k16, v16 = kv_f16(rng, n, nkv, 256), kv_f16(rng, n, nkv, 256)
    kb, vb = O.tq3_encode(k16), O.tq3_encode(v16)
    q = q_f16(rng, 1, nq, 256)
    ref = _oracle(O.KV_TQ3, q, kb, vb, nq, nkv, n)
    exact = O.attn_exact_tq3(q, kb, vb, num_q=nq, num_kv=nkv, hd=256, start_pos=n - 1, sub_n=1,
                             scale=1 / 16)
    ws = kvcache.decode_attn_tq3_workspace(nq, nkv, 1, n, dev)
    qd, kd, vd = _dev(q.view(np.uint16), dev), _dev(kb.view(np.uint8), dev), _dev(vb.view(np.uint8), dev)

    def call():
        out = torch.zeros((1, nq, 256), dtype=torch.float16, device=dev)
        kvcache.decode_attn_tq3(qd, kd, vd, out, ws, num_q=nq, num_kv=nkv, start_pos=n - 1,
                                sub_n=1, scale=1 / 16)
        torch.cuda.synchronize()
        return out.cpu().numpy().astype(np.float64)
    _timeout_cycle(dev, call, ws, ref, exact)


@pytest.mark.parametrize("sub_n", [16, 5])
def test_tq3_multi_query_merge_timeout(dev, sub_n):
    """The shared-decode multi-query path (more than 16 query-head columns):
    its mergers take their units two at a time (16 queries: 16 units per
    merger, all in pairs; 5 queries: 5 per merger, two pairs and a single),
    and a timed-out pair writes NaN rows like a single unit."""
    import torch
    from qengine_amd import kvcache
    rng = np.random.default_rng(73 + sub_n)
    n, nq, nkv = 3000, 16, 4
    k16, v16 = kv_f16(rng, n, nkv, 256), kv_f16(rng, n, nkv, 256)
    kb, vb = O.tq3_encode(k16), O.tq3_encode(v16)
    q = q_f16(rng, sub_n, nq, 256)
    start = n - sub_n
    pm, pl, po = O.attn_split(O.KV_TQ3, q, kb, vb, num_q=nq, num_kv=nkv, hd=256, start_pos=start,
                              sub_n=sub_n, sub_n_max=sub_n, active_end_max=n, scale=1 / 16,
                              k_splits=8)
    ref = O.attn_split_merge(pm, pl, po, num_q=nq, num_kv=nkv, hd=256, sub_n=sub_n,
                             sub_n_max=sub_n, k_splits=8).view(np.float16)
    exact = O.attn_exact_tq3(q, kb, vb, num_q=nq, num_kv=nkv, hd=256, start_pos=start,
                             sub_n=sub_n, scale=1 / 16)
    ws = kvcache.decode_attn_tq3_workspace(nq, nkv, sub_n, n, dev)
    qd, kd, vd = _dev(q.view(np.uint16), dev), _dev(kb.view(np.uint8), dev), _dev(vb.view(np.uint8), dev)

    def call():
        out = torch.zeros((sub_n, nq, 256), dtype=torch.float16, device=dev)
        kvcache.decode_attn_tq3(qd, kd, vd, out, ws, num_q=nq, num_kv=nkv, start_pos=start,
                                sub_n=sub_n, scale=1 / 16)
        torch.cuda.synchronize()
        return out.cpu().numpy()
    _timeout_cycle(dev, call, ws, ref, exact)


def test_q8_decode_merge_timeout(dev):
    import torch
    from qengine_amd import kvcache
    rng = np.random.default_rng(72)
    n, nq, nkv = 1500, 16, 4
    k16, v16 = kv_f16(rng, n, nkv, 256), kv_f16(rng, n, nkv, 256)
    kb, vb = O.q8_encode(k16), O.q8_encode(v16)
    q = q_f16(rng, 1, nq, 256)
    ref = _oracle(O.KV_Q8, q, kb, vb, nq, nkv, n)
    ws = kvcache.decode_attn_q8_workspace(nq, nkv, 1, n, dev)
    qd, kd, vd = _dev(q.view(np.uint16), dev), _dev(kb.view(np.uint8), dev), _dev(vb.view(np.uint8), dev)

    def call():
        out = torch.zeros((1, nq, 256), dtype=torch.float16, device=dev)
        kvcache.decode_attn_q8(qd, kd, vd, out, ws, num_q=nq, num_kv=nkv, start_pos=n - 1,
                               sub_n=1, scale=1 / 16)
        torch.cuda.synchronize()
        return out.cpu().numpy().astype(np.float64)
    _timeout_cycle(dev, call, ws, ref)



def test_noalloc_decode_merge_timeout(dev):
    """The allocation-free decode's scratch through its device-keyed status and
    reset (the caller never sees the scratch's address)."""
    import torch
    from qengine_amd import kvcache
    rng = np.random.default_rng(73)
    n, nq, nkv = 2500, 16, 4
    k16, v16 = kv_f16(rng, n, nkv, 256), kv_f16(rng, n, nkv, 256)
    kb, vb = O.tq3_encode(k16), O.tq3_encode(v16)
    q = q_f16(rng, 1, nq, 256)
    ref = _oracle(O.KV_TQ3, q, kb, vb, nq, nkv, n)
    exact = O.attn_exact_tq3(q, kb, vb, num_q=nq, num_kv=nkv, hd=256, start_pos=n - 1, sub_n=1,
                             scale=1 / 16)
    qd, kd, vd = _dev(q.view(np.uint16), dev), _dev(kb.view(np.uint8), dev), _dev(vb.view(np.uint8), dev)
    device = dev.index or 0

    def call():
        out = torch.zeros((1, nq, 256), dtype=torch.float16, device=dev)
        kvcache.decode_attn_tq3_noalloc(qd, kd, vd, out, num_q=nq, num_kv=nkv, start_pos=n - 1,
                                        sub_n=1, scale=1 / 16)
        torch.cuda.synchronize()
        return out.cpu().numpy().astype(np.float64)

    def async_status():
        st = torch.full((1,), 12345, dtype=torch.int32, device=dev)
        kvcache.decode_noalloc_status_async(st, device)
        torch.cuda.synchronize()
        return int(st.item())

    kvcache.decode_noalloc_reset(device)
    assert kvcache.decode_noalloc_status(device) == 0
    assert async_status() == 0
    try:
        kvcache.debug_set_merge_spin_limit(0)
        assert np.all(np.isnan(call())), "timed-out merge must write NaN rows"
        assert kvcache.decode_noalloc_status(device) == -8
        assert async_status() == -8
        kvcache.debug_set_merge_spin_limit(-1)
        assert np.all(np.isnan(call())), "the error is sticky until the scratch is reset"
        assert kvcache.decode_noalloc_status(device) == -8
    finally:
        kvcache.debug_set_merge_spin_limit(-1)
        kvcache.decode_noalloc_reset(device)
    assert kvcache.decode_noalloc_status(device) == 0
    assert async_status() == 0
    out = call()
    assert_tq3_attn(out, ref, exact)
    assert kvcache.decode_noalloc_status(device) == 0
