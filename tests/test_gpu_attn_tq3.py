"""GPU parity of the TQ3 split-K flash decode (attention.cuh:1905-2177) and
merge (attention.cuh:1837-1891) against the CPU oracle on identical seeded
inputs.  Bar: merged output within 2e-3 relative error (max |diff| / max |ref|),
fp32 accumulation; split partials within the same tolerance."""
import numpy as np
import pytest

from oracle import oracle as O
from tests._data import assert_tq3_attn, kv_f16, q_f16, rel_err, rel_err_global

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _torch():
    import torch
    return torch


def _dev(a, dev):
    return _torch().from_numpy(np.ascontiguousarray(a)).to(dev)


def _cache(seed, n, num_kv=4, hd=256):
    rng = np.random.default_rng(seed)
    k16 = kv_f16(rng, n, num_kv, hd)
    v16 = kv_f16(rng, n, num_kv, hd)
    return rng, O.tq3_encode(k16), O.tq3_encode(v16)


def _run_split(dev, q, kb, vb, **kw):
    from qengine_amd import kvcache
    torch = _torch()
    nq, smax, ks = kw["num_q"], kw["sub_n_max"], kw["k_splits"]
    pm = torch.full((nq, smax, ks), float("nan"), device=dev)
    pl = torch.full((nq, smax, ks), float("nan"), device=dev)
    po = torch.full((nq, smax, ks, 256), float("nan"), device=dev)
    tm = kw.pop("tree_mask", None)
    kvcache.attn_split_tq3(_dev(q.view(np.uint16), dev), _dev(kb.view(np.uint8), dev),
                           _dev(vb.view(np.uint8), dev), pm, pl, po,
                           tree_mask=None if tm is None else _dev(tm.astype(np.int32), dev), **kw)
    out = torch.zeros((kw["sub_n"], nq, 256), dtype=torch.float16, device=dev)
    kvcache.attn_split_merge(pm, pl, po, out, num_q=nq, num_kv=kw["num_kv"], sub_n=kw["sub_n"],
                             sub_n_max=smax, k_splits=ks)
    torch.cuda.synchronize()
    return pm.cpu().numpy(), pl.cpu().numpy(), po.cpu().numpy(), out.cpu().numpy()


def _check_partials(pm, pl, po, em, el, eo, sub_n):
    pm, pl, po = pm[:, :sub_n], pl[:, :sub_n], po[:, :sub_n]
    em, el, eo = em[:, :sub_n], el[:, :sub_n], eo[:, :sub_n]
    empty = ~np.isfinite(em)
    assert np.array_equal(empty, ~np.isfinite(pm)), "empty-split pattern differs"
    assert np.all(pl[empty] == 0) and np.all(po[empty] == 0)
    live = ~empty
    assert np.max(np.abs(pm[live] - em[live])) < 1e-2
    # compare l and o after bringing both to the reference max
    w = np.exp(pm[live] - em[live])
    assert np.max(np.abs(pl[live] * w - el[live]) / el[live]) < TOL
    assert rel_err_global(po[live] * w[:, None], eo[live]) < TOL


def _exact(q, kb, vb, *, num_q, num_kv=4, start_pos, sub_n, scale=1 / 16, sink_tok=0,
           window_tok=0, tree_mask=None, **_):
    return O.attn_exact_tq3(q, kb, vb, num_q=num_q, num_kv=num_kv, hd=256, start_pos=start_pos,
                            sub_n=sub_n, scale=scale, sink_tok=sink_tok, window_tok=window_tok,
                            tree_mask=tree_mask)


@pytest.mark.parametrize("n,k_splits,num_q", [(4097, 8, 16), (1000, 8, 16), (33, 8, 16),
                                              (1, 1, 16), (777, 5, 24), (2500, 32, 16)])
def test_split_decode_vs_oracle(dev, n, k_splits, num_q):
    rng, kb, vb = _cache(n, n)
    q = q_f16(rng, 1, num_q, 256)
    kw = dict(num_q=num_q, num_kv=4, start_pos=n - 1, sub_n=1, sub_n_max=16,
              active_end_max=n, scale=1 / 16, k_splits=k_splits)
    pm, pl, po, out = _run_split(dev, q, kb, vb, **kw)
    em, el, eo = O.attn_split(O.KV_TQ3, q, kb, vb, hd=256, **kw)
    exp = O.attn_split_merge(em, el, eo, num_q=num_q, num_kv=4, hd=256, sub_n=1, sub_n_max=16,
                             k_splits=k_splits)
    _check_partials(pm, pl, po, em, el, eo, 1)
    assert_tq3_attn(out, exp.view(np.float16), _exact(q, kb, vb, **kw))


@pytest.mark.parametrize("sink,window,tree", [(0, 0, False), (0, 0, True), (64, 256, False),
                                              (32, 100, True)])
def test_split_verify_masks(dev, sink, window, tree):
    n, sub_n = 3000, 16
    rng, kb, vb = _cache(7 + sink, n)
    q = q_f16(rng, sub_n, 16, 256)
    tm = None
    if tree:
        tm = np.array([(1 << t) | (int(rng.integers(0, 1 << max(t, 1))) & ((1 << t) - 1))
                       for t in range(sub_n)], np.uint32)
    kw = dict(num_q=16, num_kv=4, start_pos=n - sub_n, sub_n=sub_n, sub_n_max=16,
              active_end_max=n, scale=1 / 16, k_splits=8, sink_tok=sink, window_tok=window)
    pm, pl, po, out = _run_split(dev, q, kb, vb, tree_mask=tm, **kw)
    em, el, eo = O.attn_split(O.KV_TQ3, q, kb, vb, hd=256, tree_mask=tm, **kw)
    exp = O.attn_split_merge(em, el, eo, num_q=16, num_kv=4, hd=256, sub_n=sub_n, sub_n_max=16,
                             k_splits=8)
    _check_partials(pm, pl, po, em, el, eo, sub_n)
    assert_tq3_attn(out, exp.view(np.float16), _exact(q, kb, vb, tree_mask=tm, **kw))


@pytest.mark.parametrize("n,num_q,sub_n", [(4097, 16, 1), (32768, 16, 1), (1, 16, 1),
                                           (300, 24, 1), (2064, 16, 16), (2000, 20, 1), (1000, 28, 1),
                                           (1500, 12, 1)])
def test_fast_decode_vs_oracle(dev, n, num_q, sub_n):
    from qengine_amd import kvcache
    torch = _torch()
    rng, kb, vb = _cache(100 + n, n)
    q = q_f16(rng, sub_n, num_q, 256)
    start = n - sub_n
    ws = kvcache.decode_attn_tq3_workspace(num_q, 4, sub_n, n, dev)
    out = torch.zeros((sub_n, num_q, 256), dtype=torch.float16, device=dev)
    kvcache.decode_attn_tq3(_dev(q.view(np.uint16), dev), _dev(kb.view(np.uint8), dev),
                            _dev(vb.view(np.uint8), dev), out, ws, num_q=num_q, num_kv=4,
                            start_pos=start, sub_n=sub_n, scale=1 / 16)
    torch.cuda.synchronize()
    em, el, eo = O.attn_split(O.KV_TQ3, q, kb, vb, num_q=num_q, num_kv=4, hd=256,
                              start_pos=start, sub_n=sub_n, sub_n_max=sub_n, active_end_max=n,
                              scale=1 / 16, k_splits=8)
    exp = O.attn_split_merge(em, el, eo, num_q=num_q, num_kv=4, hd=256, sub_n=sub_n,
                             sub_n_max=sub_n, k_splits=8)
    assert_tq3_attn(out.cpu().numpy(), exp.view(np.float16),
                    _exact(q, kb, vb, num_q=num_q, start_pos=start, sub_n=sub_n))


@pytest.mark.parametrize("n,num_q,sub_n,sink,window,tree", [
    (3000, 16, 16, 0, 0, True), (3000, 16, 16, 64, 256, False), (3000, 16, 16, 32, 100, True),
    (2000, 16, 5, 0, 0, False), (1500, 16, 7, 0, 0, True), (1200, 24, 3, 0, 0, False),
    (900, 8, 11, 0, 0, True), (700, 4, 17, 0, 0, False), (20016, 16, 16, 0, 0, False),
    (800, 32, 3, 0, 0, True), (2500, 24, 2, 16, 512, False), (600, 16, 3, 0, 0, False),
    (900, 12, 7, 0, 0, True), (700, 20, 4, 0, 0, False), (650, 28, 3, 0, 0, True),
    # more than 64 columns: several query blocks per call (64 + 16, 60 + 36, 64 + 2)
    (3000, 16, 20, 0, 0, False), (2500, 24, 16, 0, 0, True), (1800, 8, 33, 0, 0, False),
    # chunks grown to keep one round of workgroups: 2 and 3 tiles per wave
    (40000, 16, 1, 0, 0, False), (70000, 24, 1, 0, 0, False), (40000, 16, 2, 128, 2048, True),
    # 16 queries x GQA 4 = 64 columns, every tile decoded once (tq3_mq_kernel):
    # 64 chunks of 512 keys, the last also taking the remainder past 32768
    # keys (16, 32 and 64 keys: joined; 65 keys: 33 chunks of 1024)
    (32784, 16, 16, 0, 0, False),
    (32800, 16, 16, 0, 0, False), (32832, 16, 16, 0, 0, True), (32833, 16, 16, 0, 0, False)])
def test_fast_decode_multi_query(dev, n, num_q, sub_n, sink, window, tree):
    """Several queries per workgroup (they share the MFMA columns): partial
    last groups, GQA 1 to 8, causal, tree and sink/window masks; calls
    with at most 8 / GQA queries carry rounded query and remainder in one
    product, up to 16 / GQA queries the remainders ride in a chained product,
    and calls with more than 16 (query, head) columns decode each tile once
    for up to 64 of them (tq3_mq_kernel; GQA 4 x 16 queries, GQA 2 x 11,
    GQA 1 x 17, GQA 8 x 3, partial column groups, several query blocks)."""
    from qengine_amd import kvcache
    torch = _torch()
    num_kv = 4
    rng, kb, vb = _cache(900 + n + sub_n, n, num_kv)
    q = q_f16(rng, sub_n, num_q, 256)
    tm = None
    if tree:
        tm = np.array([(1 << t) | (int(rng.integers(0, 1 << max(t, 1))) & ((1 << t) - 1))
                       for t in range(sub_n)], np.uint32)
    start = n - sub_n
    ws = kvcache.decode_attn_tq3_workspace(num_q, num_kv, sub_n, n, dev)
    out = torch.zeros((sub_n, num_q, 256), dtype=torch.float16, device=dev)
    tmd = None if tm is None else _dev(tm, dev)
    kvcache.decode_attn_tq3(_dev(q.view(np.uint16), dev), _dev(kb.view(np.uint8), dev),
                            _dev(vb.view(np.uint8), dev), out, ws, num_q=num_q, num_kv=num_kv,
                            start_pos=start, sub_n=sub_n, scale=1 / 16, sink_tok=sink,
                            window_tok=window, tree_mask=tmd)
    torch.cuda.synchronize()
    em, el, eo = O.attn_split(O.KV_TQ3, q, kb, vb, num_q=num_q, num_kv=num_kv, hd=256,
                              start_pos=start, sub_n=sub_n, sub_n_max=sub_n, active_end_max=n,
                              scale=1 / 16, k_splits=8, sink_tok=sink, window_tok=window,
                              tree_mask=tm)
    exp = O.attn_split_merge(em, el, eo, num_q=num_q, num_kv=num_kv, hd=256, sub_n=sub_n,
                             sub_n_max=sub_n, k_splits=8)
    assert_tq3_attn(out.cpu().numpy(), exp.view(np.float16),
                    _exact(q, kb, vb, num_q=num_q, num_kv=num_kv, start_pos=start, sub_n=sub_n,
                           sink_tok=sink, window_tok=window, tree_mask=tm))


def test_fast_decode_rejects_small_workspace(dev):
    from qengine_amd import QKVError, kvcache
    torch = _torch()
    q = torch.zeros((1, 16, 256), dtype=torch.float16, device=dev)
    kv = torch.zeros((100 * 8, 52), dtype=torch.uint8, device=dev)
    out = torch.zeros_like(q)
    ws = torch.zeros(16, dtype=torch.uint8, device=dev)
    with pytest.raises(QKVError):
        kvcache.decode_attn_tq3(q, kv, kv, out, ws, num_q=16, num_kv=4, start_pos=99, sub_n=1,
                                scale=1 / 16)


def _fast_expected(q, kb, vb, n, num_q, sub_n):
    em, el, eo = O.attn_split(O.KV_TQ3, q, kb, vb, num_q=num_q, num_kv=4, hd=256,
                              start_pos=n - sub_n, sub_n=sub_n, sub_n_max=sub_n,
                              active_end_max=n, scale=1 / 16, k_splits=8)
    return O.attn_split_merge(em, el, eo, num_q=num_q, num_kv=4, hd=256, sub_n=sub_n,
                              sub_n_max=sub_n, k_splits=8).view(np.float16)


def test_fast_decode_workspace_reuse(dev):
    """One workspace across calls of different lengths and query counts: every
    merger clears the record tags it consumed, so no call can take an earlier
    call's records for its own."""
    from qengine_amd import kvcache
    torch = _torch()
    ws = kvcache.decode_attn_tq3_workspace(16, 4, 4, 32768, dev)
    for i, (n, sub_n) in enumerate([(32768, 1), (4097, 1), (32768, 1), (1000, 4), (4097, 1),
                                    (32768, 4)]):
        rng, kb, vb = _cache(500 + i, n)
        q = q_f16(rng, sub_n, 16, 256)
        out = torch.zeros((sub_n, 16, 256), dtype=torch.float16, device=dev)
        kvcache.decode_attn_tq3(_dev(q.view(np.uint16), dev), _dev(kb.view(np.uint8), dev),
                                _dev(vb.view(np.uint8), dev), out, ws, num_q=16, num_kv=4,
                                start_pos=n - sub_n, sub_n=sub_n, scale=1 / 16)
        torch.cuda.synchronize()
        assert_tq3_attn(out.cpu().numpy(), _fast_expected(q, kb, vb, n, 16, sub_n),
                        _exact(q, kb, vb, num_q=16, start_pos=n - sub_n, sub_n=sub_n), what=(n, sub_n))


def test_fast_decode_leaves_record_tags_clear(dev):
    """After a call every record tag of the workspace is clear again (the state
    of a zero-filled workspace), while the record scalars were written."""
    from qengine_amd import kvcache
    torch = _torch()
    n, num_q = 32768, 16
    ws = kvcache.decode_attn_tq3_workspace(num_q, 4, 1, n, dev)
    for i in range(2):
        rng, kb, vb = _cache(900 + i, n)
        q = q_f16(rng, 1, num_q, 256)
        out = torch.zeros((1, num_q, 256), dtype=torch.float16, device=dev)
        kvcache.decode_attn_tq3(_dev(q.view(np.uint16), dev), _dev(kb.view(np.uint8), dev),
                                _dev(vb.view(np.uint8), dev), out, ws, num_q=num_q, num_kv=4,
                                start_pos=n - 1, sub_n=1, scale=1 / 16)
        torch.cuda.synchronize()
        assert_tq3_attn(out.cpu().numpy(), _fast_expected(q, kb, vb, n, num_q, 1),
                        _exact(q, kb, vb, num_q=num_q, start_pos=n - 1, sub_n=1))
        # 512-key chunks at this length: 64 records per q head after a 256-byte header
        ml = ws.cpu().numpy()[256:256 + num_q * 64 * 16].view(np.uint32).reshape(num_q * 64, 4)
        assert not ml[:, 2:].any(), "record tags left set"
        assert (ml[:, 1].view(np.float32) > 0).all(), "record sums missing"


def test_fast_decode_output_may_alias_query(dev):
    """The output may overwrite the query in place (model.cuh:2479-2482 merges into q_buf)."""
    from qengine_amd import kvcache
    torch = _torch()
    n = 4097
    rng, kb, vb = _cache(777, n)
    q = q_f16(rng, 1, 16, 256)
    qt = _dev(q.view(np.uint16), dev).view(torch.float16)
    ws = kvcache.decode_attn_tq3_workspace(16, 4, 1, n, dev)
    kvcache.decode_attn_tq3(qt, _dev(kb.view(np.uint8), dev), _dev(vb.view(np.uint8), dev), qt, ws,
                            num_q=16, num_kv=4, start_pos=n - 1, sub_n=1, scale=1 / 16)
    torch.cuda.synchronize()
    assert_tq3_attn(qt.cpu().numpy(), _fast_expected(q, kb, vb, n, 16, 1),
                    _exact(q, kb, vb, num_q=16, start_pos=n - 1, sub_n=1))
