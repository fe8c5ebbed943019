"""The decode paths under HIP graph capture (serving loops capture their
launch-bound inner loops).  Each test records the calls into a graph once and
replays it several times, with ordinary eager calls on other data between the
replays; every replay must reproduce the eager result bit for bit (the
kernels are deterministic), and the caches an append writes inside the graph
must equal an eager append's bytes."""
import numpy as np
import pytest

from oracle import oracle as O
from tests._data import kv_f16, q_f16

pytestmark = pytest.mark.gpu


def _dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _capture(fn):
    import torch
    fn()   # the first call outside the capture (library set-up, allocations)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


def test_tq3_decode_graph_replays(dev):
    import torch
    from qengine_amd import kvcache
    rng = np.random.default_rng(31)
    n, nq, nkv = 9000, 16, 4
    k16, v16 = kv_f16(rng, n, nkv, 256), kv_f16(rng, n, nkv, 256)
    kb, vb = _dev(O.tq3_encode(k16).view(np.uint8), dev), _dev(O.tq3_encode(v16).view(np.uint8), dev)
    q = _dev(q_f16(rng, 1, nq, 256).view(np.uint16), dev)
    q2 = _dev(q_f16(rng, 3, nq, 256).view(np.uint16), dev)
    ws = kvcache.decode_attn_tq3_workspace(nq, nkv, 3, n, dev)
    out = torch.zeros((1, nq, 256), dtype=torch.float16, device=dev)
    out2 = torch.zeros((3, nq, 256), dtype=torch.float16, device=dev)

    status = torch.full((1,), 12345, dtype=torch.int32, device=dev)

    def call():
        kvcache.decode_attn_tq3(q, kb, vb, out, ws, num_q=nq, num_kv=nkv, start_pos=n - 1, sub_n=1,
                                scale=1 / 16)
        kvcache.decode_workspace_status_async(ws, status)   # the health check rides in the graph
    call()
    torch.cuda.synchronize()
    ref = out.clone()
    g = _capture(call)
    for i in range(4):
        out.zero_()
        status.fill_(12345)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {i}"
        assert int(status.item()) == 0, f"replay {i}: workspace status"
        # eager work on the same workspace between replays (three queries)
        kvcache.decode_attn_tq3(q2, kb, vb, out2, ws, num_q=nq, num_kv=nkv, start_pos=n - 3,
                                sub_n=3, scale=1 / 16)
        torch.cuda.synchronize()
    assert kvcache.decode_workspace_status(ws) == 0


def test_tq3_noalloc_decode_graph_replays(dev):
    import torch
    from qengine_amd import kvcache
    rng = np.random.default_rng(32)
    n, nq, nkv = 5000, 24, 4
    k16, v16 = kv_f16(rng, n, nkv, 256), kv_f16(rng, n, nkv, 256)
    kb, vb = _dev(O.tq3_encode(k16).view(np.uint8), dev), _dev(O.tq3_encode(v16).view(np.uint8), dev)
    q = _dev(q_f16(rng, 2, nq, 256).view(np.uint16), dev)
    out = torch.zeros((2, nq, 256), dtype=torch.float16, device=dev)

    def call():
        kvcache.decode_attn_tq3_noalloc(q, kb, vb, out, num_q=nq, num_kv=nkv, start_pos=n - 2,
                                        sub_n=2, scale=1 / 16)
    call()
    torch.cuda.synchronize()
    ref = out.clone()
    g = _capture(call)
    for i in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {i}"
        call()   # eager call on the same scratch between replays
        torch.cuda.synchronize()
        assert torch.equal(out, ref)


def test_q8_append_and_decode_graph_replays(dev):
    """One layer of config 2 (append the new token's K and V, then decode) in a
    graph: every replay rewrites the same cache row with the same bytes and
    yields the eager output."""
    import torch
    from qengine_amd import kvcache
    rng = np.random.default_rng(33)
    ctx, nq, nkv = 4096, 16, 4
    bt = nkv * 256 // 32
    k16, v16 = kv_f16(rng, ctx, nkv, 256), kv_f16(rng, ctx, nkv, 256)
    kb = kvcache.q8_blocks((ctx + 1) * bt, dev)
    vb = kvcache.q8_blocks((ctx + 1) * bt, dev)
    kvcache.q8_append(_dev(k16, dev), kb[: ctx * bt])
    kvcache.q8_append(_dev(v16, dev), vb[: ctx * bt])
    knew = _dev(kv_f16(rng, 1, nkv, 256), dev)
    vnew = _dev(kv_f16(rng, 1, nkv, 256), dev)
    q = _dev(q_f16(rng, 1, nq, 256).view(np.uint16), dev)
    ws = kvcache.decode_attn_q8_workspace(nq, nkv, 1, ctx + 1, dev)
    out = torch.zeros((1, nq, 256), dtype=torch.float16, device=dev)

    def call():
        kvcache.q8_append_kv(knew, vnew, kb[ctx * bt:], vb[ctx * bt:])
        kvcache.decode_attn_q8(q, kb, vb, out, ws, num_q=nq, num_kv=nkv, start_pos=ctx, sub_n=1,
                               scale=1 / 16)
    call()
    torch.cuda.synchronize()
    ref, kref, vref = out.clone(), kb.clone(), vb.clone()
    g = _capture(call)
    for i in range(4):
        out.zero_()
        kb[ctx * bt:].zero_()
        vb[ctx * bt:].zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {i}"
        assert torch.equal(kb, kref) and torch.equal(vb, vref), f"replay {i}: appended rows"


def test_tq3_verify_append_in_decode_graph_replays(dev):
    """A 16-token verify block appended inside the decode launch
    (qkv_decode_attn_tq3_append, one launch at 64 query-head columns) in a
    graph: every replay rewrites the block's cache rows with the same bytes
    and yields the eager output, with an eager decode of another shape on the
    same workspace between the replays."""
    import torch
    from qengine_amd import kvcache
    rng = np.random.default_rng(57)
    hist, nv, nq, nkv = 6000, 16, 16, 4
    n = hist + nv
    kb = kvcache.tq3_blocks(n * nkv * 2, dev)
    vb = kvcache.tq3_blocks(n * nkv * 2, dev)
    kvcache.tq3_append_kv(_dev(kv_f16(rng, hist, nkv, 256), dev), _dev(kv_f16(rng, hist, nkv, 256), dev),
                          kb[: hist * nkv * 2], vb[: hist * nkv * 2])
    knew = _dev(kv_f16(rng, nv, nkv, 256), dev)
    vnew = _dev(kv_f16(rng, nv, nkv, 256), dev)
    q = _dev(q_f16(rng, nv, nq, 256).view(np.uint16), dev)
    ws = kvcache.decode_attn_tq3_workspace(nq, nkv, nv, n, dev)
    out = torch.zeros((nv, nq, 256), dtype=torch.float16, device=dev)
    q1 = _dev(q_f16(rng, 1, nq, 256).view(np.uint16), dev)
    out1 = torch.zeros((1, nq, 256), dtype=torch.float16, device=dev)

    def call():
        kvcache.decode_attn_tq3_append(q, knew, vnew, kb, vb, out, ws, num_q=nq, num_kv=nkv,
                                       start_pos=hist, sub_n=nv, scale=1 / 16)
    call()
    torch.cuda.synchronize()
    ref, kref, vref = out.clone(), kb.clone(), vb.clone()
    g = _capture(call)
    for i in range(4):
        out.zero_()
        kb[hist * nkv * 2:].zero_()
        vb[hist * nkv * 2:].zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {i}"
        assert torch.equal(kb, kref) and torch.equal(vb, vref), f"replay {i}: appended rows"
        kvcache.decode_attn_tq3(q1, kb, vb, out1, ws, num_q=nq, num_kv=nkv, start_pos=n - 1,
                                sub_n=1, scale=1 / 16)
        torch.cuda.synchronize()
