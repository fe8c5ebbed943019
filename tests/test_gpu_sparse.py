"""Block-sparse TQ3 verify on the GPU (model.cuh:4589-4662): K-pool
signatures (attention.cuh:2445-2533) and the top-k block index
(sparse_attn/sparse_index.cuh:214-330) bit-exact against the oracle; the
sparse split attention (attention.cuh:2193-2433) + merge against the oracle's
reference-order computation and the exact fp64 attention over the selected
keys (tests/_data.assert_tq3_attn), including tree masks and a full
append -> signatures -> index -> attention verify step at 32768 keys."""
import numpy as np
import pytest

from oracle import oracle as O
from tests._data import assert_tq3_attn, kv_f16, q_f16

pytestmark = pytest.mark.gpu
HD, NKV = 256, 4


def _dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _gpu_pools(dev, kb, n, stride, blk_lo=0, pools=None, bsn=64):
    import torch
    from qengine_amd import kvcache
    if pools is None:
        pools = (torch.zeros((NKV, stride, HD), dtype=torch.float16, device=dev),
                 torch.zeros((NKV, stride, HD), dtype=torch.float16, device=dev))
    kvcache.tq3_kpool_update(_dev(kb.view(np.uint8), dev), pools[0], pools[1], num_kv=NKV,
                             total_kv=n, blk_lo=blk_lo, block_size_n=bsn)
    torch.cuda.synchronize()
    return pools


@pytest.mark.parametrize("bsn", [64, 32])
def test_kpool_bitexact(dev, bsn):
    rng = np.random.default_rng(21 + bsn)
    n = 64 * 40 + 17
    kb = O.tq3_encode(kv_f16(rng, n, NKV, HD))
    stride = 4 * 64 // bsn * 20
    pools = _gpu_pools(dev, kb, n, stride, bsn=bsn)
    kp = np.zeros((NKV, stride, HD), np.uint16)
    kx = np.zeros_like(kp)
    O.tq3_kpool_update(kb, kp, kx, num_kv=NKV, hd=HD, total_kv=n, blk_lo=0, block_size_n=bsn)
    assert np.array_equal(pools[0].cpu().numpy().view(np.uint16), kp)
    assert np.array_equal(pools[1].cpu().numpy().view(np.uint16), kx)
    # the cache grows and its tail changes: rebuild from the first unfrozen block
    n2 = n + 150
    kb2 = np.concatenate([kb, O.tq3_encode(kv_f16(rng, 150, NKV, HD))])
    lo = (n // bsn) - 1
    pools = _gpu_pools(dev, kb2, n2, stride, blk_lo=lo, pools=pools, bsn=bsn)
    O.tq3_kpool_update(kb2, kp, kx, num_kv=NKV, hd=HD, total_kv=n2, blk_lo=lo, block_size_n=bsn)
    assert np.array_equal(pools[0].cpu().numpy().view(np.uint16), kp)
    assert np.array_equal(pools[1].cpu().numpy().view(np.uint16), kx)


def _oracle_pools(kb, n, stride):
    kp = np.zeros((NKV, stride, HD), np.uint16)
    kx = np.zeros_like(kp)
    O.tq3_kpool_update(kb, kp, kx, num_kv=NKV, hd=HD, total_kv=n, blk_lo=0)
    return kp, kx


def _gpu_index(dev, q, kp, kx, *, num_q, sub_n, start, top_k, nb, beta=0.5):
    import torch
    from qengine_amd import kvcache
    bi = torch.full((NKV, sub_n, top_k), 7, dtype=torch.int32, device=dev)
    kvcache.block_index_ms(_dev(q.view(np.uint16), dev), _dev(kp, dev), _dev(kx, dev), bi,
                           num_q=num_q, num_kv=NKV, sub_n=sub_n, start_pos=start, top_k=top_k,
                           n_blocks=nb, beta=beta)
    torch.cuda.synchronize()
    return bi.cpu().numpy()


@pytest.mark.parametrize("num_q,top_k,beta", [(16, 8, 0.5), (24, 13, 0.5), (16, 64, 0.5),
                                              (16, 1, 2.0), (24, 100, 0.0)])
def test_block_index_bitexact(dev, num_q, top_k, beta):
    rng = np.random.default_rng(31 + top_k)
    n, sub = 64 * 75 + 5, 16
    start = n - sub
    kb = O.tq3_encode(kv_f16(rng, n, NKV, HD))
    nb = (n + 63) // 64
    kp, kx = _oracle_pools(kb, n, nb + 3)
    q = q_f16(rng, sub, num_q, HD)
    got = _gpu_index(dev, q, kp, kx, num_q=num_q, sub_n=sub, start=start, top_k=top_k, nb=nb,
                     beta=beta)
    exp = O.block_index_ms(q, kp, kx, num_q=num_q, num_kv=NKV, hd=HD, sub_n=sub, sub_n_max=sub,
                           start_pos=start, top_k=top_k, n_blocks=nb, beta=beta)
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("nb,top_k,distinct", [(2049, 64, None), (9000, 64, 50), (9000, 300, 50),
                                                (40000, 16, 7)])
def test_block_index_many_blocks_bitexact(dev, nb, top_k, distinct):
    """Long block lists (several blocks per selecting thread, past any LDS
    budget) from synthetic signatures.  With `distinct` set, every block's
    signature is one of that many, so the scores take few values and runs of
    equal scores straddle the pick threshold (ties go to the lower block).
    The last blocks lie past the first queries' reach."""
    rng = np.random.default_rng(nb + top_k)
    sub = 4
    n_sig = distinct or nb
    bp = (rng.standard_normal((NKV, n_sig, HD)) * 0.3).astype(np.float16).view(np.uint16)
    bx = (rng.standard_normal((NKV, n_sig, HD)) * 0.6).astype(np.float16).view(np.uint16)
    pick = rng.integers(0, n_sig, nb) if distinct else np.arange(nb)
    kp, kx = np.ascontiguousarray(bp[:, pick]), np.ascontiguousarray(bx[:, pick])
    start = 64 * (nb - 3) - sub
    q = q_f16(rng, sub, 16, HD)
    got = _gpu_index(dev, q, kp, kx, num_q=16, sub_n=sub, start=start, top_k=top_k, nb=nb)
    exp = O.block_index_ms(q, kp, kx, num_q=16, num_kv=NKV, hd=HD, sub_n=sub, sub_n_max=sub,
                           start_pos=start, top_k=top_k, n_blocks=nb)
    assert np.array_equal(got, exp)


def test_block_scores_bitexact(dev):
    """The block scores the selection works from (the workspace's first
    num_kv * sub_n * n_blocks floats) bit for bit against the oracle's."""
    import torch
    from qengine_amd import kvcache
    rng = np.random.default_rng(77)
    nb, sub = 700, 16
    kp = (rng.standard_normal((NKV, nb, HD)) * 0.3).astype(np.float16).view(np.uint16)
    kx = (rng.standard_normal((NKV, nb, HD)) * 0.6).astype(np.float16).view(np.uint16)
    start = 64 * (nb - 2) - sub
    q = q_f16(rng, sub, 24, HD)
    wsb = int(kvcache.lib().qkv_block_index_ms_workspace_bytes(NKV, sub, nb))
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    bi = torch.full((NKV, sub, 8), 7, dtype=torch.int32, device=dev)
    kvcache.block_index_ms(_dev(q.view(np.uint16), dev), _dev(kp, dev), _dev(kx, dev), bi,
                           num_q=24, num_kv=NKV, sub_n=sub, start_pos=start, top_k=8,
                           n_blocks=nb, beta=0.5, workspace=ws)
    torch.cuda.synchronize()
    got = ws[:NKV * sub * nb * 4].cpu().numpy().view(np.float32).reshape(NKV, sub, nb)
    exp = O.block_scores_ms(q, kp, kx, num_q=24, num_kv=NKV, hd=HD, sub_n=sub, start_pos=start,
                            n_blocks=nb, beta=0.5)
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


def test_block_index_ties_bitexact(dev):
    rng = np.random.default_rng(41)
    n, sub = 64 * 30, 4
    kb = O.tq3_encode(kv_f16(rng, n, NKV, HD))
    kp, kx = _oracle_pools(kb, n, 30)
    kp[:, 10:20] = kp[:, 5:6]          # ten equal signatures
    kx[:, 10:20] = kx[:, 5:6]
    q = q_f16(rng, sub, 16, HD)
    for top_k, start in ((12, n - sub), (40, 64 * 3)):
        got = _gpu_index(dev, q, kp, kx, num_q=16, sub_n=sub, start=start, top_k=top_k, nb=30)
        exp = O.block_index_ms(q, kp, kx, num_q=16, num_kv=NKV, hd=HD, sub_n=sub, sub_n_max=sub,
                               start_pos=start, top_k=top_k, n_blocks=30)
        assert np.array_equal(got, exp), (top_k, start)


def _exact_selected(q, kb, vb, bi, num_q, start, sub, scale, tree_mask=None):
    """fp64 attention over each query's selected blocks (exact dequantized
    values), causal and tree-masked as the kernel's rule."""
    gqa = num_q // NKV
    k64 = O.tq3_decode_f32(kb).astype(np.float64).reshape(-1, NKV, HD)
    v64 = O.tq3_decode_f32(vb).astype(np.float64).reshape(-1, NKV, HD)
    qf = O.f16_to_f32(q.view(np.uint16).reshape(-1)).reshape(q.shape).astype(np.float64)
    out = np.zeros((sub, num_q, HD))
    for t in range(sub):
        for h in range(NKV):
            sel = bi[h, t][bi[h, t] >= 0]
            keys = np.concatenate([np.arange(64 * b, 64 * b + 64) for b in sel])
            keys = keys[keys <= start + t]
            if tree_mask is not None:
                keys = keys[(keys < start) | (((int(tree_mask[t]) >> np.maximum(keys - start, 0)) & 1) == 1)]
            for g in range(gqa):
                s = k64[keys, h] @ qf[t, h * gqa + g] * scale
                w = np.exp(s - s.max())
                out[t, h * gqa + g] = (w @ v64[keys, h]) / w.sum()
    return out


def _sparse_gpu(dev, q, kb, vb, bi, *, num_q, start, sub, top_k, ks, tree_mask=None):
    import torch
    from qengine_amd import kvcache
    pm = torch.zeros((num_q, sub, ks), dtype=torch.float32, device=dev)
    pl = torch.zeros_like(pm)
    po = torch.zeros((num_q, sub, ks, HD), dtype=torch.float32, device=dev)
    out = torch.zeros((sub, num_q, HD), dtype=torch.float16, device=dev)
    tm = None if tree_mask is None else _dev(tree_mask.astype(np.uint32), dev)
    kvcache.attn_block_sparse_split_tq3(_dev(q.view(np.uint16), dev), _dev(kb.view(np.uint8), dev),
                                        _dev(vb.view(np.uint8), dev), _dev(bi, dev), pm, pl, po,
                                        num_q=num_q, num_kv=NKV, start_pos=start, sub_n=sub,
                                        sub_n_max=sub, scale=1 / 16, top_k=top_k, k_splits=ks,
                                        tree_mask=tm)
    kvcache.attn_split_merge(pm, pl, po, out, num_q=num_q, num_kv=NKV, sub_n=sub, sub_n_max=sub,
                             k_splits=ks)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("num_q,top_k,ks,tree", [(16, 8, 8, False), (24, 13, 8, False),
                                                 (16, 64, 8, False), (16, 5, 2, True),
                                                 (24, 30, 4, True)])
def test_sparse_split_vs_oracle(dev, num_q, top_k, ks, tree):
    rng = np.random.default_rng(51 + top_k + ks)
    n, sub = 64 * 90 + 11, 16
    start = n - sub
    kb = O.tq3_encode(kv_f16(rng, n, NKV, HD))
    vb = O.tq3_encode(kv_f16(rng, n, NKV, HD))
    nb = (n + 63) // 64
    kp, kx = _oracle_pools(kb, n, nb)
    q = q_f16(rng, sub, num_q, HD)
    bi = O.block_index_ms(q, kp, kx, num_q=num_q, num_kv=NKV, hd=HD, sub_n=sub, sub_n_max=sub,
                          start_pos=start, top_k=top_k, n_blocks=nb)
    tm = None
    if tree:   # a branching tree: token t sees itself and an ancestor chain
        tm = np.array([(1 << t) | (0 if t == 0 else (1 << ((t - 1) // 2))) | 1 for t in range(sub)],
                      np.uint32)
    print(f"sparse num_q={num_q} top_k={top_k} splits={ks} tree={tree}", flush=True)
    got = _sparse_gpu(dev, q, kb, vb, bi, num_q=num_q, start=start, sub=sub, top_k=top_k, ks=ks,
                      tree_mask=tm)
    pm, pl, po = O.attn_block_sparse_split(q, kb, vb, bi, num_q=num_q, num_kv=NKV, hd=HD,
                                           start_pos=start, sub_n=sub, sub_n_max=sub,
                                           scale=1 / 16, top_k=top_k, k_splits=ks, tree_mask=tm)
    ref = O.attn_split_merge(pm, pl, po, num_q=num_q, num_kv=NKV, hd=HD, sub_n=sub, sub_n_max=sub,
                             k_splits=ks).view(np.float16)
    exact = _exact_selected(q, kb, vb, bi, num_q, start, sub, 1 / 16, tm)
    assert np.all(np.isfinite(got))
    assert_tq3_attn(got, ref, exact)


def test_sparse_verify_step_32k(dev):
    """The reference's verify step at 32768 + 16 keys on the GPU: append the
    block, update the signatures from the first unfrozen block, select
    top_k = 10% of the blocks (capped at 64), attend and merge."""
    import torch
    from qengine_amd import kvcache
    rng = np.random.default_rng(61)
    hist, sub, nq = 32768, 16, 16
    n = hist + sub
    kb = kvcache.tq3_blocks(n * 8, dev)
    vb = kvcache.tq3_blocks(n * 8, dev)
    kvcache.tq3_append_kv(_dev(kv_f16(rng, n, NKV, HD), dev), _dev(kv_f16(rng, n, NKV, HD), dev),
                          kb, vb)
    nb = (n + 63) // 64
    stride = nb + 8
    kp = torch.zeros((NKV, stride, HD), dtype=torch.float16, device=dev)
    kx = torch.zeros_like(kp)
    kvcache.tq3_kpool_update(kb, kp, kx, num_kv=NKV, total_kv=hist, blk_lo=0)
    kvcache.tq3_kpool_update(kb, kp, kx, num_kv=NKV, total_kv=n, blk_lo=(hist - 1) // 64)
    top_k = min(64, max(1, int(nb * 0.10)))
    q = q_f16(rng, sub, nq, HD)
    qd = _dev(q.view(np.uint16), dev)
    bi = torch.zeros((NKV, sub, top_k), dtype=torch.int32, device=dev)
    kvcache.block_index_ms(qd, kp, kx, bi, num_q=nq, num_kv=NKV, sub_n=sub, start_pos=hist,
                           top_k=top_k, n_blocks=nb)
    ks = 8
    pm = torch.zeros((nq, sub, ks), dtype=torch.float32, device=dev)
    pl = torch.zeros_like(pm)
    po = torch.zeros((nq, sub, ks, HD), dtype=torch.float32, device=dev)
    out = torch.zeros((sub, nq, HD), dtype=torch.float16, device=dev)
    kvcache.attn_block_sparse_split_tq3(qd, kb, vb, bi, pm, pl, po, num_q=nq, num_kv=NKV,
                                        start_pos=hist, sub_n=sub, sub_n_max=sub, scale=1 / 16,
                                        top_k=top_k, k_splits=ks)
    kvcache.attn_split_merge(pm, pl, po, out, num_q=nq, num_kv=NKV, sub_n=sub, sub_n_max=sub,
                             k_splits=ks)
    torch.cuda.synchronize()
    kbh = kb.cpu().numpy().view(O.BLOCK_TQ3).reshape(-1)
    vbh = vb.cpu().numpy().view(O.BLOCK_TQ3).reshape(-1)
    ekp, ekx = _oracle_pools(kbh, n, stride)
    assert np.array_equal(kp.cpu().numpy().view(np.uint16), ekp)
    assert np.array_equal(kx.cpu().numpy().view(np.uint16), ekx)
    ebi = O.block_index_ms(q, ekp, ekx, num_q=nq, num_kv=NKV, hd=HD, sub_n=sub, sub_n_max=sub,
                           start_pos=hist, top_k=top_k, n_blocks=nb)
    assert np.array_equal(bi.cpu().numpy(), ebi)
    pm_, pl_, po_ = O.attn_block_sparse_split(q, kbh, vbh, ebi, num_q=nq, num_kv=NKV, hd=HD,
                                              start_pos=hist, sub_n=sub, sub_n_max=sub,
                                              scale=1 / 16, top_k=top_k, k_splits=ks)
    ref = O.attn_split_merge(pm_, pl_, po_, num_q=nq, num_kv=NKV, hd=HD, sub_n=sub, sub_n_max=sub,
                             k_splits=ks).view(np.float16)
    exact = _exact_selected(q, kbh, vbh, ebi, nq, hist, sub, 1 / 16)
    assert_tq3_attn(out.cpu().numpy(), ref, exact)
