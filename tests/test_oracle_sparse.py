"""Pins the oracle's block-sparse TQ3 verify (attention.cuh:2193-2533,
sparse_attn/sparse_index.cuh:214-330) with independent checks:

- K-pool signatures against numpy over the bulk-dequantized fp16 keys
  (float32 sequential sum / count, first largest |x|), and an incremental
  update leaving earlier blocks alone;
- block index: rows ascending, -1 padded, no duplicates, nothing past the
  causal block; the selected set equals the top_k of the fp64 scores wherever
  the fp64 ranking has a margin above fp32 rounding; equal scores resolve to
  the lower block index; fewer visible blocks than top_k pad with -1;
- sparse attention: merged output against numpy fp64 softmax attention over
  exactly the selected blocks' visible keys (fp16 dequantized values), per
  element within half an fp16 ulp + 2e-6 of the row maximum; selecting every
  block reproduces the dense oracle."""
import numpy as np
import pytest

from oracle import oracle as O
from tests._data import kv_f16, q_f16, rel_err

HD, NKV = 256, 4


def _cache(seed, n):
    rng = np.random.default_rng(seed)
    return rng, O.tq3_encode(kv_f16(rng, n, NKV, HD)), O.tq3_encode(kv_f16(rng, n, NKV, HD))


def _pools(kb, n, stride):
    kp = np.zeros((NKV, stride, HD), np.uint16)
    kx = np.zeros_like(kp)
    O.tq3_kpool_update(kb, kp, kx, num_kv=NKV, hd=HD, total_kv=n, blk_lo=0)
    return kp, kx


def test_kpool_vs_numpy():
    n = 64 * 9 + 21
    rng, kb, _ = _cache(1, n)
    stride = 12
    kp, kx = _pools(kb, n, stride)
    k16 = O.f16_to_f32(O.tq3_decode(kb).reshape(-1)).reshape(n, NKV, HD)
    for h in range(NKV):
        for b in range((n + 63) // 64):
            x = k16[64 * b:min(64 * b + 64, n), h]
            mean = (np.cumsum(x, axis=0, dtype=np.float32)[-1] / np.float32(len(x))).astype(np.float16)
            amax = x[np.argmax(np.abs(x), axis=0), np.arange(HD)].astype(np.float16)
            amax[np.abs(x).max(axis=0) == 0] = 0
            assert np.array_equal(kp[h, b], mean.view(np.uint16)), (h, b)
            assert np.array_equal(kx[h, b], amax.view(np.uint16)), (h, b)
    assert np.all(kp[:, 10:] == 0) and np.all(kx[:, 10:] == 0)
    # incremental: rebuild from block 5 after rows changed only there
    kb2 = kb.copy()
    kb2[(64 * 7) * 8:] = O.tq3_encode(kv_f16(rng, n - 64 * 7, NKV, HD))
    kp2, kx2 = kp.copy(), kx.copy()
    O.tq3_kpool_update(kb2, kp2, kx2, num_kv=NKV, hd=HD, total_kv=n, blk_lo=5)
    full_p, full_x = _pools(kb2, n, stride)
    assert np.array_equal(kp2[:, :5], kp[:, :5]) and np.array_equal(kp2[:, 5:], full_p[:, 5:])
    assert np.array_equal(kx2[:, 5:], full_x[:, 5:])


def _scores64(q, kp, kx, num_q, t, nb, beta=0.5):
    gqa = num_q // NKV
    qf = O.f16_to_f32(q.view(np.uint16).reshape(-1)).reshape(q.shape).astype(np.float64)
    out = []
    for h in range(NKV):
        qa = np.float16(qf[t, h * gqa:(h + 1) * gqa].sum(0) / gqa).astype(np.float64)
        mn = O.f16_to_f32(kp[h, :nb].reshape(-1)).reshape(nb, HD).astype(np.float64)
        mx = O.f16_to_f32(kx[h, :nb].reshape(-1)).reshape(nb, HD).astype(np.float64)
        out.append(np.maximum(mn @ qa, beta * (mx @ qa)))
    return np.stack(out)


@pytest.mark.parametrize("num_q,top_k", [(16, 8), (24, 5), (16, 64)])
def test_block_index_vs_f64_ranking(num_q, top_k):
    n, sub, start = 64 * 70 + 9, 8, 64 * 70 + 1
    rng, kb, _ = _cache(2 + top_k, n)
    nb = (n + 63) // 64
    kp, kx = _pools(kb, n, nb)
    q = q_f16(rng, sub, num_q, HD)
    bi = O.block_index_ms(q, kp, kx, num_q=num_q, num_kv=NKV, hd=HD, sub_n=sub, sub_n_max=sub,
                          start_pos=start, top_k=top_k, n_blocks=nb)
    for t in range(sub):
        s64 = _scores64(q, kp, kx, num_q, t, nb)
        cmax = (start + t) // 64
        for h in range(NKV):
            row = bi[h, t]
            sel = row[row >= 0]
            assert np.all(np.diff(sel) > 0) and np.all(row[len(sel):] == -1)
            assert sel.max() <= cmax
            vis = s64[h, :cmax + 1]
            k = min(top_k, len(vis))
            assert len(sel) == k
            order = np.sort(vis)[::-1]
            kth = order[k - 1]
            margin = 1e-4 * np.abs(vis).max()
            must = np.nonzero(vis > kth + margin)[0]
            never = np.nonzero(vis < kth - margin)[0]
            assert set(must) <= set(sel) and not (set(never) & set(sel)), (h, t)


def test_block_scores_pairwise_order_and_selection():
    """block_scores_ms against a numpy float32 restatement of the pair order
    (exact fp16 x fp16 products, each pair's sum rounded once, then added to
    the running sum), bit for bit; -inf past each query's causal block; and
    block_index_ms is the first top_k of (score descending, block ascending)
    over those scores, listed ascending."""
    n, sub, start = 64 * 40 + 5, 4, 64 * 33 + 2
    rng, kb, _ = _cache(8, n)
    nb = (n + 63) // 64
    kp, kx = _pools(kb, n, nb)
    q = q_f16(rng, sub, 16, HD)
    sc = O.block_scores_ms(q, kp, kx, num_q=16, num_kv=NKV, hd=HD, sub_n=sub, start_pos=start,
                           n_blocks=nb, beta=0.5)
    gqa = 16 // NKV
    qf = O.f16_to_f32(q.view(np.uint16).reshape(-1)).reshape(q.shape)
    for h in range(NKV):
        mn = O.f16_to_f32(kp[h, :nb].reshape(-1)).reshape(nb, HD)
        mx = O.f16_to_f32(kx[h, :nb].reshape(-1)).reshape(nb, HD)
        for t in range(sub):
            acc = np.zeros(HD, np.float32)
            for g in range(gqa):
                acc = acc + qf[t, h * gqa + g]
            qa = np.float16(acc * np.float32(1.0 / gqa)).astype(np.float32)
            s_mean = np.zeros(nb, np.float32)
            s_max = np.zeros(nb, np.float32)
            for c in range(0, HD, 2):
                s_mean = s_mean + (qa[c] * mn[:, c] + qa[c + 1] * mn[:, c + 1])
                s_max = s_max + (qa[c] * mx[:, c] + qa[c + 1] * mx[:, c + 1])
            ref = np.maximum(s_mean, np.float32(0.5) * s_max)
            cmax = (start + t) // 64
            ref[cmax + 1:] = -np.inf
            assert np.array_equal(sc[h, t].view(np.uint32), ref.view(np.uint32)), (h, t)
    for top_k in (1, 7, 40):
        bi = O.block_index_ms(q, kp, kx, num_q=16, num_kv=NKV, hd=HD, sub_n=sub, sub_n_max=sub,
                              start_pos=start, top_k=top_k, n_blocks=nb)
        for h in range(NKV):
            for t in range(sub):
                v = sc[h, t]
                ok = np.nonzero(v > -np.inf)[0]
                order = ok[np.lexsort((ok, -v[ok]))][:top_k]
                exp = np.full(top_k, -1, np.int32)
                exp[:len(order)] = np.sort(order)
                assert np.array_equal(bi[h, t], exp), (top_k, h, t)


def test_block_index_ties_and_padding():
    n = 64 * 10
    rng, kb, _ = _cache(5, n)
    nb = 10
    kp, kx = _pools(kb, n, nb)
    kp[:, :] = kp[:, 3:4]          # every block's signature equal: all scores tie
    kx[:, :] = kx[:, 3:4]
    q = q_f16(rng, 2, 16, HD)
    bi = O.block_index_ms(q, kp, kx, num_q=16, num_kv=NKV, hd=HD, sub_n=2, sub_n_max=2,
                          start_pos=64 * 4 + 3, top_k=3, n_blocks=nb)
    assert np.all(bi == np.array([0, 1, 2]))                 # lowest indices win ties
    bi = O.block_index_ms(q, kp, kx, num_q=16, num_kv=NKV, hd=HD, sub_n=2, sub_n_max=2,
                          start_pos=64 * 2 + 3, top_k=6, n_blocks=nb)
    assert np.all(bi[:, :, :3] == np.array([0, 1, 2])) and np.all(bi[:, :, 3:] == -1)


def _sparse_f64(q, kb, vb, bi, num_q, start, sub, scale):
    gqa = num_q // NKV
    k64 = O.f16_to_f32(O.tq3_decode(kb).reshape(-1)).reshape(-1, NKV, HD).astype(np.float64)
    v64 = O.f16_to_f32(O.tq3_decode(vb).reshape(-1)).reshape(-1, NKV, HD).astype(np.float64)
    qf = O.f16_to_f32(q.view(np.uint16).reshape(-1)).reshape(q.shape).astype(np.float64)
    out = np.zeros((sub, num_q, HD))
    for t in range(sub):
        for h in range(NKV):
            sel = bi[h, t][bi[h, t] >= 0]
            keys = np.concatenate([np.arange(64 * b, 64 * b + 64) for b in sel]) if len(sel) else \
                np.zeros(0, int)
            keys = keys[keys <= start + t]
            for g in range(gqa):
                s = k64[keys, h] @ qf[t, h * gqa + g] * scale
                w = np.exp(s - s.max())
                out[t, h * gqa + g] = (w @ v64[keys, h]) / w.sum()
    return out


@pytest.mark.parametrize("top_k,k_splits", [(5, 8), (13, 8), (3, 2)])
def test_sparse_split_vs_f64(top_k, k_splits):
    n, sub, nq = 64 * 30 + 7, 6, 16
    start = n - sub
    rng, kb, vb = _cache(9 + top_k, n)
    nb = (n + 63) // 64
    kp, kx = _pools(kb, n, nb)
    q = q_f16(rng, sub, nq, HD)
    bi = O.block_index_ms(q, kp, kx, num_q=nq, num_kv=NKV, hd=HD, sub_n=sub, sub_n_max=sub,
                          start_pos=start, top_k=top_k, n_blocks=nb)
    pm, pl, po = O.attn_block_sparse_split(q, kb, vb, bi, num_q=nq, num_kv=NKV, hd=HD,
                                           start_pos=start, sub_n=sub, sub_n_max=sub,
                                           scale=1 / 16, top_k=top_k, k_splits=k_splits)
    got = O.attn_split_merge(pm, pl, po, num_q=nq, num_kv=NKV, hd=HD, sub_n=sub, sub_n_max=sub,
                             k_splits=k_splits).view(np.float16).astype(np.float64)
    ref = _sparse_f64(q, kb, vb, bi, nq, start, sub, 1 / 16)
    a = np.abs(ref)
    half_ulp = 0.5 * 2.0 ** (np.floor(np.log2(np.maximum(a, 2.0 ** -14))) - 10)
    bound = half_ulp * 1.0001 + 2e-6 * a.max(axis=-1, keepdims=True)
    assert np.all(np.abs(got - ref) <= bound)


def test_sparse_all_blocks_is_dense():
    n, sub, nq = 64 * 20 + 5, 4, 24
    start = n - sub
    rng, kb, vb = _cache(31, n)
    nb = (n + 63) // 64
    bi = np.tile(np.arange(nb, dtype=np.int32), (NKV, sub, 1))
    pm, pl, po = O.attn_block_sparse_split(q := q_f16(rng, sub, nq, HD), kb, vb, bi, num_q=nq,
                                           num_kv=NKV, hd=HD, start_pos=start, sub_n=sub,
                                           sub_n_max=sub, scale=1 / 16, top_k=nb, k_splits=8)
    got = O.attn_split_merge(pm, pl, po, num_q=nq, num_kv=NKV, hd=HD, sub_n=sub, sub_n_max=sub,
                             k_splits=8).view(np.float16)
    pm, pl, po = O.attn_split(O.KV_TQ3, q, kb, vb, num_q=nq, num_kv=NKV, hd=HD, start_pos=start,
                              sub_n=sub, sub_n_max=sub, active_end_max=n, scale=1 / 16, k_splits=8)
    ref = O.attn_split_merge(pm, pl, po, num_q=nq, num_kv=NKV, hd=HD, sub_n=sub, sub_n_max=sub,
                             k_splits=8).view(np.float16)
    assert rel_err(got, ref) < 1e-3
