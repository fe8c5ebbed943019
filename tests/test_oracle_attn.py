"""Pins the oracle's split-K flash decode (attention.cuh:1905-2177, 2633-2801)
and merge (attention.cuh:1837-1891) against an fp64 softmax over the decoded
fp16 K/V, per-split closed forms, and hand-checked visibility cases."""
import numpy as np
import pytest

from oracle import oracle as O
from tests._data import kv_f16, q_f16, rel_err


def _softmax_f64(q, k, v, keys, scale):
    """Brute force numpy softmax for one head: q [hd], k/v [n][hd], keys: list."""
    if len(keys) == 0:
        return np.zeros(q.shape[-1])
    s = (k[keys] @ q) * scale
    w = np.exp(s - s.max())
    return (w[:, None] * v[keys]).sum(0) / w.sum()


def test_key_visible_hand_cases():
    # causal only
    assert O.key_visible(9, 10, 0) and not O.key_visible(11, 10, 0)
    assert O.key_visible(10, 10, 0)                    # own position
    # sink 32 / window 64, query at abs pos 1000 (active_end 1001): tiles are 32-aligned
    assert O.key_visible(31, 1000, 0, 32, 64)          # sink tile
    assert not O.key_visible(32, 1000, 0, 32, 64)
    # window lower edge 937: tile [928,960) ends at 960 > 937 -> kept whole
    assert O.key_visible(928, 1000, 0, 32, 64)
    assert not O.key_visible(927, 1000, 0, 32, 64)     # tile [896,928) ends at 928 <= 937
    # sink only: even the own tile is dropped (reference tile rule)
    assert not O.key_visible(1000, 1000, 0, 32, 0)
    # tree mask bits apply at keys >= start_pos only
    tm = np.array([0b1, 0b11, 0b101], np.uint32)
    assert O.key_visible(5, 10, 2, 0, 0, tm)
    assert O.key_visible(10, 10, 2, 0, 0, tm) and not O.key_visible(11, 10, 2, 0, 0, tm)
    assert O.key_visible(12, 10, 2, 0, 0, tm)


def test_attn_ref_f64_vs_numpy_bruteforce():
    rng = np.random.default_rng(11)
    num_q, num_kv, hd, start, sub_n = 4, 2, 64, 37, 3
    n = start + sub_n
    k = rng.standard_normal((n, num_kv, hd)).astype(np.float16)
    v = rng.standard_normal((n, num_kv, hd)).astype(np.float16)
    q = q_f16(rng, sub_n, num_q, hd)
    tm = np.array([0b001, 0b011, 0b101], np.uint32)
    out = O.attn_ref_f64(q, k, v, num_q=num_q, num_kv=num_kv, hd=hd, start_pos=start,
                         sub_n=sub_n, scale=0.125, tree_mask=tm)
    for t in range(sub_n):
        for h in range(num_q):
            kvh = h // (num_q // num_kv)
            keys = list(range(start)) + [start + j for j in range(sub_n) if (tm[t] >> j) & 1 and j <= t]
            ref = _softmax_f64(q[t, h].astype(np.float64), k[:, kvh].astype(np.float64),
                               v[:, kvh].astype(np.float64), keys, 0.125)
            assert np.allclose(out[t, h], ref, atol=1e-12)


def _tq3_cache(rng, n, num_kv, hd):
    k16 = kv_f16(rng, n, num_kv, hd)
    v16 = kv_f16(rng, n, num_kv, hd)
    kb = O.tq3_encode(k16)
    vb = O.tq3_encode(v16)
    kd = O.tq3_decode(kb).view(np.float16).reshape(n, num_kv, hd)
    vd = O.tq3_decode(vb).view(np.float16).reshape(n, num_kv, hd)
    return kb, vb, kd, vd


@pytest.mark.parametrize("n,k_splits,sub_n,num_q", [(300, 1, 1, 16), (1111, 8, 1, 16),
                                                    (777, 3, 4, 16), (640, 8, 2, 24)])
def test_split_merge_vs_fp64(n, k_splits, sub_n, num_q):
    rng = np.random.default_rng(n + k_splits)
    num_kv, hd = 4, 256
    start = n - sub_n
    kb, vb, kd, vd = _tq3_cache(rng, n, num_kv, hd)
    q = q_f16(rng, sub_n, num_q, hd)
    scale = 1.0 / np.sqrt(hd)
    pm, pl, po = O.attn_split(O.KV_TQ3, q, kb, vb, num_q=num_q, num_kv=num_kv, hd=hd,
                              start_pos=start, sub_n=sub_n, sub_n_max=16, active_end_max=n,
                              scale=scale, k_splits=k_splits)
    out = O.attn_split_merge(pm, pl, po, num_q=num_q, num_kv=num_kv, hd=hd, sub_n=sub_n,
                             sub_n_max=16, k_splits=k_splits)
    ref = O.attn_ref_f64(q, kd, vd, num_q=num_q, num_kv=num_kv, hd=hd, start_pos=start,
                         sub_n=sub_n, scale=scale)
    assert rel_err(out.view(np.float16), ref) < 1e-3


def test_split_partials_closed_form():
    """Each split's (m, l, o) is max / sum exp / exp-weighted V over the
    reference's split token range [z*tps*32, min((z+1)*tps*32, end))."""
    rng = np.random.default_rng(12)
    num_q, num_kv, hd, n, ks = 8, 2, 256, 500, 5
    kb, vb, kd, vd = _tq3_cache(rng, n, num_kv, hd)
    q = q_f16(rng, 1, num_q, hd)
    scale = 0.0625
    pm, pl, po = O.attn_split(O.KV_TQ3, q, kb, vb, num_q=num_q, num_kv=num_kv, hd=hd,
                              start_pos=n - 1, sub_n=1, sub_n_max=1, active_end_max=n,
                              scale=scale, k_splits=ks)
    tiles = (n + 31) // 32
    tps = (tiles + ks - 1) // ks
    for h in range(num_q):
        kvh = h // (num_q // num_kv)
        s_all = (kd[:, kvh].astype(np.float64) @ q[0, h].astype(np.float64)) * scale
        for z in range(ks):
            lo, hi = z * tps * 32, min((z + 1) * tps * 32, n)
            if lo >= hi:
                assert pm[h, 0, z] == -np.inf and pl[h, 0, z] == 0 and np.all(po[h, 0, z] == 0)
                continue
            s = s_all[lo:hi]
            m = s.max()
            w = np.exp(s - m)
            assert abs(pm[h, 0, z] - m) < 1e-4 * max(1, abs(m))
            assert abs(pl[h, 0, z] - w.sum()) < 1e-4 * w.sum()
            o = (w[:, None] * vd[lo:hi, kvh].astype(np.float64)).sum(0)
            assert np.max(np.abs(po[h, 0, z] - o)) < 1e-4 * np.max(np.abs(o))


def test_split_count_invariance():
    rng = np.random.default_rng(13)
    num_q, num_kv, hd, n = 16, 4, 256, 900
    kb, vb, _, _ = _tq3_cache(rng, n, num_kv, hd)
    q = q_f16(rng, 1, num_q, hd)
    outs = []
    for ks in (1, 2, 7, 16):
        pm, pl, po = O.attn_split(O.KV_TQ3, q, kb, vb, num_q=num_q, num_kv=num_kv, hd=hd,
                                  start_pos=n - 1, sub_n=1, sub_n_max=1, active_end_max=n,
                                  scale=1 / 16, k_splits=ks)
        outs.append(O.attn_split_merge(pm, pl, po, num_q=num_q, num_kv=num_kv, hd=hd,
                                       sub_n=1, sub_n_max=1, k_splits=ks).view(np.float16))
    for o in outs[1:]:
        assert rel_err(o, outs[0]) < 1e-3


@pytest.mark.parametrize("sink,window,tree", [(0, 0, True), (32, 64, False), (64, 100, True)])
def test_verify_masks_vs_fp64(sink, window, tree):
    rng = np.random.default_rng(14 + sink)
    num_q, num_kv, hd, sub_n = 16, 4, 256, 16
    n = 1200
    start = n - sub_n
    kb, vb, kd, vd = _tq3_cache(rng, n, num_kv, hd)
    q = q_f16(rng, sub_n, num_q, hd)
    tm = None
    if tree:
        # BFS tree: node t attends itself and a random subset of earlier nodes
        tm = np.array([(1 << t) | int(rng.integers(0, 1 << max(t, 1))) & ((1 << t) - 1)
                       for t in range(sub_n)], np.uint32)
    scale = 1 / 16
    pm, pl, po = O.attn_split(O.KV_TQ3, q, kb, vb, num_q=num_q, num_kv=num_kv, hd=hd,
                              start_pos=start, sub_n=sub_n, sub_n_max=16, active_end_max=n,
                              scale=scale, k_splits=8, sink_tok=sink, window_tok=window,
                              tree_mask=tm)
    out = O.attn_split_merge(pm, pl, po, num_q=num_q, num_kv=num_kv, hd=hd, sub_n=sub_n,
                             sub_n_max=16, k_splits=8)
    ref = O.attn_ref_f64(q, kd, vd, num_q=num_q, num_kv=num_kv, hd=hd, start_pos=start,
                         sub_n=sub_n, scale=scale, sink_tok=sink, window_tok=window,
                         tree_mask=tm)
    assert rel_err(out.view(np.float16), ref) < 1e-3


def test_q8_split_vs_fp64():
    rng = np.random.default_rng(15)
    num_q, num_kv, hd, n = 16, 4, 256, 700
    k16 = kv_f16(rng, n, num_kv, hd, outlier_frac=0)
    v16 = kv_f16(rng, n, num_kv, hd, outlier_frac=0)
    kb, vb = O.q8_encode(k16), O.q8_encode(v16)
    kd = O.q8_decode(kb).reshape(n, num_kv, hd)
    vd = O.q8_decode(vb).reshape(n, num_kv, hd)
    q = q_f16(rng, 1, num_q, hd)
    pm, pl, po = O.attn_split(O.KV_Q8, q, kb, vb, num_q=num_q, num_kv=num_kv, hd=hd,
                              start_pos=n - 1, sub_n=1, sub_n_max=1, active_end_max=n,
                              scale=1 / 16, k_splits=8)
    out = O.attn_split_merge(pm, pl, po, num_q=num_q, num_kv=num_kv, hd=hd, sub_n=1,
                             sub_n_max=1, k_splits=8)
    ref = O.attn_ref_f64(q, kd, vd, num_q=num_q, num_kv=num_kv, hd=hd, start_pos=n - 1,
                         sub_n=1, scale=1 / 16)
    assert rel_err(out.view(np.float16), ref) < 1e-3


def test_merge_skips_empty_and_nonfinite_splits():
    hd = 8
    pm = np.array([[[1.0, -np.inf, 2.0, 0.5]]], np.float32)
    pl = np.array([[[2.0, 0.0, 1.0, 0.0]]], np.float32)
    po = np.zeros((1, 1, 4, hd), np.float32)
    po[0, 0, 0] = 4.0
    po[0, 0, 1] = np.nan
    po[0, 0, 2] = 1.0
    po[0, 0, 3] = 100.0       # l == 0 -> skipped
    out = O.attn_split_merge(pm, pl, po, num_q=1, num_kv=1, hd=hd, sub_n=1, sub_n_max=1,
                             k_splits=4).view(np.float16).astype(np.float64)
    w0, w2 = np.exp(1.0 - 2.0), 1.0
    ref = (w0 * 4.0 + w2 * 1.0) / (w0 * 2.0 + w2 * 1.0)
    assert np.allclose(out, ref, rtol=1e-3)
    # all splits empty -> zeros
    z = O.attn_split_merge(np.full((1, 1, 2), -np.inf, np.float32), np.zeros((1, 1, 2), np.float32),
                           np.zeros((1, 1, 2, hd), np.float32), num_q=1, num_kv=1, hd=hd,
                           sub_n=1, sub_n_max=1, k_splits=2)
    assert np.all(z == 0)


def test_q8k_tq3v_vs_fp64_and_closed_form():
    """Mixed-format oracle (Q8_0 keys, TQ3 values) against attn_ref_f64 over the
    same decoded rows (values rounded to fp16 for it: within 2e-3), and the
    closed form: with every key equal, each query's output is the mean of the
    visible values."""
    rng = np.random.default_rng(41)
    n, nq, nkv, sub_n = 300, 16, 4, 3
    k16, v16 = kv_f16(rng, n, nkv, 256), kv_f16(rng, n, nkv, 256)
    kq, vt = O.q8_encode(k16), O.tq3_encode(v16)
    q = q_f16(rng, sub_n, nq, 256)
    kw = dict(num_q=nq, num_kv=nkv, hd=256, start_pos=n - sub_n, sub_n=sub_n, scale=1 / 16)
    got = O.attn_q8k_tq3v_f64(q, kq, vt, **kw)
    ref = O.attn_ref_f64(q, O.q8_decode(kq), O.tq3_decode(vt), **kw)
    assert rel_err(got, ref) < 2e-3
    same = O.q8_encode(np.tile(k16[:1], (n, 1, 1)))
    flat = O.attn_q8k_tq3v_f64(q, same, vt, **kw)
    v32 = O.tq3_decode_f32(vt).astype(np.float64).reshape(n, nkv, 256)
    for t in range(sub_n):
        mean = v32[:n - sub_n + t + 1].mean(axis=0)               # [nkv][256]
        assert np.allclose(flat[t], np.repeat(mean, nq // nkv, axis=0), rtol=1e-9, atol=1e-12)


def test_attn_ref_f32kv_matches_f16_core():
    """The float-input fp64 reference is the fp16-input one on fp16-representable
    rows (bit for bit), masks included; the exact-TQ3 truth is that reference
    over tq3_decode_f32 (pinned in test_oracle_codec), which differs from the
    fp16-rounded dequantization by the reference's own rounding only."""
    rng = np.random.default_rng(11)
    n, nq, nkv = 300, 8, 2
    k16, v16 = kv_f16(rng, n, nkv, 256), kv_f16(rng, n, nkv, 256)
    q = q_f16(rng, 4, nq, 256)
    kw = dict(num_q=nq, num_kv=nkv, hd=256, start_pos=n - 4, sub_n=4, scale=1 / 16)
    tm = np.array([1, 3, 5, 15], np.uint32)
    for extra in ({}, {"sink_tok": 32, "window_tok": 64}, {"tree_mask": tm}):
        a = O.attn_ref_f64(q, k16, v16, **kw, **extra)
        b = O.attn_ref_f64_f32kv(q, O.f16_to_f32(k16.view(np.uint16)),
                                 O.f16_to_f32(v16.view(np.uint16)), **kw, **extra)
        assert np.array_equal(a, b)
    kb, vb = O.tq3_encode(k16), O.tq3_encode(v16)
    ex = O.attn_exact_tq3(q, kb, vb, **kw)
    rd = O.attn_ref_f64(q, O.tq3_decode(kb), O.tq3_decode(vb), **kw)
    assert 0 < rel_err(rd, ex) < 5e-3
