"""GPU parity of chunked-prefill attention over a TQ3 cache (BASELINE config 5(i))
against the CPU oracle on identical seeded inputs.

Reference numerics (model.cuh:5189-5214, 5256-5330; attention.cuh:1690-1831):
the history is dequantized to fp16 (tq3_dequantize_kernel), the chunk's own
keys and values stay fp16, and the chunk attends causally (token t sees keys
0 .. start_pos + t).  The oracle builds exactly that fp16 key/value array and
runs its split-K reference decode + merge over it.  The kernel reproduces those
numerics (the history bit-exact to the reference's fp16 dequantization, exact
fp16 products, fp32 sums), so the bar is per row: every (token, head) output
row within 2e-3 of the oracle's, relative to the row's largest magnitude
(tests/_data.rel_err)."""
import numpy as np
import pytest

from oracle import oracle as O
from tests._data import check_rel, kv_f16, q_f16, record_margin

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _torch():
    import torch
    return torch


def _t(a, dev):
    return _torch().from_numpy(np.ascontiguousarray(a)).to(dev)


def _inputs(seed, start_pos, n_tok, num_q, num_kv=4):
    rng = np.random.default_rng(seed)
    hk = kv_f16(rng, max(start_pos, 1), num_kv, 256)[:start_pos]
    hv = kv_f16(rng, max(start_pos, 1), num_kv, 256)[:start_pos]
    ck = kv_f16(rng, n_tok, num_kv, 256)
    cv = kv_f16(rng, n_tok, num_kv, 256)
    q = q_f16(rng, n_tok, num_q, 256)
    return q, hk, hv, ck, cv


def _gpu(dev, q, kb, vb, ck, cv, *, num_q, num_kv, start_pos, scale):
    from qengine_amd import kvcache
    torch = _torch()
    n_tok = q.shape[0]
    out = torch.zeros((n_tok, num_q, 256), dtype=torch.float16, device=dev)
    ws = kvcache.prefill_attn_tq3_workspace(num_q, num_kv, n_tok, start_pos, dev)
    kbt = _t(kb.view(np.uint8), dev) if start_pos else None
    vbt = _t(vb.view(np.uint8), dev) if start_pos else None
    kvcache.prefill_attn_tq3(_t(q, dev), kbt, vbt, _t(ck, dev), _t(cv, dev), out, ws,
                             num_q=num_q, num_kv=num_kv, start_pos=start_pos, scale=scale)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _oracle_kv(kb, vb, ck, cv, num_kv):
    """The reference's fp16 scratch: dequantized history then the raw chunk."""
    hk = O.tq3_decode(kb).view(np.float16).reshape(-1, num_kv, 256) if len(kb) else \
        np.zeros((0, num_kv, 256), np.float16)
    hv = O.tq3_decode(vb).view(np.float16).reshape(-1, num_kv, 256) if len(vb) else \
        np.zeros((0, num_kv, 256), np.float16)
    return np.concatenate([hk, ck]), np.concatenate([hv, cv])


def _oracle(q, k_all, v_all, *, num_q, num_kv, start_pos, scale, k_splits=8):
    n_tok = q.shape[0]
    pm, pl, po = O.attn_split(O.KV_F16, q, k_all, v_all, num_q=num_q, num_kv=num_kv, hd=256,
                              start_pos=start_pos, sub_n=n_tok, sub_n_max=n_tok,
                              active_end_max=start_pos + n_tok, scale=scale, k_splits=k_splits)
    return O.attn_split_merge(pm, pl, po, num_q=num_q, num_kv=num_kv, hd=256, sub_n=n_tok,
                              sub_n_max=n_tok, k_splits=k_splits).view(np.float16)


@pytest.mark.parametrize("start_pos,n_tok,num_q", [
    (0, 40, 16),        # no history: the chunk attends to itself only (64-token workgroup, 8 + 32 tokens)
    (1000, 70, 16),     # partial history tile, partial chunk tiles; the second workgroup's
                        # second 32-token wave group holds no token
    (4096, 128, 16),    # whole tiles
    (777, 33, 24),      # GQA 6 (two workgroups of three heads x two token groups per kv head)
    (300, 1, 16),       # single-token chunk
    (64, 200, 24),
])
def test_prefill_vs_oracle(dev, start_pos, n_tok, num_q):
    num_kv, scale = 4, 1 / 16
    q, hk, hv, ck, cv = _inputs(start_pos * 7 + n_tok, start_pos, n_tok, num_q)
    if start_pos:
        kb, vb = O.tq3_encode(hk), O.tq3_encode(hv)
    else:
        kb = vb = np.zeros(0, O.BLOCK_TQ3)
    got = _gpu(dev, q, kb, vb, ck, cv, num_q=num_q, num_kv=num_kv, start_pos=start_pos,
               scale=scale)
    k_all, v_all = _oracle_kv(kb, vb, ck, cv, num_kv)
    ref = _oracle(q, k_all, v_all, num_q=num_q, num_kv=num_kv, start_pos=start_pos, scale=scale)
    assert np.all(np.isfinite(got))
    check_rel(got, ref, TOL)


@pytest.mark.parametrize("scale,grow", [
    (-1 / 16, False),   # negative scale (carried by the query's sign)
    (0.0, False),       # uniform weights over the visible keys
    (1.0, False),       # peaked weights: the running maximum moves by more than 2^12
    (1 / 16, True),     # keys growing along the sequence: the maximum rises tile after tile
])
def test_prefill_scales_and_rescaling(dev, scale, grow):
    num_q, num_kv, start_pos, n_tok = 16, 4, 700, 80
    q, hk, hv, ck, cv = _inputs(29, start_pos, n_tok, num_q)
    if grow:   # key magnitude rising 1x .. 6x over history and chunk
        ramp = np.linspace(1.0, 6.0, start_pos + n_tok, dtype=np.float32)[:, None, None]
        hk = (hk.astype(np.float32) * ramp[:start_pos]).astype(np.float16)
        ck = (ck.astype(np.float32) * ramp[start_pos:]).astype(np.float16)
    kb, vb = O.tq3_encode(hk), O.tq3_encode(hv)
    got = _gpu(dev, q, kb, vb, ck, cv, num_q=num_q, num_kv=num_kv, start_pos=start_pos,
               scale=scale)
    k_all, v_all = _oracle_kv(kb, vb, ck, cv, num_kv)
    ref = _oracle(q, k_all, v_all, num_q=num_q, num_kv=num_kv, start_pos=start_pos, scale=scale)
    assert np.all(np.isfinite(got))
    check_rel(got, ref, TOL)


def test_prefill_vs_fp64(dev):
    """Independent fp64 softmax reference on the same fp16 key/value array."""
    num_q, num_kv, start_pos, n_tok, scale = 16, 4, 500, 24, 1 / 16
    q, hk, hv, ck, cv = _inputs(11, start_pos, n_tok, num_q)
    kb, vb = O.tq3_encode(hk), O.tq3_encode(hv)
    got = _gpu(dev, q, kb, vb, ck, cv, num_q=num_q, num_kv=num_kv, start_pos=start_pos,
               scale=scale)
    k_all, v_all = _oracle_kv(kb, vb, ck, cv, num_kv)
    ref = O.attn_ref_f64(q, k_all, v_all, num_q=num_q, num_kv=num_kv, hd=256,
                         start_pos=start_pos, sub_n=n_tok, scale=scale)
    check_rel(got, ref, TOL)


def test_prefill_causal_rows_ignore_later_tokens(dev):
    """Token t's row must not change when tokens after t change (causality)."""
    num_q, num_kv, start_pos, n_tok, scale = 16, 4, 256, 96, 1 / 16
    q, hk, hv, ck, cv = _inputs(5, start_pos, n_tok, num_q)
    kb, vb = O.tq3_encode(hk), O.tq3_encode(hv)
    a = _gpu(dev, q, kb, vb, ck, cv, num_q=num_q, num_kv=num_kv, start_pos=start_pos,
             scale=scale)
    ck2, cv2 = ck.copy(), cv.copy()
    ck2[50:] = -ck2[50:]
    cv2[50:] = cv2[50:] * 3
    b = _gpu(dev, q, kb, vb, ck2, cv2, num_q=num_q, num_kv=num_kv, start_pos=start_pos,
             scale=scale)
    assert np.array_equal(a[:50].view(np.uint16), b[:50].view(np.uint16))
    assert not np.array_equal(a[50:].view(np.uint16), b[50:].view(np.uint16))


def test_prefill_config5_full_size(dev):
    """BASELINE config 5(i) at full size: a 131072-token TQ3 history (built by
    the GPU append) and a 2048-token chunk.  64 rows -- eight runs of eight
    consecutive tokens spread over the chunk, its first and last tokens
    included -- against the reference numerics (the oracle over the fp16
    scratch of dequantized history + raw chunk), per row."""
    from qengine_amd import kvcache
    torch = _torch()
    num_q, num_kv, start_pos, n_tok, scale = 16, 4, 131072, 2048, 1 / 16
    rng = np.random.default_rng(55)
    hk = kv_f16(rng, start_pos, num_kv, 256)
    hv = kv_f16(rng, start_pos, num_kv, 256)
    ck = kv_f16(rng, n_tok, num_kv, 256)
    cv = kv_f16(rng, n_tok, num_kv, 256)
    q = q_f16(rng, n_tok, num_q, 256)
    kbt = kvcache.tq3_blocks(start_pos * 8, dev)
    vbt = kvcache.tq3_blocks(start_pos * 8, dev)
    kvcache.tq3_append_kv(_t(hk, dev), _t(hv, dev), kbt, vbt)
    out = torch.zeros((n_tok, num_q, 256), dtype=torch.float16, device=dev)
    ws = kvcache.prefill_attn_tq3_workspace(num_q, num_kv, n_tok, start_pos, dev)
    kvcache.prefill_attn_tq3(_t(q, dev), kbt, vbt, _t(ck, dev), _t(cv, dev), out, ws,
                             num_q=num_q, num_kv=num_kv, start_pos=start_pos, scale=scale)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.all(np.isfinite(got))
    kb = kbt.cpu().numpy().view(O.BLOCK_TQ3).reshape(-1)
    vb = vbt.cpu().numpy().view(O.BLOCK_TQ3).reshape(-1)
    k_all, v_all = _oracle_kv(kb, vb, ck, cv, num_kv)
    worst = 0.0
    for t0 in (0, 293, 585, 877, 1169, 1461, 1753, 2040):
        end = start_pos + t0 + 8
        ref = _oracle(q[t0:t0 + 8], k_all[:end], v_all[:end], num_q=num_q, num_kv=num_kv,
                      start_pos=start_pos + t0, scale=scale, k_splits=32)
        e = check_rel(got[t0:t0 + 8], ref, TOL, what=("config 5(i) rows", t0))
        worst = max(worst, e)
    record_margin("prefill_fullsize_worst_row", err=worst, bar=TOL)
    print(f"config 5(i): worst per-row rel err over 64 rows {worst:.3e}")


# ---------------------------------------------------------------------------
# Multi-token verify (model.cuh:4566-4571, 4663-4687): the verify block is
# appended to the cache first and every key, its own included, is read from
# the cache; causal within the block.  Oracle: the reference split decode over
# the TQ3 cache with sub_n = n_tok.
# ---------------------------------------------------------------------------
def _verify_gpu(dev, q, kb, vb, *, num_q, num_kv, start_pos, scale):
    from qengine_amd import kvcache
    torch = _torch()
    n_tok = q.shape[0]
    out = torch.zeros((n_tok, num_q, 256), dtype=torch.float16, device=dev)
    ws = kvcache.prefill_attn_tq3_workspace(num_q, num_kv, n_tok, start_pos, dev)
    kvcache.prefill_attn_tq3(_t(q, dev), _t(kb.view(np.uint8), dev), _t(vb.view(np.uint8), dev),
                             None, None, out, ws, num_q=num_q, num_kv=num_kv,
                             start_pos=start_pos, scale=scale)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("start_pos,n_tok,num_q", [(1000, 16, 16), (5000, 7, 16), (0, 16, 16),
                                                   (777, 16, 24), (63, 40, 16)])
def test_verify_from_cache_vs_oracle(dev, start_pos, n_tok, num_q):
    num_kv, scale = 4, 1 / 16
    rng = np.random.default_rng(start_pos + 3 * n_tok)
    n = start_pos + n_tok
    kb = O.tq3_encode(kv_f16(rng, n, num_kv, 256))
    vb = O.tq3_encode(kv_f16(rng, n, num_kv, 256))
    q = q_f16(rng, n_tok, num_q, 256)
    got = _verify_gpu(dev, q, kb, vb, num_q=num_q, num_kv=num_kv, start_pos=start_pos, scale=scale)
    pm, pl, po = O.attn_split(O.KV_TQ3, q, kb, vb, num_q=num_q, num_kv=num_kv, hd=256,
                              start_pos=start_pos, sub_n=n_tok, sub_n_max=n_tok,
                              active_end_max=n, scale=scale, k_splits=8)
    ref = O.attn_split_merge(pm, pl, po, num_q=num_q, num_kv=num_kv, hd=256, sub_n=n_tok,
                             sub_n_max=n_tok, k_splits=8).view(np.float16)
    assert np.all(np.isfinite(got))
    check_rel(got, ref, TOL)


def test_verify_matches_decode_path(dev):
    """The MFMA verify and the split-K decode kernel (sub_n = 16) over a
    32768-token cache: the verify per row against the reference oracle, the
    decode to its own bar (tests/_data.assert_tq3_attn), and the two within
    the sum of their bars of each other."""
    from qengine_amd import kvcache
    from tests._data import assert_tq3_attn
    torch = _torch()
    num_q, num_kv, start_pos, n_tok, scale = 16, 4, 32768, 16, 1 / 16
    rng = np.random.default_rng(9)
    n = start_pos + n_tok
    kbt, vbt = kvcache.tq3_blocks(n * 8, dev), kvcache.tq3_blocks(n * 8, dev)
    kvcache.tq3_append_kv(_t(kv_f16(rng, n, num_kv, 256), dev), _t(kv_f16(rng, n, num_kv, 256), dev),
                          kbt, vbt)
    q = q_f16(rng, n_tok, num_q, 256)
    qt = _t(q, dev)
    a = torch.zeros((n_tok, num_q, 256), dtype=torch.float16, device=dev)
    ws = kvcache.prefill_attn_tq3_workspace(num_q, num_kv, n_tok, start_pos, dev)
    kvcache.prefill_attn_tq3(qt, kbt, vbt, None, None, a, ws, num_q=num_q, num_kv=num_kv,
                             start_pos=start_pos, scale=scale)
    b = torch.zeros_like(a)
    wsd = kvcache.decode_attn_tq3_workspace(num_q, num_kv, n_tok, n, dev)
    kvcache.decode_attn_tq3(qt, kbt, vbt, b, wsd, num_q=num_q, num_kv=num_kv, start_pos=start_pos,
                            sub_n=n_tok, scale=scale)
    torch.cuda.synchronize()
    a, b = a.cpu().numpy(), b.cpu().numpy()
    kb = kbt.cpu().numpy().view(O.BLOCK_TQ3).reshape(-1)
    vb = vbt.cpu().numpy().view(O.BLOCK_TQ3).reshape(-1)
    pm, pl, po = O.attn_split(O.KV_TQ3, q, kb, vb, num_q=num_q, num_kv=num_kv, hd=256,
                              start_pos=start_pos, sub_n=n_tok, sub_n_max=n_tok,
                              active_end_max=n, scale=scale, k_splits=8)
    ref = O.attn_split_merge(pm, pl, po, num_q=num_q, num_kv=num_kv, hd=256, sub_n=n_tok,
                             sub_n_max=n_tok, k_splits=8).view(np.float16)
    exact = O.attn_exact_tq3(q, kb, vb, num_q=num_q, num_kv=num_kv, hd=256, start_pos=start_pos,
                             sub_n=n_tok, scale=scale)
    check_rel(a, ref, TOL)
    assert_tq3_attn(b, ref, exact)
    check_rel(a, b, 2 * TOL)
