"""GPU parity of the Q8_0 split-K flash decode (attention.cuh:2633-2801) and its
merge (attention.cuh:1837-1891) against the CPU oracle on identical seeded
inputs.  Bar: merged output within 2e-3 relative error (max |diff| / max |ref|),
fp32 accumulation; split partials within the same tolerance."""
import numpy as np
import pytest

from oracle import oracle as O
from tests._data import check_rel, kv_f16, q_f16

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
    return rng, O.q8_encode(k16), O.q8_encode(v16)


def _run(dev, q, kb, vb, **kw):
    from qengine_amd import kvcache
    torch = _torch()
    nq, smax, ks = kw["num_q"], kw["sub_n_max"], kw["k_splits"]
    pm = torch.full((nq, smax, ks), float("nan"), device=dev)
    pl = torch.full((nq, smax, ks), float("nan"), device=dev)
    po = torch.full((nq, smax, ks, 256), float("nan"), device=dev)
    kvcache.attn_split_q8(_dev(q.view(np.uint16), dev), _dev(kb.view(np.uint8), dev),
                          _dev(vb.view(np.uint8), dev), pm, pl, po, **kw)
    out = torch.zeros((kw["sub_n"], nq, 256), dtype=torch.float16, device=dev)
    kvcache.attn_split_merge(pm, pl, po, out, num_q=nq, num_kv=kw["num_kv"], sub_n=kw["sub_n"],
                             sub_n_max=smax, k_splits=ks)
    torch.cuda.synchronize()
    return pm.cpu().numpy(), pl.cpu().numpy(), po.cpu().numpy(), out.cpu().numpy()


@pytest.mark.parametrize("n,k_splits,num_q,sub_n", [
    (4097, 8, 16, 1),      # config 2: one token appended to a 4096-token Q8 cache
    (4097, 16, 16, 1),
    (1000, 8, 16, 1),
    (33, 8, 16, 1),
    (1, 4, 16, 1),
    (700, 8, 24, 1),       # GQA 6
    (530, 4, 16, 16),      # 16 causal queries (verify-style)
])
def test_q8_split_decode_vs_oracle(dev, n, k_splits, num_q, sub_n):
    rng, kb, vb = _cache(300 + n + k_splits, n)
    q = q_f16(rng, sub_n, num_q, 256)
    kw = dict(num_q=num_q, num_kv=4, start_pos=n - sub_n, sub_n=sub_n, sub_n_max=sub_n,
              active_end_max=n, scale=1 / 16, k_splits=k_splits)
    pm, pl, po, out = _run(dev, q, kb, vb, **kw)
    em, el, eo = O.attn_split(O.KV_Q8, q, kb, vb, hd=256, **kw)
    exp = O.attn_split_merge(em, el, eo, num_q=num_q, num_kv=4, hd=256, sub_n=sub_n,
                             sub_n_max=sub_n, k_splits=k_splits)
    # partials: same empty-split pattern, m/l/o within tolerance after a common rescale
    empty = ~np.isfinite(em)
    assert np.array_equal(empty, ~np.isfinite(pm)), "empty-split pattern differs"
    assert np.all(pl[empty] == 0) and np.all(po[empty] == 0)
    live = ~empty
    assert np.max(np.abs(pm[live] - em[live])) < 1e-2
    w = np.exp(pm[live] - em[live])
    assert np.max(np.abs(pl[live] * w - el[live]) / el[live]) < TOL
    check_rel(po[live] * w[:, None], eo[live], TOL)
    check_rel(out, exp.view(np.float16), TOL)


def test_q8_split_rejects_bad_shapes(dev):
    from qengine_amd import QKVError, kvcache
    torch = _torch()
    q = torch.zeros((1, 16, 256), dtype=torch.float16, device=dev)
    kv = torch.zeros((10 * 32, 36), dtype=torch.uint8, device=dev)
    pm = torch.zeros((16, 1, 8), device=dev)
    po = torch.zeros((16, 1, 8, 256), device=dev)
    with pytest.raises(QKVError):   # head_dim 128 is not compiled
        kvcache.attn_split_q8(q, kv, kv, pm, pm, po, num_q=16, num_kv=4, start_pos=9, sub_n=1,
                              sub_n_max=1, active_end_max=10, scale=1 / 16, k_splits=8,
                              head_dim=128)
    with pytest.raises(QKVError):   # sub_n > sub_n_max
        kvcache.attn_split_q8(q, kv, kv, pm, pm, po, num_q=16, num_kv=4, start_pos=9, sub_n=2,
                              sub_n_max=1, active_end_max=10, scale=1 / 16, k_splits=8)


def _expected(q, kb, vb, n, num_q, sub_n):
    kw = dict(num_q=num_q, num_kv=4, start_pos=n - sub_n, sub_n=sub_n, sub_n_max=sub_n,
              active_end_max=n, scale=1 / 16, k_splits=8)
    em, el, eo = O.attn_split(O.KV_Q8, q, kb, vb, hd=256, **kw)
    return O.attn_split_merge(em, el, eo, num_q=num_q, num_kv=4, hd=256, sub_n=sub_n,
                              sub_n_max=sub_n, k_splits=8).view(np.float16)


@pytest.mark.parametrize("n,num_q,sub_n", [
    (4097, 16, 1),     # config 2
    (1, 16, 1), (127, 16, 1), (129, 16, 1), (16384, 16, 1), (20000, 16, 1),
    (700, 24, 1),      # GQA 6
    (530, 16, 16),     # 16 causal queries
])
def test_q8_fast_decode_vs_oracle(dev, n, num_q, sub_n):
    """Single-launch Q8 decode (records merged in the kernel) against the
    oracle's reference split + merge."""
    from qengine_amd import kvcache
    torch = _torch()
    rng, kb, vb = _cache(700 + n + sub_n, n)
    q = q_f16(rng, sub_n, num_q, 256)
    ws = kvcache.decode_attn_q8_workspace(num_q, 4, sub_n, n, dev)
    out = torch.zeros((sub_n, num_q, 256), dtype=torch.float16, device=dev)
    kvcache.decode_attn_q8(_dev(q.view(np.uint16), dev), _dev(kb.view(np.uint8), dev),
                           _dev(vb.view(np.uint8), dev), out, ws, num_q=num_q, num_kv=4,
                           start_pos=n - sub_n, sub_n=sub_n, scale=1 / 16)
    torch.cuda.synchronize()
    check_rel(out.cpu().numpy(), _expected(q, kb, vb, n, num_q, sub_n), TOL)


def test_q8_fast_decode_workspace_reuse(dev):
    """One workspace across calls of different lengths and query counts."""
    from qengine_amd import kvcache
    torch = _torch()
    ws = kvcache.decode_attn_q8_workspace(16, 4, 4, 8192, dev)
    for i, (n, sub_n) in enumerate([(8192, 1), (4097, 1), (1000, 4), (8192, 1), (300, 4)]):
        rng, kb, vb = _cache(800 + i, n)
        q = q_f16(rng, sub_n, 16, 256)
        out = torch.zeros((sub_n, 16, 256), dtype=torch.float16, device=dev)
        kvcache.decode_attn_q8(_dev(q.view(np.uint16), dev), _dev(kb.view(np.uint8), dev),
                               _dev(vb.view(np.uint8), dev), out, ws, num_q=16, num_kv=4,
                               start_pos=n - sub_n, sub_n=sub_n, scale=1 / 16)
        torch.cuda.synchronize()
        check_rel(out.cpu().numpy(), _expected(q, kb, vb, n, 16, sub_n), TOL, what=(n, sub_n))


def test_q8_append_kv_matches_two_appends(dev):
    from qengine_amd import kvcache
    torch = _torch()
    g = torch.Generator(device=dev).manual_seed(11)
    k = torch.randn(3000 * 32, generator=g, device=dev).half()
    v = torch.randn(3000 * 32, generator=g, device=dev).half()
    a1, a2 = kvcache.q8_blocks(3000, dev), kvcache.q8_blocks(3000, dev)
    b1, b2 = kvcache.q8_blocks(3000, dev), kvcache.q8_blocks(3000, dev)
    kvcache.q8_append_kv(k, v, a1, a2)
    kvcache.q8_append(k, b1)
    kvcache.q8_append(v, b2)
    torch.cuda.synchronize()
    assert torch.equal(a1, b1) and torch.equal(a2, b2)


@pytest.mark.parametrize("n_old,num_q", [
    (4096, 16),    # config 2: 4096 cached keys + the new one
    (0, 16), (31, 16), (32, 16), (127, 16), (128, 16), (5000, 16),
    (700, 24),     # GQA 6
])
def test_q8_fused_append_decode_matches_two_calls(dev, n_old, num_q):
    """qkv_decode_attn_q8_append (quantize the new token into row n_old and
    attend keys 0..n_old in one launch) against qkv_q8_append_kv followed by
    qkv_decode_attn_q8: identical cache bytes (pad fields untouched) and
    identical output bits; the output also against the oracle."""
    from qengine_amd import kvcache
    torch = _torch()
    n = n_old + 1
    rng, kb, vb = _cache(900 + n_old + num_q, n)
    kn = _torch().from_numpy(kv_f16(rng, 1, 4, 256).reshape(-1).view(np.uint16).copy())
    vn = _torch().from_numpy(kv_f16(rng, 1, 4, 256).reshape(-1).view(np.uint16).copy())
    q = q_f16(rng, 1, num_q, 256)
    k_new, v_new = kn.view(torch.float16).to(dev), vn.view(torch.float16).to(dev)
    # cache rows past n_old hold a marker pattern: the fused call must write row
    # n_old exactly as the append does and leave the pad half-words alone
    kc = _dev(kb.view(np.uint8), dev).reshape(n, -1)
    vc = _dev(vb.view(np.uint8), dev).reshape(n, -1)
    kc[n_old:] = 0x5A
    vc[n_old:] = 0xA5
    k1, v1, k2, v2 = kc.clone(), vc.clone(), kc.clone(), vc.clone()
    qd = _dev(q.view(np.uint16), dev)
    ws1 = kvcache.decode_attn_q8_workspace(num_q, 4, 1, n, dev)
    ws2 = kvcache.decode_attn_q8_workspace(num_q, 4, 1, n, dev)
    o1 = torch.zeros((1, num_q, 256), dtype=torch.float16, device=dev)
    o2 = torch.zeros((1, num_q, 256), dtype=torch.float16, device=dev)
    row = 4 * 8 * 36
    kvcache.q8_append_kv(k_new, v_new, k1.view(-1)[n_old * row:], v1.view(-1)[n_old * row:])
    kvcache.decode_attn_q8(qd, k1, v1, o1, ws1, num_q=num_q, num_kv=4, start_pos=n_old,
                           sub_n=1, scale=1 / 16)
    kvcache.decode_attn_q8_append(qd, k_new, v_new, k2, v2, o2, ws2, num_q=num_q, num_kv=4,
                                  start_pos=n_old, scale=1 / 16)
    torch.cuda.synchronize()
    assert torch.equal(k1, k2) and torch.equal(v1, v2)
    assert torch.equal(o1, o2)
    kb2 = k2.cpu().numpy().reshape(-1).view(kb.dtype)
    vb2 = v2.cpu().numpy().reshape(-1).view(vb.dtype)
    check_rel(o2.cpu().numpy(), _expected(q, kb2, vb2, n, num_q, 1), TOL)
