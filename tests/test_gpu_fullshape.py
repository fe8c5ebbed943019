"""GPU parity at the full shapes bench.py measures (BASELINE configs 4 and
5(ii)), against the CPU oracle on the same bytes.

Config 4: 8 slots, 24 q / 4 kv heads, 256-token blocks, contexts drawn as in
bench.py (seeded U[1K, 64K], slots 0-3 sharing a 4096-token prefix through
common block indices); one step = paged append of one token per slot + paged
decode of all 8 slots.  The pool (≈ 400K token rows) is built on the GPU by
the bit-exact append; sampled slots (both ends of the context range and the
prefix-sharing ones) are checked against the reference split decode over the
slot's gathered rows (oracle.decode_paged).

Config 5(ii): one slot, 16 q / 4 kv heads, 131072-token TQ3 history plus a
16-token verify block appended first (model.cuh:4566-4571), attended with
causal masking within the block through qkv_decode_attn_tq3 (sub_n = 16), all
16 x 16 output rows against the reference split decode + merge.

Bar (tests/_data.assert_tq3_attn): every (query, head) output row within 2e-3
of the exact fp64 attention over the exactly dequantized cache, and the output
within 2e-3 (global) of the reference-order oracle."""
import numpy as np
import pytest

from oracle import oracle as O
from tests._data import assert_tq3_attn

pytestmark = pytest.mark.gpu
TOL = 2e-3
HD, NUM_KV = 256, 4


def _rnd(torch, gen, dev, *shape):
    return torch.randn(*shape, generator=gen, device=dev).to(torch.float16)


def test_config4_full_shape_vs_oracle(dev):
    import torch
    from qengine_amd import kvcache
    gen = torch.Generator(device=dev).manual_seed(404)
    # contexts and block tables exactly as bench.py's config 4
    rng = np.random.default_rng(4)
    n_slots, nq, bt_tok = 8, 24, 256
    ctx_s = rng.integers(1024, 65537, size=n_slots)
    ctx_s[:4] = np.maximum(ctx_s[:4], 4096 + 1)
    new_s = ctx_s + 1
    max_ctx = int(new_s.max())
    max_blocks = (max_ctx + bt_tok - 1) // bt_tok
    shared = 4096 // bt_tok
    tables = np.zeros((n_slots, max_blocks), np.int32)
    nxt = shared
    for s in range(n_slots):
        nb = (int(new_s[s]) + bt_tok - 1) // bt_tok
        for b in range(nb):
            if s < 4 and b < shared:
                tables[s, b] = b
            else:
                tables[s, b] = nxt
                nxt += 1
    pool_rows = nxt * bt_tok
    kp = kvcache.tq3_blocks(pool_rows * 8, dev)
    vp = kvcache.tq3_blocks(pool_rows * 8, dev)
    for r0 in range(0, pool_rows, 65536):
        n = min(65536, pool_rows - r0)
        kvcache.tq3_append_kv(_rnd(torch, gen, dev, n, NUM_KV, HD), _rnd(torch, gen, dev, n, NUM_KV, HD),
                              kp[r0 * 8:(r0 + n) * 8], vp[r0 * 8:(r0 + n) * 8])
    bt_d = torch.from_numpy(tables).to(dev)
    k1, v1 = _rnd(torch, gen, dev, n_slots, 1, NUM_KV, HD), _rnd(torch, gen, dev, n_slots, 1, NUM_KV, HD)
    q = _rnd(torch, gen, dev, n_slots, nq, HD)
    out = torch.zeros(n_slots, nq, HD, dtype=torch.float16, device=dev)
    ws = kvcache.decode_attn_tq3_paged_workspace(nq, NUM_KV, n_slots, max_ctx, dev)
    kvcache.tq3_append_kv_paged(k1, v1, kp, vp, bt_d, torch.from_numpy(ctx_s.astype(np.int32)).to(dev),
                                block_tokens=bt_tok)
    kvcache.decode_attn_tq3_paged(q, kp, vp, out, ws, bt_d,
                                  torch.from_numpy(new_s.astype(np.int32)).to(dev), num_q=nq,
                                  num_kv=NUM_KV, max_ctx=max_ctx, block_tokens=bt_tok, scale=1 / 16)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    kph = kp.cpu().numpy().view(O.BLOCK_TQ3).reshape(-1)
    vph = vp.cpu().numpy().view(O.BLOCK_TQ3).reshape(-1)
    qh = q.cpu().numpy()
    order = np.argsort(new_s)
    sample = sorted({int(order[0]), int(order[-1]), 0, 3})   # shortest, longest, two prefix sharers
    for s in sample:
        exp = O.decode_paged(O.KV_TQ3, qh[s:s + 1], kph, vph, tables[s:s + 1], new_s[s:s + 1],
                             num_q=nq, num_kv=NUM_KV, hd=HD, block_tokens=bt_tok,
                             scale=1 / 16).view(np.float16)
        rows = O.paged_rows(tables[s], int(new_s[s]), bt_tok)
        ex = O.attn_exact_tq3(qh[s:s + 1], O.gather_rows(kph, rows, 8), O.gather_rows(vph, rows, 8),
                              num_q=nq, num_kv=NUM_KV, hd=HD, start_pos=int(new_s[s]) - 1, sub_n=1,
                              scale=1 / 16)
        assert_tq3_attn(got[s:s + 1], exp, ex, what=(s, int(new_s[s])))


def test_config5_verify16_full_shape_vs_oracle(dev):
    import torch
    from qengine_amd import kvcache
    gen = torch.Generator(device=dev).manual_seed(505)
    hist, nv, nq = 131072, 16, 16
    kb = kvcache.tq3_blocks((hist + nv) * 8, dev)
    vb = kvcache.tq3_blocks((hist + nv) * 8, dev)
    for r0 in range(0, hist, 65536):
        kvcache.tq3_append_kv(_rnd(torch, gen, dev, 65536, NUM_KV, HD),
                              _rnd(torch, gen, dev, 65536, NUM_KV, HD),
                              kb[r0 * 8:(r0 + 65536) * 8], vb[r0 * 8:(r0 + 65536) * 8])
    kvcache.tq3_append_kv(_rnd(torch, gen, dev, nv, NUM_KV, HD), _rnd(torch, gen, dev, nv, NUM_KV, HD),
                          kb[hist * 8:], vb[hist * 8:])
    q = _rnd(torch, gen, dev, nv, nq, HD)
    out = torch.zeros(nv, nq, HD, dtype=torch.float16, device=dev)
    ws = kvcache.decode_attn_tq3_workspace(nq, NUM_KV, nv, hist + nv, dev)
    kvcache.decode_attn_tq3(q, kb, vb, out, ws, num_q=nq, num_kv=NUM_KV, start_pos=hist, sub_n=nv,
                            scale=1 / 16)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    kbh = kb.cpu().numpy().view(O.BLOCK_TQ3).reshape(-1)
    vbh = vb.cpu().numpy().view(O.BLOCK_TQ3).reshape(-1)
    ks = 8
    pm, pl, po = O.attn_split(O.KV_TQ3, q.cpu().numpy(), kbh, vbh, num_q=nq, num_kv=NUM_KV, hd=HD,
                              start_pos=hist, sub_n=nv, sub_n_max=nv, active_end_max=hist + nv,
                              scale=1 / 16, k_splits=ks)
    exp = O.attn_split_merge(pm, pl, po, num_q=nq, num_kv=NUM_KV, hd=HD, sub_n=nv, sub_n_max=nv,
                             k_splits=ks).view(np.float16)
    ex = O.attn_exact_tq3(q.cpu().numpy(), kbh, vbh, num_q=nq, num_kv=NUM_KV, hd=HD,
                          start_pos=hist, sub_n=nv, scale=1 / 16)
    assert_tq3_attn(got, exp, ex)
