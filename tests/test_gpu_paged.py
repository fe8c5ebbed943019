"""GPU parity of the paged, ragged decode and the paged append (BASELINE
config 4: per-slot int32 block tables over one block pool, shared prefix
blocks, ragged context lengths).  The reference keeps slots contiguous
(model.cuh:1708-1715); the paged path is defined by gathering each slot's
rows and running the reference decode on them (oracle.decode_paged), and an
identity table must reproduce the contiguous fast path bit for bit.
Bar: 2e-3 relative error for attention, bit-exact blocks for the append."""
import numpy as np
import pytest

from oracle import oracle as O
from tests._data import assert_tq3_attn, kv_f16, q_f16, rel_err

pytestmark = pytest.mark.gpu
TOL = 2e-3
HD = 256


def _torch():
    import torch
    return torch


def _dev(a, dev):
    return _torch().from_numpy(np.ascontiguousarray(a)).to(dev)


def _pool(rng, rows, num_kv):
    k16 = kv_f16(rng, rows, num_kv, HD)
    v16 = kv_f16(rng, rows, num_kv, HD)
    return O.tq3_encode(k16), O.tq3_encode(v16)


def _tables(rng, ctx_lens, block_tokens, max_blocks, n_phys, shared_prefix_blocks=0,
            shared_slots=0):
    """Random distinct physical blocks per slot; the first shared_slots slots
    point their first shared_prefix_blocks entries at the same blocks."""
    n_slots = len(ctx_lens)
    perm = rng.permutation(n_phys)
    bt = np.zeros((n_slots, max_blocks), np.int32)
    nxt = 0
    shared = perm[:shared_prefix_blocks]
    nxt = shared_prefix_blocks
    for s, ctx in enumerate(ctx_lens):
        nb = (int(ctx) + block_tokens - 1) // block_tokens
        for b in range(max_blocks):
            if s < shared_slots and b < shared_prefix_blocks:
                bt[s, b] = shared[b]
            elif b < nb:
                bt[s, b] = perm[nxt]
                nxt += 1
            else:
                bt[s, b] = -1   # never read: beyond the slot's context
    assert nxt <= n_phys
    return bt


def _exact_paged(q, kp, vp, bt, ctx, *, num_q, num_kv, block_tokens):
    """Exact fp64 attention of each slot over its gathered rows (zero row for ctx 0)."""
    q = np.ascontiguousarray(q).view(np.uint16).reshape(len(ctx), num_q, HD)
    out = np.zeros((len(ctx), num_q, HD))
    bpr = num_kv * HD // 128
    for s, c in enumerate(ctx):
        c = int(c)
        if c <= 0:
            continue
        rows = O.paged_rows(bt[s], c, block_tokens)
        out[s] = O.attn_exact_tq3(q[s:s + 1], O.gather_rows(kp, rows, bpr),
                                  O.gather_rows(vp, rows, bpr), num_q=num_q, num_kv=num_kv, hd=HD,
                                  start_pos=c - 1, sub_n=1, scale=1 / 16)[0]
    return out


def _decode(dev, q, kp, vp, bt, ctx, *, num_q, num_kv, max_ctx, block_tokens, ws=None):
    from qengine_amd import kvcache
    torch = _torch()
    n_slots = q.shape[0]
    if ws is None:
        ws = kvcache.decode_attn_tq3_paged_workspace(num_q, num_kv, n_slots, max_ctx, dev)
    out = torch.zeros((n_slots, num_q, HD), dtype=torch.float16, device=dev)
    kvcache.decode_attn_tq3_paged(_dev(q.view(np.uint16), dev).view(torch.float16),
                                  _dev(kp.view(np.uint8), dev), _dev(vp.view(np.uint8), dev), out,
                                  ws, _dev(bt, dev), _dev(np.asarray(ctx, np.int32), dev),
                                  num_q=num_q, num_kv=num_kv, max_ctx=max_ctx,
                                  block_tokens=block_tokens, scale=1 / 16)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("n", [1, 300, 4097, 32768])
def test_identity_table_matches_contiguous(dev, n):
    """Identity block table over a slot's contiguous rows == qkv_decode_attn_tq3."""
    from qengine_amd import kvcache
    torch = _torch()
    rng = np.random.default_rng(900 + n)
    kp, vp = _pool(rng, n, 4)
    q = q_f16(rng, 1, 16, HD)
    bt_tok = 256
    max_blocks = (n + bt_tok - 1) // bt_tok
    bt = np.arange(max_blocks, dtype=np.int32)[None, :]
    got = _decode(dev, q, kp, vp, bt, [n], num_q=16, num_kv=4, max_ctx=n, block_tokens=bt_tok)
    ws = kvcache.decode_attn_tq3_workspace(16, 4, 1, n, dev)
    out = torch.zeros((1, 16, HD), dtype=torch.float16, device=dev)
    kvcache.decode_attn_tq3(_dev(q.view(np.uint16), dev), _dev(kp.view(np.uint8), dev),
                            _dev(vp.view(np.uint8), dev), out, ws, num_q=16, num_kv=4,
                            start_pos=n - 1, sub_n=1, scale=1 / 16)
    torch.cuda.synchronize()
    assert np.array_equal(got.view(np.uint16), out.cpu().numpy().view(np.uint16))


@pytest.mark.parametrize("block_tokens,num_q", [(256, 24), (64, 16), (512, 24)])
def test_ragged_shared_prefix_vs_oracle(dev, block_tokens, num_q):
    rng = np.random.default_rng(block_tokens + num_q)
    ctx = np.array([2048 + 17, 1, 4097, 2500, 256, 3000, 777, 64 * 5], np.int64)
    max_ctx = int(ctx.max())
    max_blocks = (max_ctx + block_tokens - 1) // block_tokens
    n_phys = int(sum((c + block_tokens - 1) // block_tokens for c in ctx)) + 4
    shared = 1024 // block_tokens if block_tokens <= 1024 else 1
    # slots 0..3 share their first `shared` blocks (prefix); slot 1 has one key
    # and uses only the first shared block
    bt = _tables(rng, ctx, block_tokens, max_blocks, n_phys, shared, 4)
    kp, vp = _pool(rng, n_phys * block_tokens, 4)
    q = q_f16(rng, len(ctx), num_q, HD)
    got = _decode(dev, q, kp, vp, bt, ctx, num_q=num_q, num_kv=4, max_ctx=max_ctx,
                  block_tokens=block_tokens)
    exp = O.decode_paged(O.KV_TQ3, q, kp, vp, bt, ctx, num_q=num_q, num_kv=4, hd=HD,
                         block_tokens=block_tokens, scale=1 / 16).view(np.float16)
    ex = _exact_paged(q, kp, vp, bt, ctx, num_q=num_q, num_kv=4, block_tokens=block_tokens)
    for s in range(len(ctx)):
        assert_tq3_attn(got[s], exp[s], ex[s], what=s)


def test_zero_and_clamped_context(dev):
    """ctx 0 gives a zero row; ctx beyond max_ctx is clamped to max_ctx."""
    rng = np.random.default_rng(5)
    bt_tok, max_ctx = 256, 1000
    max_blocks = 4
    kp, vp = _pool(rng, 4 * bt_tok, 4)
    bt = np.tile(np.arange(4, dtype=np.int32), (3, 1))
    q = q_f16(rng, 3, 16, HD)
    got = _decode(dev, q, kp, vp, bt, [0, 5000, max_ctx], num_q=16, num_kv=4, max_ctx=max_ctx,
                  block_tokens=bt_tok)
    assert np.all(got[0] == 0)
    exp = O.decode_paged(O.KV_TQ3, q, kp, vp, bt, [0, max_ctx, max_ctx], num_q=16, num_kv=4,
                         hd=HD, block_tokens=bt_tok, scale=1 / 16).view(np.float16)
    ex = _exact_paged(q, kp, vp, bt, [0, max_ctx, max_ctx], num_q=16, num_kv=4,
                      block_tokens=bt_tok)
    assert_tq3_attn(got[1], exp[1], ex[1])
    assert_tq3_attn(got[2], exp[2], ex[2])


@pytest.mark.parametrize("n_tok", [1, 3, 300])
def test_paged_append_bitexact(dev, n_tok):
    from qengine_amd import kvcache
    torch = _torch()
    rng = np.random.default_rng(40 + n_tok)
    n_slots, num_kv, bt_tok, max_blocks = 5, 4, 64, 16
    pool_rows = n_slots * max_blocks * bt_tok
    bt = rng.permutation(n_slots * max_blocks).astype(np.int32).reshape(n_slots, max_blocks)
    pos = rng.integers(0, max_blocks * bt_tok - n_tok, size=n_slots).astype(np.int32)
    pos[0] = max_blocks * bt_tok - n_tok            # ends exactly at the last row
    k16 = kv_f16(rng, n_slots * n_tok, num_kv, HD).reshape(n_slots, n_tok, num_kv, HD)
    v16 = kv_f16(rng, n_slots * n_tok, num_kv, HD).reshape(n_slots, n_tok, num_kv, HD)
    kpool = kvcache.tq3_blocks(pool_rows * 8, dev)
    vpool = kvcache.tq3_blocks(pool_rows * 8, dev)
    kvcache.tq3_append_kv_paged(_dev(k16.view(np.uint16), dev).view(torch.float16),
                                _dev(v16.view(np.uint16), dev).view(torch.float16), kpool, vpool,
                                _dev(bt, dev), _dev(pos, dev), block_tokens=bt_tok)
    torch.cuda.synchronize()
    for pool, x in ((kpool, k16), (vpool, v16)):
        got = pool.cpu().numpy().reshape(pool_rows, 8 * 52)
        written = np.zeros(pool_rows, bool)
        for s in range(n_slots):
            rows = O.paged_rows(bt[s], pos[s] + n_tok, bt_tok)[pos[s]:]
            exp = O.tq3_encode(x[s]).view(np.uint8).reshape(n_tok, 8 * 52)
            assert np.array_equal(got[rows], exp), s
            written[rows] = True
        assert np.all(got[~written] == 0), "rows outside the appended tokens were written"


def test_paged_append_skips_rows_outside_pool(dev):
    from qengine_amd import kvcache
    torch = _torch()
    rng = np.random.default_rng(3)
    bt_tok, pool_rows = 64, 128
    bt = np.array([[0, 5, 1]], np.int32)          # block 5 lies beyond the 2-block pool
    pos = np.array([60], np.int32)                 # tokens at 60..67: rows 60..63, 320..323
    k16 = kv_f16(rng, 8, 4, HD).reshape(1, 8, 4, HD)
    kpool = kvcache.tq3_blocks(pool_rows * 8, dev)
    vpool = kvcache.tq3_blocks(pool_rows * 8, dev)
    kt = _dev(k16.view(np.uint16), dev).view(torch.float16)
    kvcache.tq3_append_kv_paged(kt, kt, kpool, vpool, _dev(bt, dev), _dev(pos, dev),
                                block_tokens=bt_tok)
    torch.cuda.synchronize()
    got = kpool.cpu().numpy().reshape(pool_rows, 416)
    exp = O.tq3_encode(k16[0]).view(np.uint8).reshape(8, 416)
    assert np.array_equal(got[60:64], exp[:4])
    assert np.all(got[64:] == 0) and np.all(got[:60] == 0)


def test_config4_step_append_then_decode(dev):
    """One continuous-batching step at reduced size: 8 slots, GQA 6, 256-token
    blocks, slots 0-3 sharing a prefix; append 1 token per slot, then decode."""
    from qengine_amd import kvcache
    torch = _torch()
    rng = np.random.default_rng(44)
    n_slots, num_q, num_kv, bt_tok = 8, 24, 4, 256
    ctx_old = rng.integers(1024, 6000, size=n_slots)
    ctx_old[:4] = np.maximum(ctx_old[:4], 1024 + 1)
    ctx_new = ctx_old + 1
    max_ctx = int(ctx_new.max())
    max_blocks = (max_ctx + bt_tok - 1) // bt_tok
    n_phys = int(sum((c + bt_tok - 1) // bt_tok for c in ctx_new)) + 2
    bt = _tables(rng, ctx_new, bt_tok, max_blocks, n_phys, 1024 // bt_tok, 4)
    kp, vp = _pool(rng, n_phys * bt_tok, num_kv)
    kpt, vpt = _dev(kp.view(np.uint8), dev), _dev(vp.view(np.uint8), dev)
    knew = kv_f16(rng, n_slots, num_kv, HD).reshape(n_slots, 1, num_kv, HD)
    vnew = kv_f16(rng, n_slots, num_kv, HD).reshape(n_slots, 1, num_kv, HD)
    kvcache.tq3_append_kv_paged(_dev(knew.view(np.uint16), dev).view(torch.float16),
                                _dev(vnew.view(np.uint16), dev).view(torch.float16), kpt, vpt,
                                _dev(bt, dev), _dev(ctx_old.astype(np.int32), dev),
                                block_tokens=bt_tok)
    q = q_f16(rng, n_slots, num_q, HD)
    ws = kvcache.decode_attn_tq3_paged_workspace(num_q, num_kv, n_slots, max_ctx, dev)
    out = torch.zeros((n_slots, num_q, HD), dtype=torch.float16, device=dev)
    kvcache.decode_attn_tq3_paged(_dev(q.view(np.uint16), dev).view(torch.float16), kpt, vpt,
                                  out, ws, _dev(bt, dev), _dev(ctx_new.astype(np.int32), dev),
                                  num_q=num_q, num_kv=num_kv, max_ctx=max_ctx,
                                  block_tokens=bt_tok, scale=1 / 16)
    torch.cuda.synchronize()
    # host model of the step: encode the new tokens into their rows, then decode
    kp2, vp2 = kp.copy(), vp.copy()
    for s in range(n_slots):
        r = int(O.paged_rows(bt[s], ctx_new[s], bt_tok)[-1])
        kp2[r * 8:(r + 1) * 8] = O.tq3_encode(knew[s])
        vp2[r * 8:(r + 1) * 8] = O.tq3_encode(vnew[s])
    assert np.array_equal(kpt.cpu().numpy().reshape(-1), kp2.view(np.uint8).reshape(-1))
    exp = O.decode_paged(O.KV_TQ3, q, kp2, vp2, bt, ctx_new, num_q=num_q, num_kv=num_kv, hd=HD,
                         block_tokens=bt_tok, scale=1 / 16).view(np.float16)
    got = out.cpu().numpy()
    ex = _exact_paged(q, kp2, vp2, bt, ctx_new, num_q=num_q, num_kv=num_kv, block_tokens=bt_tok)
    for s in range(n_slots):
        assert_tq3_attn(got[s], exp[s], ex[s], what=s)


def test_pool_beyond_4gib(dev):
    """A paged pool larger than 4 GiB per tensor (10.5M token rows of 416 B):
    the append writes, and the decode reads, blocks at the top of the pool
    (64-bit row offsets).  Results are bit-identical to the same slots in a
    small pool, which in turn is checked against the oracle."""
    from qengine_amd import kvcache
    torch = _torch()
    rng = np.random.default_rng(4242)
    num_q, num_kv, bt_tok = 16, 4, 256
    ctx = [2900, 1700]
    max_blocks = 12
    n_tok = max(ctx)
    k16 = kv_f16(rng, 2 * n_tok, num_kv, HD).reshape(2, n_tok, num_kv, HD)
    v16 = kv_f16(rng, 2 * n_tok, num_kv, HD).reshape(2, n_tok, num_kv, HD)
    q = q_f16(rng, 2, num_q, HD)
    big_rows = 10_500_000 // bt_tok * bt_tok          # 4.37e9 bytes per tensor
    assert big_rows * num_kv * 104 > 2 ** 32
    top = big_rows // bt_tok - 2 * max_blocks         # first block index used at the top
    bt_small = np.arange(2 * max_blocks, dtype=np.int32).reshape(2, max_blocks)
    bt_big = bt_small + np.int32(top)
    out = {}
    blocks = {}
    for name, rows, bt in (("small", 2 * max_blocks * bt_tok, bt_small), ("big", big_rows, bt_big)):
        kp = torch.zeros((rows * 8, 52), dtype=torch.uint8, device=dev)
        vp = torch.zeros((rows * 8, 52), dtype=torch.uint8, device=dev)
        btd = _dev(bt, dev)
        kvcache.tq3_append_kv_paged(_dev(k16, dev), _dev(v16, dev), kp, vp, btd,
                                    _dev(np.zeros(2, np.int32), dev), block_tokens=bt_tok)
        ws = kvcache.decode_attn_tq3_paged_workspace(num_q, num_kv, 2, max(ctx), dev)
        o = torch.zeros((2, num_q, HD), dtype=torch.float16, device=dev)
        kvcache.decode_attn_tq3_paged(_dev(q, dev), kp, vp, o, ws, btd,
                                      _dev(np.asarray(ctx, np.int32), dev), num_q=num_q,
                                      num_kv=num_kv, max_ctx=max(ctx), block_tokens=bt_tok,
                                      scale=1 / 16)
        torch.cuda.synchronize()
        out[name] = o.cpu().numpy()
        r0 = int(bt[0, 0]) * bt_tok
        blocks[name] = (kp[r0 * 8:(r0 + 2 * max_blocks * bt_tok) * 8].cpu().numpy(),
                        vp[r0 * 8:(r0 + 2 * max_blocks * bt_tok) * 8].cpu().numpy())
        del kp, vp
        torch.cuda.empty_cache()
    assert np.array_equal(blocks["big"][0], blocks["small"][0])
    assert np.array_equal(blocks["big"][1], blocks["small"][1])
    assert np.array_equal(out["big"].view(np.uint16), out["small"].view(np.uint16))
    kb, vb = blocks["small"]
    ref = O.decode_paged(O.KV_TQ3, q, np.ascontiguousarray(kb).view(O.BLOCK_TQ3).reshape(-1),
                         np.ascontiguousarray(vb).view(O.BLOCK_TQ3).reshape(-1), bt_small,
                         np.asarray(ctx, np.int32), num_q=num_q, num_kv=num_kv, hd=HD,
                         block_tokens=bt_tok, scale=1 / 16)
    ex = _exact_paged(q, np.ascontiguousarray(kb).view(O.BLOCK_TQ3).reshape(-1),
                      np.ascontiguousarray(vb).view(O.BLOCK_TQ3).reshape(-1), bt_small, ctx,
                      num_q=num_q, num_kv=num_kv, block_tokens=bt_tok)
    assert_tq3_attn(out["small"].astype(np.float64), ref.view(np.float16).astype(np.float64), ex)
