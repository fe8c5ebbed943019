"""KV inject from DFK2 planes and paged slot snapshot / restore (the packed
formats beside the cache, model.cuh:149-159, 3077-3240, 3314-3459).

- qkv_dfk2_dequant: bit-exact against the oracle's dfki2_dequant_kernel;
- qkv_tq3_append_dfk2 / qkv_q8_append_dfk2: bit-exact against the reference
  pair they fuse (dequantize to fp16, then tq3_quantize_kernel /
  quantize_kv_q8_0_kern), i.e. oracle.tq3_encode / q8_encode of
  oracle.dfk2_dequant; the Q8 pad bytes keep what the cache held;
- qkv_kv_gather_rows / qkv_kv_scatter_rows: byte-exact against numpy
  indexing through the block table (oracle.paged_rows), for TQ3, Q8_0 and
  fp16 row sizes and a row size that is not a multiple of 16 bytes; unmapped
  table entries gather zeros and are skipped by the scatter; gather after
  scatter returns the flat rows."""
import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu
KV_DIM = 1024


def _dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _plane(rng, rows, special=False):
    q = rng.integers(-128, 128, size=(rows, KV_DIM), dtype=np.int8)
    s = (np.abs(rng.standard_normal((rows, KV_DIM // 128))) * 0.03 + 1e-3).astype(np.float16)
    if special and rows >= 4:
        q[0] = 0                                   # zero rows: norm 0, codes 0
        s[1] = np.float16(6e-8)                    # subnormal scales
        q[2, :128] = 127
        s[2, 0] = np.float16(500.0)                # values beyond the fp16 range
        q[3] = -128
    return q, s


@pytest.mark.parametrize("rows", [1, 3, 100, 2048])
def test_dfk2_dequant_bitexact(dev, rows):
    import torch
    from qengine_amd import kvcache
    q, s = _plane(np.random.default_rng(rows), rows, special=True)
    out = torch.zeros((rows, KV_DIM), dtype=torch.float16, device=dev)
    kvcache.dfk2_dequant(_dev(q, dev), _dev(s, dev), out, kv_dim=KV_DIM)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint16), O.dfk2_dequant(q, s, KV_DIM))


@pytest.mark.parametrize("rows", [1, 3, 100, 2048, 16384])
def test_tq3_append_dfk2_bitexact(dev, rows):
    import torch
    from qengine_amd import kvcache
    q, s = _plane(np.random.default_rng(100 + rows), rows, special=True)
    print(f"tq3 dfk2 rows={rows}", flush=True)
    out = kvcache.tq3_blocks(rows * KV_DIM // 128, dev)
    kvcache.tq3_append_dfk2(_dev(q, dev), _dev(s, dev), out)
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(O.BLOCK_TQ3).reshape(-1)
    exp = O.tq3_encode(O.dfk2_dequant(q, s, KV_DIM).view(np.float16).reshape(-1, 128))
    bad = np.nonzero((got.view(np.uint8).reshape(len(got), -1) !=
                      exp.view(np.uint8).reshape(len(exp), -1)).any(1))[0]
    assert bad.size == 0, f"{bad.size} blocks differ, first {bad[:5]}"


@pytest.mark.parametrize("rows", [1, 3, 100, 2048])
def test_q8_append_dfk2_bitexact(dev, rows):
    import torch
    from qengine_amd import kvcache
    q, s = _plane(np.random.default_rng(200 + rows), rows, special=True)
    n_blocks = rows * KV_DIM // 32
    out = kvcache.q8_blocks(n_blocks, dev)
    out.fill_(0xAB)                                # pad bytes must keep this
    kvcache.q8_append_dfk2(_dev(q, dev), _dev(s, dev), out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    exp = O.q8_encode(O.dfk2_dequant(q, s, KV_DIM).view(np.float16).reshape(-1, 32))
    eb = exp.view(np.uint8).reshape(n_blocks, 36)
    assert np.array_equal(got[:, :32], eb[:, :32])
    assert np.array_equal(got[:, 34:], eb[:, 34:])
    assert np.all(got[:, 32:34] == 0xAB)


def _table(rng, n_rows, block_tokens, pool_blocks, holes=()):
    nb = (n_rows + block_tokens - 1) // block_tokens
    t = rng.permutation(pool_blocks)[:nb].astype(np.int32)
    for h in holes:
        t[h] = -1
    return t


@pytest.mark.parametrize("row_bytes,block_tokens,n_rows", [
    (416, 256, 1000),      # TQ3 row (8 blocks of 52 B)
    (1152, 16, 333),       # Q8_0 row (32 blocks of 36 B)
    (2048, 64, 200),       # fp16 row
    (52, 7, 50),           # a row of one TQ3 block: whole dwords, not 16-byte units
])
def test_gather_scatter_vs_numpy(dev, row_bytes, block_tokens, n_rows):
    import torch
    from qengine_amd import kvcache
    rng = np.random.default_rng(row_bytes + n_rows)
    pool_blocks = (n_rows + block_tokens - 1) // block_tokens * 2 + 3
    pool_rows = pool_blocks * block_tokens
    kp = rng.integers(0, 256, size=(pool_rows, row_bytes), dtype=np.uint8)
    vp = rng.integers(0, 256, size=(pool_rows, row_bytes), dtype=np.uint8)
    holes = (1,) if n_rows > block_tokens else ()
    table = _table(rng, n_rows, block_tokens, pool_blocks, holes)
    rows = O.paged_rows(np.maximum(table, 0), n_rows, block_tokens)
    mapped = np.repeat(table >= 0, block_tokens)[:n_rows]
    kpd, vpd, td = _dev(kp, dev), _dev(vp, dev), _dev(table, dev)
    kf = torch.full((n_rows, row_bytes), 7, dtype=torch.uint8, device=dev)
    vf = torch.full_like(kf, 7)
    kvcache.kv_gather_rows(kpd, vpd, kf, vf, td, n_rows=n_rows, block_tokens=block_tokens,
                           k_row_bytes=row_bytes, v_row_bytes=row_bytes)
    torch.cuda.synchronize()
    for got, pool in ((kf.cpu().numpy(), kp), (vf.cpu().numpy(), vp)):
        assert np.array_equal(got[mapped], pool[rows[mapped]])
        assert np.all(got[~mapped] == 0)
    # restore a different snapshot into the pool (K only, then K and V)
    nk = rng.integers(0, 256, size=(n_rows, row_bytes), dtype=np.uint8)
    nv = rng.integers(0, 256, size=(n_rows, row_bytes), dtype=np.uint8)
    kvcache.kv_scatter_rows(kpd, None, _dev(nk, dev), None, td, n_rows=n_rows,
                            block_tokens=block_tokens, k_row_bytes=row_bytes)
    kvcache.kv_scatter_rows(kpd, vpd, _dev(nk, dev), _dev(nv, dev), td, n_rows=n_rows,
                            block_tokens=block_tokens, k_row_bytes=row_bytes,
                            v_row_bytes=row_bytes)
    torch.cuda.synchronize()
    ek, ev = kp.copy(), vp.copy()
    ek[rows[mapped]] = nk[mapped]
    ev[rows[mapped]] = nv[mapped]
    assert np.array_equal(kpd.cpu().numpy(), ek)
    assert np.array_equal(vpd.cpu().numpy(), ev)
    kvcache.kv_gather_rows(kpd, vpd, kf, vf, td, n_rows=n_rows, block_tokens=block_tokens,
                           k_row_bytes=row_bytes, v_row_bytes=row_bytes)
    torch.cuda.synchronize()
    assert np.array_equal(kf.cpu().numpy()[mapped], nk[mapped])
    assert np.array_equal(vf.cpu().numpy()[mapped], nv[mapped])


def test_snapshot_restore_roundtrip_decodes_identically(dev):
    """A TQ3 slot saved from one paged pool and restored into another pool with
    a different block table decodes to the same bits."""
    import torch
    from qengine_amd import kvcache
    from tests._data import kv_f16, q_f16
    rng = np.random.default_rng(8)
    n, bt, nq = 3000, 256, 16
    nb = (n + bt - 1) // bt
    t1 = rng.permutation(nb + 4)[:nb].astype(np.int32)
    t2 = rng.permutation(nb + 9)[:nb].astype(np.int32)
    k16, v16 = kv_f16(rng, n, 4, 256), kv_f16(rng, n, 4, 256)
    rows1 = O.paged_rows(t1, n, bt)
    kp1 = np.zeros(((nb + 4) * bt * 8,), O.BLOCK_TQ3)
    vp1 = np.zeros_like(kp1)
    kp1.reshape(-1, 8)[rows1] = O.tq3_encode(k16).reshape(-1, 8)
    vp1.reshape(-1, 8)[rows1] = O.tq3_encode(v16).reshape(-1, 8)
    kpd1, vpd1 = _dev(kp1.view(np.uint8), dev), _dev(vp1.view(np.uint8), dev)
    kf = torch.zeros((n, 416), dtype=torch.uint8, device=dev)
    vf = torch.zeros_like(kf)
    kvcache.kv_gather_rows(kpd1, vpd1, kf, vf, _dev(t1, dev), n_rows=n, block_tokens=bt,
                           k_row_bytes=416, v_row_bytes=416)
    kpd2 = torch.zeros(((nb + 9) * bt * 8 * 52,), dtype=torch.uint8, device=dev)
    vpd2 = torch.zeros_like(kpd2)
    kvcache.kv_scatter_rows(kpd2, vpd2, kf, vf, _dev(t2, dev), n_rows=n, block_tokens=bt,
                            k_row_bytes=416, v_row_bytes=416)
    q = _dev(q_f16(rng, 1, nq, 256).view(np.uint16), dev)
    outs = []
    for kp, vp, t in ((kpd1, vpd1, t1), (kpd2, vpd2, t2)):
        out = torch.zeros((1, nq, 256), dtype=torch.float16, device=dev)
        ws = kvcache.decode_attn_tq3_paged_workspace(nq, 4, 1, n, dev)
        kvcache.decode_attn_tq3_paged(q, kp, vp, out, ws, _dev(t.reshape(1, -1), dev),
                                      _dev(np.array([n], np.int32), dev), num_q=nq, num_kv=4,
                                      max_ctx=n, block_tokens=bt, scale=1 / 16)
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    assert np.array_equal(outs[0].view(np.uint16), outs[1].view(np.uint16))
