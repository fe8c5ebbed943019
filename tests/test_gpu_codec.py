"""GPU parity of the append (encode) and dequant kernels against the CPU
oracle: bit-exact packed codes, norms, fp16 outputs and Q8 blocks.
References: turboquant.cuh:112-200, attention.cuh:2587-2626."""
import numpy as np
import pytest

from oracle import oracle as O
from tests._data import kv_f16

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


def _to_dev(a, dev):
    torch = _torch()
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _special_blocks(rng):
    extra = [
        np.zeros(128, np.float16), np.full(128, -0.0, np.float16),
        np.eye(128, dtype=np.float16)[7] * np.float16(3.0),
        (np.eye(128)[0] + np.eye(128)[1]).astype(np.float16),
        np.full(128, np.float16(6e-8)), np.full(128, np.float16(65504.0)),
        np.full(128, np.float16(-65504.0)),
        (rng.uniform(-1, 1, 128) * 1e-3).astype(np.float16),
    ]
    return np.stack(extra)


def _tq3_gpu(x16, dev):
    from qengine_amd import kvcache
    torch = _torch()
    n = x16.size // 128
    out = kvcache.tq3_blocks(n, dev)
    kvcache.tq3_append(_to_dev(x16.reshape(-1), dev), out)
    torch.cuda.synchronize()
    return out.cpu().numpy().view(O.BLOCK_TQ3).reshape(-1)


def _diff_report(got, exp):
    gb = got.view(np.uint8).reshape(len(got), -1)
    eb = exp.view(np.uint8).reshape(len(exp), -1)
    bad = np.nonzero((gb != eb).any(1))[0]
    return bad


# Appends of at most 16384 blocks (all tensors together) take the small-append
# kernel (a block per 16-lane row), larger ones the lane-pair kernel: sizes on
# both sides of that limit.
@pytest.mark.parametrize("n_blocks", [1, 7, 63, 64, 65, 257, 1000, 16383, 16384, 16385, 20000])
def test_tq3_append_bitexact_odd_sizes(dev, n_blocks):
    rng = np.random.default_rng(n_blocks)
    x = kv_f16(rng, n_blocks, 1, 128)
    got = _tq3_gpu(x, dev)
    exp = O.tq3_encode(x)
    bad = _diff_report(got, exp)
    assert bad.size == 0, f"{bad.size} blocks differ, first {bad[:5]}"


@pytest.mark.parametrize("n_tok,reps", [(1024, 1), (100, 1), (1024, 2)])
def test_tq3_append_config1_and_specials(dev, n_tok, reps):
    # config 1: 1024 tokens x 4 heads x 256 (K), 2% x8 outlier channels, seed 0
    # (8200 blocks) and its first 100 tokens: small kernel; the 8200 blocks
    # twice over (16400): lane-pair kernel
    rng = np.random.default_rng(0)
    x = np.concatenate([kv_f16(rng, 1024, 4, 256).reshape(-1, 128)[: n_tok * 8], _special_blocks(rng)])
    x = np.tile(x, (reps, 1))
    got = _tq3_gpu(x, dev)
    exp = O.tq3_encode(x)
    assert np.array_equal(got["norm"].view(np.uint32), exp["norm"].view(np.uint32))
    bad = _diff_report(got, exp)
    assert bad.size == 0, f"{bad.size} of {len(exp)} blocks differ, first {bad[:5]}"


@pytest.mark.parametrize("reps", [1, 1026])
def test_tq3_append_nonfinite_and_extreme_blocks(dev, reps):
    """Blocks with inf / NaN elements: the reference bins the NaN WHT outputs
    to 0, so the codes are zero and the norm is inf or NaN.  Blocks mixing
    the largest and the smallest fp16 magnitudes reach the smallest nonzero
    WHT outputs."""
    rng = np.random.default_rng(5)
    x = kv_f16(rng, 16, 1, 128).reshape(16, 128)
    x[0, 3] = np.inf
    x[1, 100] = -np.inf
    x[2, 0] = np.nan
    x[3, :] = np.nan
    x[4, 5] = np.inf
    x[4, 6] = -np.inf
    x[8, :] = np.float16(6e-8)
    x[8, 17] = np.float16(65504.0)
    x[9, :] = -np.float16(6e-8)
    x[9, 90] = np.float16(-65504.0)
    x[10, ::2] = np.float16(6e-8)
    x[10, 1::2] = np.float16(-6e-8)
    x[10, 64] = np.float16(65504.0)
    x = np.tile(x, (reps, 1))   # 16 blocks: small kernel; 16416: lane-pair kernel
    got = _tq3_gpu(x, dev)
    exp = O.tq3_encode(x)
    gn, en = got["norm"], exp["norm"]
    assert np.array_equal(np.isnan(gn), np.isnan(en))
    ok = ~np.isnan(en)
    assert np.array_equal(gn[ok].view(np.uint32), en[ok].view(np.uint32))
    assert np.array_equal(got["qs"], exp["qs"])
    assert not exp["qs"][:5].any()


def test_tq3_append_large_bitexact(dev):
    """Config-3 layer build size: 32768 tokens x 8 blocks (262144 blocks)."""
    torch = _torch()
    g = torch.Generator(device=dev).manual_seed(3)
    x = torch.randn(32768 * 8 * 128, generator=g, device=dev).to(torch.float16)
    from qengine_amd import kvcache
    out = kvcache.tq3_blocks(32768 * 8, dev)
    kvcache.tq3_append(x, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(O.BLOCK_TQ3).reshape(-1)
    exp = O.tq3_encode(x.cpu().numpy().view(np.uint16))
    bad = _diff_report(got, exp)
    assert bad.size == 0, f"{bad.size} blocks differ"


def test_tq3_append_kv_matches_two_appends(dev):
    from qengine_amd import kvcache
    torch = _torch()
    rng = np.random.default_rng(21)
    k = _to_dev(kv_f16(rng, 77, 4, 256).reshape(-1), dev)
    v = _to_dev(kv_f16(rng, 77, 4, 256).reshape(-1), dev)
    n = k.numel() // 128
    ko, vo = kvcache.tq3_blocks(n, dev), kvcache.tq3_blocks(n, dev)
    kvcache.tq3_append_kv(k, v, ko, vo)
    k1, v1 = kvcache.tq3_blocks(n, dev), kvcache.tq3_blocks(n, dev)
    kvcache.tq3_append(k, k1)
    kvcache.tq3_append(v, v1)
    torch.cuda.synchronize()
    assert torch.equal(ko, k1) and torch.equal(vo, v1)


@pytest.mark.parametrize("n_tok", [1024, 1025, 1])
def test_tq3_append_kv_bitexact(dev, n_tok):
    """K and V in one launch against the oracle: 1024 tokens (2 x 8192
    blocks, the small kernel's limit), 1025 (the lane-pair kernel) and one
    token (a decode step)."""
    from qengine_amd import kvcache
    torch = _torch()
    rng = np.random.default_rng(22 + n_tok)
    k16, v16 = kv_f16(rng, n_tok, 4, 256), kv_f16(rng, n_tok, 4, 256)
    n = n_tok * 8
    ko, vo = kvcache.tq3_blocks(n, dev), kvcache.tq3_blocks(n, dev)
    kvcache.tq3_append_kv(_to_dev(k16.reshape(-1), dev), _to_dev(v16.reshape(-1), dev), ko, vo)
    torch.cuda.synchronize()
    for got, x in ((ko, k16), (vo, v16)):
        bad = _diff_report(got.cpu().numpy().view(O.BLOCK_TQ3).reshape(-1), O.tq3_encode(x))
        assert bad.size == 0, f"{bad.size} blocks differ, first {bad[:5]}"


def test_tq3_append_writes_only_its_blocks(dev):
    """Appending at a cache offset leaves neighbouring blocks untouched."""
    from qengine_amd import kvcache
    torch = _torch()
    rng = np.random.default_rng(22)
    cache = torch.full((100, 52), 0xAB, dtype=torch.uint8, device=dev)
    x = _to_dev(kv_f16(rng, 1, 4, 256).reshape(-1), dev)     # one token: 8 blocks
    kvcache.tq3_append(x, cache[40:48])
    torch.cuda.synchronize()
    c = cache.cpu().numpy()
    assert np.all(c[:40] == 0xAB) and np.all(c[48:] == 0xAB)
    exp = O.tq3_encode(x.cpu().numpy().view(np.uint16))
    assert np.array_equal(c[40:48].reshape(-1), exp.view(np.uint8))


def test_tq3_dequant_bitexact(dev):
    from qengine_amd import kvcache
    torch = _torch()
    rng = np.random.default_rng(23)
    x = np.concatenate([kv_f16(rng, 300, 4, 256).reshape(-1, 128), _special_blocks(rng)])
    blocks = O.tq3_encode(x)
    got = kvcache.tq3_dequant(_to_dev(blocks.view(np.uint8).reshape(-1, 52), dev))
    torch.cuda.synchronize()
    exp = O.tq3_decode(blocks)
    g = got.cpu().numpy().view(np.uint16)
    bad = np.nonzero(g != exp)[0]
    detail = [(int(i // 128), int(i % 128), hex(g[i]), hex(exp[i])) for i in bad[:8]]
    assert bad.size == 0, f"{bad.size} elements differ (block, elem, got, exp): {detail}"


@pytest.mark.parametrize("n_blocks", [1, 5, 64, 4097 * 32])
def test_q8_append_bitexact_pad_untouched(dev, n_blocks):
    from qengine_amd import kvcache
    torch = _torch()
    rng = np.random.default_rng(n_blocks)
    x = rng.standard_normal(n_blocks * 32).astype(np.float16)
    x[:32] = 0                                                   # amax == 0 block
    if n_blocks > 1:
        x[32:64] = np.array([127.0, 2.5, 3.5, -2.5, -3.5, 0.5, -0.5] + [0] * 25, np.float16)
    cache = torch.full((n_blocks, 36), 0x5A, dtype=torch.uint8, device=dev)
    kvcache.q8_append(_to_dev(x, dev), cache)
    torch.cuda.synchronize()
    got = cache.cpu().numpy()
    exp = np.zeros(n_blocks, O.BLOCK_Q8)
    exp["pad"] = 0x5A5A
    exp_enc = O.q8_encode(x)
    exp["qs"], exp["d"] = exp_enc["qs"], exp_enc["d"]
    assert np.array_equal(got.reshape(-1), exp.view(np.uint8))


def test_q8_dequant_bitexact(dev):
    from qengine_amd import kvcache
    torch = _torch()
    rng = np.random.default_rng(31)
    blocks = O.q8_encode(rng.standard_normal(512 * 32).astype(np.float16) * 3)
    got = kvcache.q8_dequant(_to_dev(blocks.view(np.uint8).reshape(-1, 36), dev))
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy().view(np.uint16), O.q8_decode(blocks))
