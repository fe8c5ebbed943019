"""Pins the oracle's restatement of the reference's short-context decode
(model.cuh:2544-2664; attention.cuh:277-316, 400-483, 531-575, 885-907,
920-989) with checks that do not retype it:

- fp64 softmax attention over the same fp16 scratch (or the fp32 dequantized
  values for the TQ_FUSED kernels): every output element within half an fp16
  ulp of the fp64 value plus 2e-6 of its row's largest magnitude;
- the softmax rows against fp64 softmax of fp64 scores within 2e-6 (relative),
  and each row summing to 1 within 1e-6;
- with integer-valued query and keys every partial sum of the score
  reduction is exact, so the probabilities must equal the fp64 softmax of the
  exact integer scores to within fp32 exp/sum rounding;
- seq_len 1: probability exactly 1 and the output the value row itself.
A dropped term, a wrong key/head index or a wrong reduction width fails the
first two by orders of magnitude."""
import numpy as np
import pytest

from oracle import oracle as O
from tests._data import kv_f16, q_f16

HD, NKV = 256, 4


def _half_ulp(x):
    """Half an fp16 ulp of |x| (subnormal spacing below 2^-14)."""
    a = np.abs(x)
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
    return 0.5 * 2.0 ** (e - 10)


def _check_vs_f64(out_bits, ref, tag):
    out = out_bits.view(np.float16).astype(np.float64).reshape(ref.shape)
    rowmax = np.abs(ref).max(axis=-1, keepdims=True)
    bound = _half_ulp(ref) * 1.0001 + 2e-6 * rowmax
    bad = np.abs(out - ref) > bound
    assert not bad.any(), (tag, int(bad.sum()), float(np.max(np.abs(out - ref) - bound)))


def _softmax64(q, k64, num_q, seq_len, scale):
    gqa = num_q // NKV
    qf = q.reshape(num_q, HD).astype(np.float64)
    s = np.stack([k64[:seq_len, h // gqa] @ qf[h] for h in range(num_q)]) * scale
    w = np.exp(s - s.max(axis=1, keepdims=True))
    return w / w.sum(axis=1, keepdims=True)


@pytest.mark.parametrize("seq_len", [1, 2, 3, 100, 256, 300, 1000, 4095])
@pytest.mark.parametrize("kind", ["tq3", "q8", "f16", "q8k_tq3v"])
def test_legacy_default_vs_f64(kind, seq_len):
    rng = np.random.default_rng(seq_len * 13 + len(kind))
    num_q = 16
    k16, v16 = kv_f16(rng, seq_len, NKV, HD), kv_f16(rng, seq_len, NKV, HD)
    q = q_f16(rng, 1, num_q, HD)
    if kind == "tq3":
        kk, vk, k, v = O.KV_TQ3, O.KV_TQ3, O.tq3_encode(k16), O.tq3_encode(v16)
        ks, vs = O.tq3_decode(k), O.tq3_decode(v)
    elif kind == "q8":
        kk, vk, k, v = O.KV_Q8, O.KV_Q8, O.q8_encode(k16), O.q8_encode(v16)
        ks, vs = O.q8_decode(k), O.q8_decode(v)
    elif kind == "f16":
        kk, vk, k, v = O.KV_F16, O.KV_F16, k16, v16
        ks, vs = k16.view(np.uint16), v16.view(np.uint16)
    else:   # TQ_KEYS_Q8: keys Q8_0, values TQ3 (model.cuh:2574-2588, 2626-2645)
        kk, vk, k, v = O.KV_Q8, O.KV_TQ3, O.q8_encode(k16), O.tq3_encode(v16)
        ks, vs = O.q8_decode(k), O.tq3_decode(v)
    k64 = O.f16_to_f32(np.asarray(ks).reshape(-1)).astype(np.float64).reshape(seq_len, NKV, HD)
    v64 = O.f16_to_f32(np.asarray(vs).reshape(-1)).astype(np.float64).reshape(seq_len, NKV, HD)
    out, probs = O.legacy_decode(kk, vk, q, k, v, num_q=num_q, num_kv=NKV, hd=HD,
                                 seq_len=seq_len, scale=1 / 16, return_probs=True)
    p64 = _softmax64(q, k64, num_q, seq_len, 1 / 16)
    assert np.allclose(probs, p64, rtol=2e-6, atol=1e-12), np.max(np.abs(probs - p64) / p64)
    assert np.allclose(probs.astype(np.float64).sum(axis=1), 1.0, atol=1e-6)
    gqa = num_q // NKV
    ref = np.stack([p64[h] @ v64[:, h // gqa] for h in range(num_q)])
    _check_vs_f64(out, ref, (kind, seq_len))


@pytest.mark.parametrize("seq_len", [1, 5, 257, 2000])
def test_legacy_tq_fused_vs_f64(seq_len):
    """TQ_FUSED kernels: fp32 dequantization without fp16 rounding; reference
    values are the fp64 rotation of the codes (tq3_decode_f32 is within one
    fp32 ulp of it)."""
    rng = np.random.default_rng(77 + seq_len)
    num_q = 24
    kb, vb = O.tq3_encode(kv_f16(rng, seq_len, NKV, HD)), O.tq3_encode(kv_f16(rng, seq_len, NKV, HD))
    q = q_f16(rng, 1, num_q, HD)
    k64 = O.tq3_decode_f32(kb).astype(np.float64).reshape(seq_len, NKV, HD)
    v64 = O.tq3_decode_f32(vb).astype(np.float64).reshape(seq_len, NKV, HD)
    out, probs = O.legacy_decode(O.KV_TQ3, O.KV_TQ3, q, kb, vb, num_q=num_q, num_kv=NKV, hd=HD,
                                 seq_len=seq_len, scale=1 / 16, tq_fused=True, return_probs=True)
    p64 = _softmax64(q, k64, num_q, seq_len, 1 / 16)
    assert np.allclose(probs, p64, rtol=4e-6, atol=1e-12)
    gqa = num_q // NKV
    ref = np.stack([p64[h] @ v64[:, h // gqa] for h in range(num_q)])
    _check_vs_f64(out, ref, ("fused", seq_len))


def test_legacy_integer_scores_exact():
    """Integer-valued q and k (|q|, |k| <= 8): the fp32 score sums are exact,
    whatever the association, so the probabilities match fp64 to exp/sum
    rounding only; a missing or doubled warp sum breaks it."""
    rng = np.random.default_rng(5)
    seq_len, num_q = 600, 16
    k = rng.integers(-8, 9, size=(seq_len, NKV, HD)).astype(np.float16)
    v = rng.integers(-8, 9, size=(seq_len, NKV, HD)).astype(np.float16)
    q = rng.integers(-8, 9, size=(1, num_q, HD)).astype(np.float16)
    scale = 2.0 ** -8
    out, probs = O.legacy_decode(O.KV_F16, O.KV_F16, q, k, v, num_q=num_q, num_kv=NKV, hd=HD,
                                 seq_len=seq_len, scale=scale, return_probs=True)
    p64 = _softmax64(q, k.astype(np.float64), num_q, seq_len, scale)
    assert np.allclose(probs, p64, rtol=2e-6, atol=1e-30)


def test_legacy_single_row():
    rng = np.random.default_rng(9)
    k16, v16 = kv_f16(rng, 1, NKV, HD), kv_f16(rng, 1, NKV, HD)
    q = q_f16(rng, 1, 16, HD)
    out, probs = O.legacy_decode(O.KV_F16, O.KV_F16, q, k16, v16, num_q=16, num_kv=NKV, hd=HD,
                                 seq_len=1, scale=1 / 16, return_probs=True)
    assert np.all(probs == 1.0)
    for h in range(16):
        assert np.array_equal(out[h], v16[0, h // 4].view(np.uint16))


def test_legacy_rejects_bad_shapes():
    q = np.zeros((16, HD), np.float16)
    k = np.zeros((4, NKV, HD), np.float16)
    with pytest.raises(ValueError):
        O.legacy_decode(O.KV_F16, O.KV_F16, q, k, k, num_q=16, num_kv=NKV, hd=HD, seq_len=0,
                        scale=1.0)
