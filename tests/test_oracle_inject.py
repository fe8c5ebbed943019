"""Pins the oracle's DFK2 plane dequantization (dfki2_dequant_kernel,
model.cuh:149-159) against numpy: float32 product of the int8 code and its
group-128 fp16 scale (exact), rounded to fp16 by numpy's float16 cast, over
every int8 value, random and extreme scales (subnormal, overflow to inf,
negative zero, NaN)."""
import numpy as np

from oracle import oracle as O


def _numpy(q, s, kv_dim):
    sf = np.repeat(s.astype(np.float32).reshape(q.shape[0], kv_dim // 128), 128, axis=1)
    with np.errstate(over="ignore", invalid="ignore"):
        return (q.astype(np.float32) * sf).astype(np.float16).view(np.uint16)


def test_dfk2_dequant_matches_numpy():
    rng = np.random.default_rng(11)
    kv_dim, rows = 1024, 300
    q = rng.integers(-128, 128, size=(rows, kv_dim), dtype=np.int8)
    q[0, :256] = np.arange(-128, 128, dtype=np.int16).astype(np.int8)   # every code
    s = (rng.standard_normal((rows, kv_dim // 128)) * 0.02).astype(np.float16)
    s[1] = np.array([6e-8, -6e-8, 65504, -65504, 0, -0.0, np.inf, np.nan], np.float16)
    s[2] = np.float16(600.0)    # 127 * 600 overflows fp16
    got = O.dfk2_dequant(q, s, kv_dim)
    exp = _numpy(q, s, kv_dim)
    nan = np.isnan(exp.view(np.float16))
    assert np.array_equal(np.isnan(got.view(np.float16)), nan)
    assert np.array_equal(got[~nan], exp[~nan])


def test_dfk2_dequant_row_of_one_group():
    q = np.arange(-64, 64, dtype=np.int8).reshape(1, 128)
    s = np.array([[0.5]], np.float16)
    assert np.array_equal(O.dfk2_dequant(q, s, 128).view(np.float16),
                          (np.arange(-64, 64) * 0.5).astype(np.float16).reshape(1, 128))
