"""Pins the CPU oracle's codec functions with checks that do not restate its
formulas: known answers, textbook identities, numpy/scipy routines and fp64
mathematics.  Reference: src/turboquant.cuh, src/attention.cuh:2587-2626."""
import os

import numpy as np
import pytest
from scipy.linalg import hadamard
from scipy.stats import norm as normal

from oracle import oracle as O
from tests._data import kv_f16

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

RS64 = 1.0 / np.sqrt(128.0)


# ---- fp16 conversions ------------------------------------------------------

def test_f16_to_f32_exhaustive():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.f16_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_matches_numpy():
    rng = np.random.default_rng(1)
    f = np.concatenate([
        rng.standard_normal(1 << 18).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 1 << 18),
        rng.integers(0, 2**32, 1 << 18, dtype=np.uint64).astype(np.uint32).view(np.float32),
        # halfway cases between adjacent halves, both parities
        ((np.arange(1, 4096, dtype=np.uint32) << 13) | 0x1000).view(np.float32),
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 5.96e-8, 2.98e-8, 2.99e-8,
                  np.inf, -np.inf], np.float32),
    ]).astype(np.float32)
    got = O.f32_to_f16(f)
    with np.errstate(over="ignore"):
        ref = f.astype(np.float16).view(np.uint16)
    nan = np.isnan(f)
    assert np.array_equal(got[~nan], ref[~nan])
    assert np.all((got[nan] & 0x7C00) == 0x7C00) and np.all((got[nan] & 0x3FF) != 0)


# ---- constants ---------------------------------------------------------------

def test_signs_known_answer():
    # turboquant.cuh:288-302; answer fixed independently of this oracle.
    s = O.tq3_signs()
    assert set(np.unique(s)) == {-1.0, 1.0}
    assert "".join("+" if x > 0 else "-" for x in s[:16]) == "+-+---+--+-----+"
    assert int((s > 0).sum()) == 69
    bits = (s > 0).astype(np.uint64)
    words = [int(sum(int(bits[32 * w + i]) << i for i in range(32))) for w in range(4)]
    assert words == [0xFAE78245, 0xAFCC059F, 0x7D6B44DC, 0x3849957E]


def test_centroids_are_lloyd_max_gaussian_levels():
    c = np.array([-2.1, -1.3, -0.75, -0.25, 0.25, 0.75, 1.3, 2.1])
    for _ in range(500):
        b = (c[1:] + c[:-1]) / 2
        e = np.concatenate([[-np.inf], b, [np.inf]])
        c = (normal.pdf(e[:-1]) - normal.pdf(e[1:])) / (normal.cdf(e[1:]) - normal.cdf(e[:-1]))
    cent = O.tq3_centroids().astype(np.float64)
    assert np.max(np.abs(cent - c * RS64)) < 1.5e-4
    assert np.all(np.diff(cent) > 0)
    assert np.array_equal(cent, -cent[::-1])


def test_bounds_are_centroid_midpoints():
    cent = O.tq3_centroids().astype(np.float64)
    b = O.tq3_bounds().astype(np.float64)
    assert np.max(np.abs(b - (cent[1:] + cent[:-1]) / 2)) < 1e-6
    assert b[3] == 0.0


def test_wht_scale_is_rounded_rsqrt128():
    rs = np.float32(O.wht_scale())
    assert rs.view(np.uint32) == 0x3DB504F3
    assert abs(float(rs) - RS64) <= np.spacing(np.float32(RS64)) / 2


# ---- WHT -------------------------------------------------------------------------

def test_wht_basis_is_sylvester_hadamard():
    H = hadamard(128)
    rs = np.float32(O.wht_scale())
    out = O.wht128(np.eye(128, dtype=np.float32))
    # column i of H (symmetric), times rs, exactly
    assert np.array_equal(out, (H.T * rs).astype(np.float32))


def test_wht_random_vs_fp64_and_involution():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((64, 128)).astype(np.float32)
    y = O.wht128(x)
    ref = (x.astype(np.float64) @ hadamard(128).T) * RS64
    assert np.max(np.abs(y - ref)) < 2e-6
    back = O.wht128(y)
    assert np.max(np.abs(back - x)) < 4e-6


# ---- bins and packing -----------------------------------------------------------

def test_find_bin_matches_searchsorted():
    b = O.tq3_bounds()
    rng = np.random.default_rng(3)
    v = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 0.1,
        b, np.nextafter(b, np.float32(np.inf)), np.nextafter(b, np.float32(-np.inf)),
        np.array([0.0, -0.0, 1e30, -1e30, np.inf, -np.inf], np.float32),
    ]).astype(np.float32)
    got = O.find_bin(v)
    ref = np.searchsorted(b, v, side="left")  # number of bounds strictly below v
    assert np.array_equal(got, ref)
    assert O.find_bin(np.array([np.nan], np.float32))[0] == 0
    assert O.find_bin(np.array([-0.0], np.float32))[0] == 3


def _np_pack(codes):
    """Little-endian 3-bit stream: element e at bits 3e..3e+2."""
    bits = ((codes[:, None] >> np.arange(3)) & 1).astype(np.uint8).reshape(-1)
    return np.packbits(bits, bitorder="little")


def test_pack_unpack_vs_numpy_bitstream():
    rng = np.random.default_rng(4)
    for _ in range(2000):
        idx = rng.integers(0, 8, 8).astype(np.uint8)
        p = O.pack_3bit_8(idx)
        assert np.array_equal(p, _np_pack(idx))
        assert np.array_equal(O.unpack_3bit_8(p), idx)


# ---- TQ3 encode/decode --------------------------------------------------------

def _blocks_input(seed=5):
    rng = np.random.default_rng(seed)
    x = kv_f16(rng, 256, 4, 256).reshape(-1, 128)                  # config-1 regime
    extra = [
        np.zeros(128, np.float16),                                   # zero block
        np.full(128, -0.0, np.float16),
        np.eye(128, dtype=np.float16)[7] * np.float16(3.0),          # one-hot
        (np.eye(128)[0] + np.eye(128)[1]).astype(np.float16),        # exact zeros after WHT
        np.full(128, np.float16(6e-8)),                              # subnormal halves
        np.full(128, np.float16(65504.0)),                           # max half
        (rng.uniform(-1, 1, 128) * 0.1).astype(np.float16),
    ]
    return np.concatenate([x, np.stack(extra)]).astype(np.float16)


def test_encode_norm_is_sequential_fp32_sum():
    x = _blocks_input()
    blocks = O.tq3_encode(x)
    x32 = x.astype(np.float32)
    seq = np.cumsum(x32 * x32, axis=1, dtype=np.float32)[:, -1]  # sequential add.accumulate
    ref = np.sqrt(seq).astype(np.float32)
    assert np.array_equal(blocks["norm"].view(np.uint32), ref.view(np.uint32))


def test_encode_codes_vs_fp64_rotation():
    x = _blocks_input()
    blocks, rot = O.tq3_encode_rotated(x)
    s = O.tq3_signs().astype(np.float64)
    b = O.tq3_bounds().astype(np.float64)
    x64 = x.astype(np.float64)
    nrm = np.sqrt((x64 ** 2).sum(1, keepdims=True))
    live = nrm[:, 0] >= 1e-10
    y = np.zeros_like(x64)
    y[live] = ((x64[live] / nrm[live]) * s) @ hadamard(128).T * RS64
    assert np.max(np.abs(rot[live] - y[live])) < 1e-6
    codes = np.stack([np.concatenate([O.unpack_3bit_8(bl["qs"][3 * g:3 * g + 3])
                                      for g in range(16)]) for bl in blocks])
    exp = np.searchsorted(b, y, side="left").astype(np.uint8)
    near = np.min(np.abs(y[..., None] - b), axis=-1) < 1e-6
    ok = (codes == exp) | near
    assert ok[live].all()
    assert near[live].mean() < 1e-3
    # zero blocks: norm stored, all-zero packed bytes (turboquant.cuh:133-140)
    assert np.all(blocks["qs"][~live] == 0)
    assert np.all(blocks["norm"][~live] == 0)


def test_encode_code_histogram_is_gaussian_like():
    rng = np.random.default_rng(6)
    x = kv_f16(rng, 1024, 4, 256, outlier_frac=0.0).reshape(-1, 128)
    blocks = O.tq3_encode(x)
    codes = np.stack([np.concatenate([O.unpack_3bit_8(bl["qs"][3 * g:3 * g + 3])
                                      for g in range(16)]) for bl in blocks[:2048]])
    hist = np.bincount(codes.ravel(), minlength=8) / codes.size
    # P(bin) under N(0, 1/128) for the Lloyd-Max bounds (closed form)
    e = np.concatenate([[-np.inf], O.tq3_bounds().astype(np.float64) / RS64, [np.inf]])
    p = normal.cdf(e[1:]) - normal.cdf(e[:-1])
    assert np.max(np.abs(hist - p)) < 0.01


def test_decode_vs_fp64_inverse_rotation():
    x = _blocks_input()
    blocks = O.tq3_encode(x)
    c = O.tq3_centroids().astype(np.float64)
    s = O.tq3_signs().astype(np.float64)
    codes = np.stack([np.concatenate([O.unpack_3bit_8(bl["qs"][3 * g:3 * g + 3])
                                      for g in range(16)]) for bl in blocks])
    ref = (c[codes] @ hadamard(128).T) * RS64 * s * blocks["norm"][:, None].astype(np.float64)
    got32 = O.tq3_decode_f32(blocks).reshape(-1, 128)
    scale = np.maximum(blocks["norm"][:, None].astype(np.float64), 1e-30)
    assert np.max(np.abs(got32 - ref) / scale) < 2e-6
    got16 = O.tq3_decode(blocks).reshape(-1, 128)
    with np.errstate(over="ignore"):
        assert np.array_equal(got16, got32.astype(np.float16).view(np.uint16))


def test_roundtrip_relmse_matches_gaussian_theory():
    rng = np.random.default_rng(7)
    x = kv_f16(rng, 1024, 4, 256, outlier_frac=0.0).reshape(-1, 128)
    blocks = O.tq3_encode(x)
    y = O.f16_to_f32(O.tq3_decode(blocks)).reshape(-1, 128).astype(np.float64)
    x64 = x.astype(np.float64)
    rel = ((y - x64) ** 2).sum() / (x64 ** 2).sum()
    assert 0.030 < rel < 0.040            # 3-bit Lloyd-Max Gaussian MSE = 0.0345


# ---- Q8_0 -------------------------------------------------------------------------

def test_q8_closed_form_bounds():
    rng = np.random.default_rng(42)
    x = rng.uniform(-3, 3, (64, 32)).astype(np.float16)   # tools/test_q8kv_roundtrip.cu regime
    blk = O.q8_encode(x)
    x32 = x.astype(np.float32)
    amax = np.abs(x32).max(1)
    scale = (amax / np.float32(127.0)).astype(np.float32)
    assert np.array_equal(blk["d"], scale.astype(np.float16).view(np.uint16))
    q = blk["qs"].astype(np.float64)
    assert np.all(np.abs(q) <= 127)
    assert np.all(np.abs(x32 - q * scale[:, None]) <= scale[:, None] * 0.5 * (1 + 1e-6))
    assert np.all(np.abs(q[np.arange(64), np.abs(x32).argmax(1)]) == 127)
    assert np.all(blk["pad"] == 0)
    inv = np.where(scale > 0, np.float32(1.0) / scale, np.float32(0)).astype(np.float32)
    assert np.array_equal(blk["qs"], np.rint((x32 * inv[:, None]).astype(np.float32)).astype(np.int8))


def test_q8_special_cases():
    z = O.q8_encode(np.zeros((1, 32), np.float16))
    assert z["d"][0] == 0 and np.all(z["qs"] == 0)
    # amax = 127 -> scale 1.0 exactly; halfway values round to even
    x = np.zeros(32, np.float16)
    x[0] = 127.0
    x[1:7] = [2.5, 3.5, -2.5, -3.5, 0.5, -0.5]
    blk = O.q8_encode(x)
    assert list(blk["qs"][0][:7]) == [127, 2, 4, -2, -4, 0, 0]
    assert np.float16(1.0).view(np.uint16) == blk["d"][0]


def test_q8_decode_vs_numpy():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((128, 32)).astype(np.float16)
    blk = O.q8_encode(x)
    d = blk["d"].view(np.float16).astype(np.float32)
    ref = (blk["qs"].astype(np.float32) * d[:, None]).astype(np.float16).view(np.uint16)
    assert np.array_equal(O.q8_decode(blk).reshape(128, 32), ref)


# ---------------------------------------------------------------------------
# Pre-scale bin thresholds used by the GPU encoder: binning the WHT output w
# against them is the same as binning fl(w * rs) against the reference bounds
# (turboquant.cuh:145-150), for every fp32 value.
# ---------------------------------------------------------------------------
PRESCALE_THR = [0xbfdfd5e2, 0xbf86719c, 0xbf002dd8, 0x00000005,
                0x3f002dd8, 0x3f86719c, 0x3fdfd5e3]
# for a lane that carries its butterfly output negated (v = -w):
# bin(w) = 7 - #{m : v > T_m},  T_m = prev(-R_{6-m})
PRESCALE_THR_NEG = [0xbfdfd5e4, 0xbf86719d, 0xbf002dd9, 0x80000006,
                    0x3f002dd7, 0x3f86719b, 0x3fdfd5e1]


def test_prescale_thresholds_match_device_header():
    import re
    hdr = open(os.path.join(ROOT, "qengine_amd", "csrc", "qkv_device.h")).read()
    pinned = {int(k): int(v, 16) for k, v in re.findall(r"kBinThrBits\[(\d)\] == (0x[0-9a-f]+)u", hdr)}
    assert pinned == dict(enumerate(PRESCALE_THR))
    neg = {int(k): int(v, 16) for k, v in re.findall(r"kBinThrNegBits\[(\d)\] == (0x[0-9a-f]+)u", hdr)}
    assert neg == dict(enumerate(PRESCALE_THR_NEG))


FOLD_A = 0x4b800001          # 2^24 + 2
FOLD_Q = [0x4b002dd9, 0x4b86719d, 0x4bdfd5e4]


def test_fold_thresholds_match_device_header():
    import re
    hdr = open(os.path.join(ROOT, "qengine_amd", "csrc", "qkv_device.h")).read()
    pinned = {int(k): int(v, 16) for k, v in re.findall(r"kFoldQBits\[(\d)\] == (0x[0-9a-f]+)u", hdr)}
    assert pinned == dict(enumerate(FOLD_Q))
    a = re.search(r"kFoldA = ([0-9.]+)f;", hdr).group(1)
    assert np.float32(float(a)).view(np.uint32) == FOLD_A


@pytest.mark.parametrize("negated", [False, True])
def test_fold_binning_exhaustive(negated):
    assert O.fold_mismatches(FOLD_A, FOLD_Q, negated=negated) == 0


@pytest.mark.parametrize("k,delta", [(0, 1), (0, -1), (1, 1), (1, -1), (2, 1), (2, -1)])
def test_fold_binning_one_ulp_off_fails(k, delta):
    q = list(FOLD_Q)
    q[k] += delta
    # the patterns near the pre-scale threshold pair this Q separates
    for neg in (False, True):
        assert O.fold_mismatches(FOLD_A, FOLD_Q, 0x3f000000, 0x40000000, negated=neg) == 0
    bad = sum(O.fold_mismatches(FOLD_A, q, lo, hi, negated=neg)
              for lo, hi in ((0x3f000000, 0x40000000), (0xbf000000, 0xc0000000))
              for neg in (False, True))
    assert bad > 0


def test_fold_binning_needs_the_offset():
    # A = 2^24 (no asymmetry between the sides) cannot serve both signs
    q = [int(np.float32(np.float64(np.uint32(b).view(np.float32)) * 2.0**24).view(np.uint32))
         for b in PRESCALE_THR[4:]]
    bad = sum(O.fold_mismatches(0x4b800000, q, lo, hi, negated=False)
              for lo, hi in ((0x3f000000, 0x40000000), (0xbf000000, 0xc0000000)))
    assert bad > 0


def test_prescale_thresholds_exhaustive():
    assert O.prescale_threshold_mismatches(PRESCALE_THR) == 0


def test_prescale_thresholds_negated_exhaustive():
    assert O.prescale_threshold_mismatches(PRESCALE_THR_NEG, negated=True) == 0


@pytest.mark.parametrize("k,delta", [(0, -1), (3, 1), (4, 1), (6, 1)])
def test_prescale_thresholds_negated_one_ulp_off_fails(k, delta):
    thr = list(PRESCALE_THR_NEG)
    thr[k] = (thr[k] + delta) & 0xffffffff
    lo, hi = max(0, thr[k] - (1 << 15)), min(0xFFFFFFFF, thr[k] + (1 << 15))
    assert O.prescale_threshold_mismatches(PRESCALE_THR_NEG, lo, hi, negated=True) == 0
    assert O.prescale_threshold_mismatches(thr, lo, hi, negated=True) > 0


@pytest.mark.parametrize("k,delta", [(0, 1), (1, -1), (2, -1), (3, -5), (4, 1), (5, 1), (6, -1)])
def test_prescale_thresholds_one_ulp_off_fails(k, delta):
    """Moving any threshold by one ulp (the zero bound's to +0) breaks the
    equivalence; the search window is the 2^16 patterns around it."""
    thr = list(PRESCALE_THR)
    thr[k] = (thr[k] + delta) & 0xffffffff
    lo, hi = max(0, thr[k] - (1 << 15)), min(0xFFFFFFFF, thr[k] + (1 << 15))
    assert O.prescale_threshold_mismatches(PRESCALE_THR, lo, hi) == 0
    assert O.prescale_threshold_mismatches(thr, lo, hi) > 0


def test_move_token_rows_known_answer():
    """The reference's per-token copies in list order (model.cuh:7430-7471):
    rows A B C D E with moves 2->0, 0->3, 4->4 (no-op), 1->2 give C B B C E,
    worked out by hand (the second move copies the row the first one wrote)."""
    rows = np.array([[ord(c)] * 4 for c in "ABCDE"], np.uint8)
    got = O.move_token_rows(rows, [(2, 0), (0, 3), (4, 4), (1, 2)])
    assert bytes(got[:, 0]).decode() == "CBBCE"
    got = O.move_token_rows(rows, [(0, 1)], slot_row0=2)     # slot starting at row 2
    assert bytes(got[:, 0]).decode() == "ABCCE"
