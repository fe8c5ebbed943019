// qkv_device.h -- device-side constants and helpers shared by the gfx950 kernels.
//
// Codec data follows the reference exactly:
//   centroids / bounds           turboquant.cuh:27-37 (data, kept identical)
//   sign vector                  turboquant.cuh:288-302 (xorshift64 from 0xCAFEF00D),
//                                evaluated here at compile time into 4 bit masks
//   WHT scale rsqrtf(128)        turboquant.cuh:61, correctly rounded 0x3DB504F3
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qkv {

constexpr int kTqBlock = 128;      // turboquant.cuh:16
constexpr int kTqQsBytes = 48;     // turboquant.cuh:75
constexpr int kTqBlockBytes = 52;  // turboquant.cuh:77
constexpr int kTqBlockDwords = 13;
constexpr int kQ8Block = 32;       // quant_gemv.cuh:8
constexpr int kQ8BlockBytes = 36;  // quant_gemv.cuh:19
constexpr int kQ8BlockDwords = 9;

// ---- sign vector: bit i of kSignMask[i/32] is 1 where sign[i] = +1 --------
constexpr uint64_t xorshift_step(uint64_t s) {
  s ^= s << 13;
  s ^= s >> 7;
  s ^= s << 17;
  return s;
}
constexpr uint32_t sign_word(int w) {
  uint64_t s = 0xCAFEF00DULL;
  uint32_t m = 0;
  for (int i = 0; i < kTqBlock; i++) {
    s = xorshift_step(s);
    if (i / 32 == w && (s & 1u)) m |= 1u << (i % 32);
  }
  return m;
}
constexpr uint32_t kSignMask[4] = {sign_word(0), sign_word(1), sign_word(2), sign_word(3)};
constexpr bool sign_pos(int i) { return (kSignMask[i >> 5] >> (i & 31)) & 1u; }
// Sign word w (0..3) for a runtime w, selected from immediates: indexing the
// constexpr array with a runtime value would turn it into a memory load.
__device__ __forceinline__ uint32_t sign_word_sel(int w) {
  const uint32_t lo = (w & 1) ? kSignMask[1] : kSignMask[0];
  const uint32_t hi = (w & 1) ? kSignMask[3] : kSignMask[2];
  return (w & 2) ? hi : lo;
}
static_assert(sign_word(0) == 0xfae78245u && sign_word(3) == 0x3849957eu,
              "sign vector must match the reference seed");

// ---- codebook ------------------------------------------------------------
__device__ constexpr float kCentroids[8] = {-0.190303f, -0.118828f, -0.066847f, -0.021664f,
                                            0.021664f,  0.066847f,  0.118828f,  0.190303f};
constexpr float kBounds[7] = {-0.154566f, -0.092838f, -0.044256f, 0.000000f,
                              0.044256f,  0.092838f,  0.154566f};
constexpr float kCentroidsHost[8] = {-0.190303f, -0.118828f, -0.066847f, -0.021664f,
                                     0.021664f,  0.066847f,  0.118828f,  0.190303f};

__device__ __forceinline__ float wht_scale() { return __uint_as_float(0x3DB504F3u); }

// turboquant.cuh:79-87: number of bounds strictly below y (NaN -> 0).
__device__ __forceinline__ uint32_t tq3_bin(float y) {
  uint32_t idx = 0;
#pragma unroll
  for (int i = 0; i < 7; i++) idx += (y > kBounds[i]) ? 1u : 0u;
  return idx;
}

// ---- bin thresholds on the WHT output before the x rs scaling -------------
// The reference bins y = fl(w * rs) (turboquant.cuh:145-150).  w -> fl(w * rs)
// is monotone non-decreasing for rs > 0, so for every bound B there is an fp32
// value R with  fl(w * rs) > B  <=>  w > R  for all w (NaN compares false on
// both sides).  R is found by bisection over the bit patterns of non-negative
// floats (ordered like the floats themselves), evaluated at compile time with
// IEEE round-to-nearest-even products:
//   B >= 0:  R = largest w >= 0 with fl(w * rs) <= B
//   B <  0:  fl(w * rs) > B  <=>  fl(-w * rs) < -B  <=>  -w < Q,  Q = smallest
//            w >= 0 with fl(w * rs) >= -B, so R = -Q.
// Some bounds are hit exactly by fl(w * rs), so the negative thresholds are not
// the mirror images of the positive ones; the static_assert pins the values.
constexpr float bits_to_float(uint32_t b) { return __builtin_bit_cast(float, b); }
constexpr uint32_t float_to_bits(float f) { return __builtin_bit_cast(uint32_t, f); }
constexpr float kWhtScaleHost = bits_to_float(0x3DB504F3u);
constexpr uint32_t last_bits_at_most(float bound) {   // largest w >= 0, fl(w*rs) <= bound
  uint32_t lo = 0u, hi = 0x7f800000u;                  // f(lo) <= bound < f(hi)
  while (hi - lo > 1u) {
    const uint32_t mid = lo + (hi - lo) / 2u;
    if (bits_to_float(mid) * kWhtScaleHost <= bound) lo = mid; else hi = mid;
  }
  return lo;
}
constexpr uint32_t first_bits_at_least(float bound) {  // smallest w >= 0, fl(w*rs) >= bound
  uint32_t lo = 0u, hi = 0x7f800000u;                  // f(lo) < bound <= f(hi)
  while (hi - lo > 1u) {
    const uint32_t mid = lo + (hi - lo) / 2u;
    if (bits_to_float(mid) * kWhtScaleHost >= bound) hi = mid; else lo = mid;
  }
  return hi;
}
constexpr uint32_t bin_threshold_bits(int k) {
  return kBounds[k] >= 0.0f ? last_bits_at_most(kBounds[k])
                            : (first_bits_at_least(-kBounds[k]) | 0x80000000u);
}
constexpr uint32_t kBinThrBits[7] = {bin_threshold_bits(0), bin_threshold_bits(1),
                                     bin_threshold_bits(2), bin_threshold_bits(3),
                                     bin_threshold_bits(4), bin_threshold_bits(5),
                                     bin_threshold_bits(6)};
// A lane holding its butterfly output negated (v = -w) bins w as
// 7 - #{m : v > T_m} with T_m = prev(-R_{6-m}) (the next float towards -inf):
// v > prev(-R) <=> v >= -R <=> w <= R <=> NOT fl(w*rs) > B.
constexpr uint32_t prev_float_bits(uint32_t b) {   // next float towards -inf (b finite, != +-0 handled)
  return (b & 0x80000000u) ? b + 1u : (b == 0u ? 0x80000001u : b - 1u);
}
constexpr uint32_t bin_threshold_neg_bits(int m) {
  return prev_float_bits(bin_threshold_bits(6 - m) ^ 0x80000000u);
}
constexpr uint32_t kBinThrNegBits[7] = {bin_threshold_neg_bits(0), bin_threshold_neg_bits(1),
                                        bin_threshold_neg_bits(2), bin_threshold_neg_bits(3),
                                        bin_threshold_neg_bits(4), bin_threshold_neg_bits(5),
                                        bin_threshold_neg_bits(6)};
static_assert(kBinThrNegBits[0] == 0xbfdfd5e4u && kBinThrNegBits[1] == 0xbf86719du &&
                  kBinThrNegBits[2] == 0xbf002dd9u && kBinThrNegBits[3] == 0x80000006u &&
                  kBinThrNegBits[4] == 0x3f002dd7u && kBinThrNegBits[5] == 0x3f86719bu &&
                  kBinThrNegBits[6] == 0x3fdfd5e1u,
              "negated-lane bin thresholds (checked exhaustively on the host)");
static_assert(kBinThrBits[0] == 0xbfdfd5e2u && kBinThrBits[1] == 0xbf86719cu &&
                  kBinThrBits[2] == 0xbf002dd8u && kBinThrBits[3] == 0x00000005u &&
                  kBinThrBits[4] == 0x3f002dd8u && kBinThrBits[5] == 0x3f86719cu &&
                  kBinThrBits[6] == 0x3fdfd5e3u,
              "pre-scale bin thresholds (checked exhaustively against fl(w*rs) on the host)");

// ---- sign-folded binning: one FMA and three compares per element ----------
// y = fma(w, -A, |w|) = -w (A - 1) for w > 0 and |w| (A + 1) for w < 0 (one
// rounding; +0 for w = +-0).  Its sign bit is [w > 0], which is bit 2 of the
// bin (bins 4..7 are w > R_3 = 5 denormal ulps, and no reachable nonzero w is
// that small).  |y| carries |w| scaled by A - 1 on the positive side and by
// A + 1 on the negative side, and that difference absorbs the asymmetry of the
// thresholds (the negative bounds are met with >=, the positive with >), so
// three thresholds Q_j on |y| serve both sides:
//   w > 0:  bin = 4 + m,  w <= 0:  bin = 3 - m,   m = #{j : |y| > Q_j}.
// Q_j lies in [fl(P_j (A-1)), fl(next(P_j)(A-1))) (positive side, P_j = R_{4+j})
// and in [fl(prev(N_j)(A+1)), fl(N_j (A+1))) (negative side, N_j = -R_{2-j});
// A = 2^24 + 2 makes the two intervals overlap for j = 0, 1, 2.  The
// products are exact in double, so the double -> float conversion is the one
// rounding.  Reachable inputs: nonzero WHT outputs of a block with a finite
// norm >= 1e-10 are multiples of 2^-67 (every scaled element is an fp16 value
// over a norm below 2^20), so |w| >= 2^-67; the table is checked exhaustively
// on that domain on the host.
constexpr float kFoldA = 16777218.0f;
constexpr uint32_t fold_product_bits(uint32_t wbits, double c) {
  return float_to_bits((float)((double)bits_to_float(wbits) * c));
}
constexpr uint32_t fold_lo(int j) {
  const uint32_t p = fold_product_bits(kBinThrBits[4 + j], (double)kFoldA - 1.0);
  const uint32_t n = fold_product_bits((kBinThrBits[2 - j] & 0x7fffffffu) - 1u, (double)kFoldA + 1.0);
  return p > n ? p : n;
}
constexpr uint32_t fold_hi(int j) {
  const uint32_t p = fold_product_bits(kBinThrBits[4 + j] + 1u, (double)kFoldA - 1.0);
  const uint32_t n = fold_product_bits(kBinThrBits[2 - j] & 0x7fffffffu, (double)kFoldA + 1.0);
  return p < n ? p : n;
}
static_assert(fold_lo(0) < fold_hi(0) && fold_lo(1) < fold_hi(1) && fold_lo(2) < fold_hi(2),
              "fold constant A separates both sides of every threshold");
constexpr uint32_t kFoldQBits[3] = {fold_lo(0), fold_lo(1), fold_lo(2)};
static_assert(kFoldQBits[0] == 0x4b002dd9u && kFoldQBits[1] == 0x4b86719du &&
                  kFoldQBits[2] == 0x4bdfd5e4u,
              "sign-folded thresholds (checked exhaustively on the host)");

// ---- vector types and raw buffer resources --------------------------------
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef float f2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u3_t __attribute__((ext_vector_type(3)));
typedef uint32_t u2_t __attribute__((ext_vector_type(2)));

// Word 3 of a raw buffer resource on gfx9-family GPUs (32-bit data format).
// Buffer loads past num_records return zero and stores past it are dropped.
constexpr int kBufferRsrcWord3 = 0x00020000;

// ---- fp16 helpers (bit level) ---------------------------------------------
__device__ __forceinline__ float h2f(uint32_t bits16) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16)));
}
__device__ __forceinline__ uint32_t f2h(float f) {  // round-to-nearest-even
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

}  // namespace qkv
