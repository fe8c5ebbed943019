// tq3_encode.h -- TQ3 encoding of one 128-element fp16 block spread over a
// 16-lane DPP row (turboquant.cuh:112-165), shared by the small-append kernel
// and the decode kernel that appends a verify block's rows itself.
//
// Lane t of the row holds elements 8t..8t+7 (one 16-byte piece):
//   - norm: the reference's sequential sum runs through the row, each lane
//     adding its 8 squares to its left neighbour's partial (row_shr:1), 16
//     steps; lane 15 ends with the block's sum;
//   - scaling with the random sign folded into the factor;
//   - WHT stages 1..4 in registers, stages 8..64 across lanes t ^ 1, t ^ 2,
//     t ^ 4 and t ^ 8 of the row (DPP quad_perm, half_mirror, mirror): the
//     lower element of a pair becomes own + other, the upper other - own,
//     the reference's roundings;
//   - bins in the sign-folded form, 8 codes = 24 bits per lane (bits
//     24t..24t+23 of the code stream), gathered into the 12 code dwords by
//     lanes 0..11 (ds_bpermute).
// Every float operation that feeds a code or the norm is the reference's
// single-rounding IEEE operation in its order (no contraction), so the block
// is bit-identical to the reference's.
#pragma once
#include "qkv_device.h"

namespace qkv {

template <int CTRL>
__device__ __forceinline__ float row_dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf,
                                                            false));
}

// One cross-lane WHT stage on the lane's 8 elements: partner values through
// the DPP path P (1: t ^ 1, 2: t ^ 2, 4: t ^ 4, 8: t ^ 8 within the row).
template <int P>
__device__ __forceinline__ void row_stage(float (&x)[8], bool upper) {
  const uint32_t flip = upper ? 0x80000000u : 0u;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    float o;
    if constexpr (P == 1) o = row_dpp<0xB1>(x[i]);                   // quad_perm [1,0,3,2]
    else if constexpr (P == 2) o = row_dpp<0x4E>(x[i]);              // quad_perm [2,3,0,1]
    else if constexpr (P == 4) o = row_dpp<0x1B>(row_dpp<0x141>(x[i]));   // i^7, then i^3
    else o = row_dpp<0x141>(row_dpp<0x140>(x[i]));                   // i^15, then i^7
    // lower: own + other; upper: other - own (= other + (-own), one rounding)
    x[i] = o + __uint_as_float(__float_as_uint(x[i]) ^ flip);
  }
}

// Encode the block whose 16-byte piece `raw` this lane holds (lane & 15 = t).
// Returns the dword lane t stores into the 13-dword block: dword 1 + t (code
// dword t) for t < 12, dword 0 (the fp32 norm) for t == 12; lanes 13..15
// store nothing.  All 16 lanes of the row must be active.
__device__ __forceinline__ uint32_t tq3_encode_row16(uint4 raw, int lane) {
#pragma clang fp contract(off)
  const int t = lane & 15;
  const uint32_t rw[4] = {raw.x, raw.y, raw.z, raw.w};
  float h[8];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    h[2 * k] = h2f(rw[k] & 0xffffu);
    h[2 * k + 1] = h2f(rw[k] >> 16);
  }
  // norm (reference order): lane t continues lane t - 1's partial
  float part = 0.0f;
#pragma unroll
  for (int r = 0; r < 16; r++) {
    float s = part;
#pragma unroll
    for (int i = 0; i < 8; i++) s = __builtin_fmaf(h[i], h[i], s);
    part = r < 15 ? __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                                  0, __builtin_bit_cast(int, s), 0x111, 0xf, 0xf, false))
                  : s;   // row_shr:1
  }
  const float norm_sq =
      __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((lane | 15) << 2, __builtin_bit_cast(int, part)));
  const float norm = __builtin_sqrtf(norm_sq);
  const float inv = 1.0f / norm;
  // x * inv * sign (turboquant.cuh:141-149)
  const uint32_t sbits = sign_word_sel(t >> 2) >> (8 * (t & 3));   // elements 8t..8t+7
  float x[8];
#pragma unroll
  for (int i = 0; i < 8; i++) x[i] = __builtin_fmaf(h[i], ((sbits >> i) & 1u) ? inv : -inv, 0.0f);
  // WHT stages 1, 2, 4 in registers, 8 .. 64 across the row (turboquant.cuh:50-59)
#pragma unroll
  for (int step = 1; step < 8; step <<= 1) {
#pragma unroll
    for (int i = 0; i < 8; i += 2 * step) {
#pragma unroll
      for (int j = i; j < i + step; j++) {
        const float a = x[j], c = x[j + step];
        x[j] = a + c;
        x[j + step] = a - c;
      }
    }
  }
  row_stage<1>(x, (t & 1) != 0);
  row_stage<2>(x, (t & 2) != 0);
  row_stage<4>(x, (t & 4) != 0);
  row_stage<8>(x, (t & 8) != 0);
  // bins, sign-folded: bit 2 = [w > 0] (sign of y), bits 1..0 = the
  // thermometer count m of |y| against the fold thresholds, inverted for w <= 0
  const float q0 = __uint_as_float(kFoldQBits[0]), q1 = __uint_as_float(kFoldQBits[1]),
              q2 = __uint_as_float(kFoldQBits[2]);
  uint32_t v = 0u;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const float y = __builtin_fmaf(x[i], -kFoldA, __builtin_fabsf(x[i]));
    const float ay = __builtin_fabsf(y);
    const uint32_t m = (uint32_t)(ay > q0) + (uint32_t)(ay > q1) + (uint32_t)(ay > q2);
    const uint32_t code = (__float_as_uint(y) >> 31) ? 4u + m : 3u - m;
    v |= code << (3 * i);
  }
  const bool keep = norm >= 1e-10f && norm < __builtin_inff();
  // code dword k (k = t < 12): bytes 4k..4k+3 of the stream, from lanes a and
  // a + 1 of the row, a = 4k / 3
  const int a = (4 * t) / 3, off = 4 * t - 3 * a;
  const int row0 = lane & ~15;
  const uint32_t va = (uint32_t)__builtin_amdgcn_ds_bpermute((row0 + a) << 2, (int)v);
  const uint32_t vb = (uint32_t)__builtin_amdgcn_ds_bpermute((row0 + min(a + 1, 15)) << 2, (int)v);
  const uint64_t pair = (uint64_t)va | ((uint64_t)vb << 24);
  const uint32_t word = keep ? (uint32_t)(pair >> (8 * off)) : 0u;
  return t == 12 ? __float_as_uint(norm) : word;
}

}  // namespace qkv
