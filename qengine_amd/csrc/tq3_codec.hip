// tq3_codec.hip -- TQ3 append (encode) and dequant kernels for gfx950.
//
// Reference arithmetic: turboquant.cuh:112-165 (encode) and 169-200 (decode).
//
// Append layout on the GPU: a lane pair encodes two 128-element blocks; lane
// l of a 64-block wave tile holds the first half of block l and the second
// half of block l ^ 1, loaded straight into registers.  Waves are persistent
// (three per SIMD) and take 64-block tiles in turn.  Each lane runs the
// reference's sequential norm over its first half, hands the partial to the
// other lane of the pair, which continues over its second half; then the
// unit scaling with the random signs and the butterfly WHT in registers (the
// last stage across the lane pair through DPP, after which lane l holds all
// of block l), bins the result in a sign-folded form that reproduces binning
// fl(w * rs) exactly, and the wave writes its 64 x 52-byte output through an
// LDS staging area with dword stores that cover whole cache lines.  Every
// float operation that feeds a code or a norm is the same single-rounding
// IEEE operation in the same order as the reference, so codes and norms are
// bit-identical.  The dequant kernel keeps one lane per block.
#include <algorithm>
#include <atomic>

#include "qkv_device.h"
#include "qkv_launch.h"
#include "tq3_encode.h"

// Bit-exact codec: no FMA contraction across the reference's separate roundings.
#pragma clang fp contract(off)

namespace qkv {

constexpr int kCodecWaves = 4;                  // waves per workgroup
constexpr int kCodecThreads = 64 * kCodecWaves;
constexpr int kInPitchDw = 68;                  // 64 dwords of fp16 + 4 pad
constexpr int kWaveLdsDw = 64 * kInPitchDw;     // 17408 B per wave

// ---------------------------------------------------------------------------
// In-register 128-point Walsh-Hadamard butterflies (turboquant.cuh:50-59).
// Each stage pairs (j, j+step) -> (a+b, a-b), exactly as the reference.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void wht128_butterflies(float (&x)[128]) {
#pragma unroll
  for (int step = 1; step < 128; step <<= 1) {
#pragma unroll
    for (int i = 0; i < 128; i += 2 * step) {
#pragma unroll
      for (int j = i; j < i + step; j++) {
        float a = x[j], b = x[j + step];
        x[j] = a + b;
        x[j + step] = a - b;
      }
    }
  }
}

// Bit planes of two elements from their sign-folded values ya, yb (see
// kFoldQBits): c_j = [|y| > Q_j] is a thermometer code of m, so bit 1 of m is
// c_1 and bit 0 is c_0 ^ c_1 ^ c_2.  pa[0] = bit 1, pa[1] = bit 0 of element
// a's m (likewise pb); the XORs run on the scalar unit.  The sign fix (bits
// 0 and 1 of the bin are those of m, or inverted for w <= 0) is applied to
// the packed words afterwards.
__device__ __forceinline__ void fold_planes2(float ya, float yb, const uint32_t (&q)[3],
                                             uint64_t (&pa)[2], uint64_t (&pb)[2]) {
  uint64_t a2, b2;
  asm("v_cmp_gt_f32_e64 %[a1], |%[ya]|, %[q1]\n\t"
      "v_cmp_gt_f32_e64 %[b1], |%[yb]|, %[q1]\n\t"
      "v_cmp_gt_f32_e64 %[a0], |%[ya]|, %[q0]\n\t"
      "v_cmp_gt_f32_e64 %[a2], |%[ya]|, %[q2]\n\t"
      "v_cmp_gt_f32_e64 %[b0], |%[yb]|, %[q0]\n\t"
      "v_cmp_gt_f32_e64 %[b2], |%[yb]|, %[q2]\n\t"
      "s_xor_b64 %[a0], %[a0], %[a2]\n\t"
      "s_xor_b64 %[b0], %[b0], %[b2]\n\t"
      "s_xor_b64 %[a0], %[a0], %[a1]\n\t"
      "s_xor_b64 %[b0], %[b0], %[b1]"
      : [a1] "=&s"(pa[0]), [a0] "=&s"(pa[1]), [a2] "=&s"(a2), [b1] "=&s"(pb[0]),
        [b0] "=&s"(pb[1]), [b2] "=&s"(b2)
      : [ya] "v"(ya), [yb] "v"(yb), [q0] "s"(q[0]), [q1] "s"(q[1]), [q2] "s"(q[2]));
}

// acc = 2 * acc + (sign bit of y): shifts bit 2 of a bin in.
__device__ __forceinline__ void shift_in_sign(uint32_t& acc, float y) {
  acc = __builtin_amdgcn_alignbit(acc, __float_as_uint(y), 31);
}

// Mask of the bit-2 positions (bit 3e+2 of the code stream) in word w.
constexpr uint32_t bit2_mask(int w) {
  uint32_t m = 0u;
  for (int p = 0; p < 32; p++)
    if ((32 * w + p) % 3 == 2) m |= 1u << p;
  return m;
}

// Sign fix of packed words (w0 .. w0+n-1 of the stream, whose last element
// ends inside them): for every element with bit 2 clear (w <= 0), invert bits
// 1 and 0.  nb = the bit-2 positions that are clear, moved down by one and by
// two bits (across word boundaries with a funnel shift).
template <int W0, int N>
__device__ __forceinline__ void sign_fix(uint32_t* acc) {
  uint32_t nb[N + 1];
#pragma unroll
  for (int i = 0; i < N; i++) nb[i] = ~acc[i] & bit2_mask(W0 + i);
  nb[N] = 0u;
#pragma unroll
  for (int i = 0; i < N; i++)
    acc[i] ^= __builtin_amdgcn_alignbit(nb[i + 1], nb[i], 1) ^
              __builtin_amdgcn_alignbit(nb[i + 1], nb[i], 2);
}

// acc = 2 * acc + (this lane's bit of the mask): shifts one plane bit in.
__device__ __forceinline__ void shift_in(uint32_t& acc, uint64_t plane) {
  uint64_t cy;
  asm("v_addc_co_u32_e64 %[a], %[cy], %[a], %[a], %[p]"
      : [a] "+v"(acc), [cy] "=&s"(cy) : [p] "s"(plane));
}

// This lane's index (0..63) from mbcnt of a mask the compiler cannot see as
// constant, so that it is formed where it is used instead of being hoisted
// and kept (or spilled) across a loop.
__device__ __forceinline__ int opaque_lane() {
  uint32_t all = ~0u;
  asm volatile("" : "+s"(all));
  return (int)__builtin_amdgcn_mbcnt_hi(all, __builtin_amdgcn_mbcnt_lo(all, 0u));
}

// Output block of input block i for a paged append (PagedRows), or -1 when
// the row it maps to lies outside the pool (then nothing is written).  The
// divisions run in 32 bits: i < n_blocks < 2^31, and a position past INT_MAX
// (int32 positions, as in the reference) maps to no row.
__device__ __forceinline__ long paged_block(const PagedRows& pr, long i) {
  const int ii = (int)i;
  const int tok = ii / pr.blocks_per_row;
  const int j = ii - tok * pr.blocks_per_row;
  const int s = tok / pr.n_tok, t = tok - s * pr.n_tok;
  const long pos = (long)pr.positions[s] + t;
  if (pos < 0 || pos > 0x7fffffffL) return -1;
  const int b = (int)pos / pr.block_tokens;
  if (b >= pr.max_blocks) return -1;
  const long row = (long)pr.block_tables[(long)s * pr.max_blocks + b] * pr.block_tokens +
                   (pos - b * pr.block_tokens);
  if (row < 0 || row >= pr.pool_rows) return -1;
  return row * pr.blocks_per_row + j;
}

// dfki2_dequant_kernel's element (model.cuh:149-159): half(float(q) * float(s));
// the product of an int8 and an fp16 is exact in fp32, then one rounding.
__device__ __forceinline__ uint32_t dfk2_pair(uint32_t word, int byte, float s) {
  const float a = (float)(int8_t)((word >> (8 * byte)) & 0xffu) * s;
  const float b = (float)(int8_t)((word >> (8 * byte + 8)) & 0xffu) * s;
  return f2h(a) | (f2h(b) << 16);
}

template <int CTRL>
__device__ __forceinline__ float lane_dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                       __builtin_bit_cast(int, v), __builtin_bit_cast(int, v),
                                       CTRL, 0xf, 0xf, false));
}

// ---------------------------------------------------------------------------
// Append: a lane pair encodes two blocks.
//
// Lane l of a 64-block wave tile holds R1 = elements 0..63 of block l and
// R2 = elements 64..127 of block l ^ 1 (16 KiB of fp16 per tile), loaded
// straight into registers (lane l reads the 128-byte lines it needs; the 8
// loads of a line are consecutive, so the line is fetched once).  No
// prefetch registers: three waves per SIMD cover each other's load waits.
// Per tile:
//   - norm: the reference's sequential sum of block b runs over its first
//     half in lane b (R1), then -- the partial handed over by DPP -- over its
//     second half in lane b ^ 1 (R2).  Every chain step is useful: a lane runs
//     128 steps for its 128 elements (a pair with one block would run 128 steps
//     for 64 elements per lane);
//   - scaling by the inverse norms with the random signs folded into the
//     factors (R1: block l's factor, R2: block l ^ 1's);
//   - WHT stages 1..32 in registers on R1 and on R2; stage 64 pairs element k
//     of R1 in lane l with element k of R2 in lane l ^ 1 (both halves of block
//     l): a DPP-sourced add and reverse subtract give a + b and a - b, so lane
//     l then holds all 128 outputs of block l;
//   - bins in the sign-folded form (kFoldQBits), codes words 0..5 from the
//     first 64 outputs and 6..11 from the last 64; the lane writes its whole
//     block (through LDS and coalesced dword stores when contiguous).
// ---------------------------------------------------------------------------
constexpr int kAp4Waves = 4;
constexpr int kAp4Threads = 64 * kAp4Waves;
constexpr int kAp4Tile = 64;                           // blocks per wave tile
constexpr int kAp4WaveLdsDw = kAp4Tile * 13;           // output staging, 3328 B per wave

// This lane's halves of a 64-block tile (blocks b0 .. b0+nb-1): h1 = fp16
// elements 0..63 of block b0 + lane, h2 = elements 64..127 of block
// b0 + (lane ^ 1).  Blocks past the last read zero (range-checked resource).
// A DFK2 source (int8 rows, one fp16 scale per block) is dequantized here to
// the reference's fp16 values.
template <bool kDfk2>
__device__ __forceinline__ void load_halves(uint32_t (&h1)[32], uint32_t (&h2)[32],
                                            const uint4* __restrict__ in,
                                            const uint16_t* __restrict__ sc, int b0, int nb,
                                            int lane) {
  if constexpr (kDfk2) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint4*>(in + (long)b0 * 8), 0, nb * 128, kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t rsc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(sc + b0), 0, nb * 2, kBufferRsrcWord3);
    u4_t c1[4], c2[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      c1[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, lane * 128, 16 * k, 0);
      c2[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, (lane ^ 1) * 128 + 64, 16 * k, 0);
    }
    const float s1 = h2f(__builtin_amdgcn_raw_buffer_load_b16(rsc, lane * 2, 0, 0));
    const float s2 = h2f(__builtin_amdgcn_raw_buffer_load_b16(rsc, (lane ^ 1) * 2, 0, 0));
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
      for (int w = 0; w < 4; w++) {
        h1[8 * k + 2 * w] = dfk2_pair(c1[k][w], 0, s1);
        h1[8 * k + 2 * w + 1] = dfk2_pair(c1[k][w], 2, s1);
        h2[8 * k + 2 * w] = dfk2_pair(c2[k][w], 0, s2);
        h2[8 * k + 2 * w + 1] = dfk2_pair(c2[k][w], 2, s2);
      }
  } else {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint4*>(in + (long)b0 * 16), 0, nb * 256, kBufferRsrcWord3);
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const u4_t v = __builtin_amdgcn_raw_buffer_load_b128(rs, lane * 256, 16 * k, 0);
      h1[4 * k] = v.x;
      h1[4 * k + 1] = v.y;
      h1[4 * k + 2] = v.z;
      h1[4 * k + 3] = v.w;
    }
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const u4_t v = __builtin_amdgcn_raw_buffer_load_b128(rs, (lane ^ 1) * 256 + 128, 16 * k, 0);
      h2[4 * k] = v.x;
      h2[4 * k + 1] = v.y;
      h2[4 * k + 2] = v.z;
      h2[4 * k + 3] = v.w;
    }
  }
}

// Stage 64 of the WHT for elements k0 .. k0+7 of a block whose first half is
// a (this lane) and second half b (the other lane of the pair, read through
// DPP quad_perm [1,0,3,2]): lo = a + b, hi = a - b, the reference's two
// roundings.  A DPP read of a VGPR needs two wait states after the VALU write
// of that VGPR: the s_nop provides them, and nothing inside the block writes
// a register that a later instruction of it reads through DPP.
__device__ __forceinline__ void pair_stage8(const float (&a)[64], const float (&b)[64],
                                            float (&lo)[64], float (&hi)[64], int k0) {
  asm volatile(
      "s_nop 1\n\t"
      "v_add_f32_dpp %0, %16, %24 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
      "v_subrev_f32_dpp %8, %16, %24 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
      "v_add_f32_dpp %1, %17, %25 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
      "v_subrev_f32_dpp %9, %17, %25 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
      "v_add_f32_dpp %2, %18, %26 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
      "v_subrev_f32_dpp %10, %18, %26 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
      "v_add_f32_dpp %3, %19, %27 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
      "v_subrev_f32_dpp %11, %19, %27 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
      "v_add_f32_dpp %4, %20, %28 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
      "v_subrev_f32_dpp %12, %20, %28 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
      "v_add_f32_dpp %5, %21, %29 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
      "v_subrev_f32_dpp %13, %21, %29 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
      "v_add_f32_dpp %6, %22, %30 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
      "v_subrev_f32_dpp %14, %22, %30 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
      "v_add_f32_dpp %7, %23, %31 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
      "v_subrev_f32_dpp %15, %23, %31 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf"
      : "=&v"(lo[k0]), "=&v"(lo[k0 + 1]), "=&v"(lo[k0 + 2]), "=&v"(lo[k0 + 3]), "=&v"(lo[k0 + 4]),
        "=&v"(lo[k0 + 5]), "=&v"(lo[k0 + 6]), "=&v"(lo[k0 + 7]), "=&v"(hi[k0]), "=&v"(hi[k0 + 1]),
        "=&v"(hi[k0 + 2]), "=&v"(hi[k0 + 3]), "=&v"(hi[k0 + 4]), "=&v"(hi[k0 + 5]), "=&v"(hi[k0 + 6]),
        "=&v"(hi[k0 + 7])
      : "v"(b[k0]), "v"(b[k0 + 1]), "v"(b[k0 + 2]), "v"(b[k0 + 3]), "v"(b[k0 + 4]), "v"(b[k0 + 5]),
        "v"(b[k0 + 6]), "v"(b[k0 + 7]), "v"(a[k0]), "v"(a[k0 + 1]), "v"(a[k0 + 2]), "v"(a[k0 + 3]),
        "v"(a[k0 + 4]), "v"(a[k0 + 5]), "v"(a[k0 + 6]), "v"(a[k0 + 7]));
}

// Codes of 64 consecutive transformed elements (one half of a block) go to
// the 6 words of that half's 192-bit stream in two chains, k = 63..32 (words
// 3..5) and k = 31..0 (words 0..2); bin_steps runs chain steps I0 .. I0+N-1
// (elements 63-i and 31-i), so that each group of outputs is binned as soon
// as it exists, and the sign fix follows the last step.
template <int I0, int N>
__device__ __forceinline__ void bin_steps(const float (&x)[64], const uint32_t (&q)[3],
                                          uint32_t (&acc)[6]) {
#pragma unroll
  for (int i = I0; i < I0 + N; i++) {
    const int ka = 63 - i, kb = 31 - i;
    const float ya = __builtin_fmaf(x[ka], -kFoldA, __builtin_fabsf(x[ka]));
    const float yb = __builtin_fmaf(x[kb], -kFoldA, __builtin_fabsf(x[kb]));
    uint64_t pa[2], pb[2];
    fold_planes2(ya, yb, q, pa, pb);
    shift_in_sign(acc[(3 * ka + 2) >> 5], ya);
    shift_in_sign(acc[(3 * kb + 2) >> 5], yb);
    shift_in(acc[(3 * ka + 1) >> 5], pa[0]);
    shift_in(acc[(3 * kb + 1) >> 5], pb[0]);
    shift_in(acc[(3 * ka) >> 5], pa[1]);
    shift_in(acc[(3 * kb) >> 5], pb[1]);
  }
}

template <bool kDfk2, bool kPaged>
__global__ __launch_bounds__(kAp4Threads, 3) void tq3_append4_kernel(
    const uint4* __restrict__ in0, uint32_t* __restrict__ out0, const uint4* __restrict__ in1,
    uint32_t* __restrict__ out1, int n_blocks, int n_tensors, PagedRows pr,
    const uint16_t* __restrict__ sc0, const uint16_t* __restrict__ sc1) {
  __shared__ uint32_t lds[kAp4Waves * kAp4WaveLdsDw];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  uint32_t* wl = lds + wave * kAp4WaveLdsDw;
  // 32-bit tile bookkeeping (n_blocks < 2^31, so tiles * n_tensors < 2^27).
  // Work item t is tile t % tiles of tensor t / tiles; the wave's items are
  // t0, t0 + stride, ...: the tile and tensor advance without a division.
  const int tiles = (n_blocks + kAp4Tile - 1) / kAp4Tile;
  const int total = tiles * n_tensors;
  const int stride = (int)gridDim.x * kAp4Waves;
  int t = (int)blockIdx.x * kAp4Waves + wave;
  if (t >= total) return;
  int tile = t, tensor = 0;
  while (tile >= tiles) { tile -= tiles; tensor++; }
  const int s_tiles = stride % tiles, s_tensors = stride / tiles;   // scalar, once

  uint32_t q[3];
#pragma unroll
  for (int k = 0; k < 3; k++) q[k] = __builtin_amdgcn_readfirstlane(kFoldQBits[k]);

  for (;;) {
    uint32_t* __restrict__ out = tensor ? out1 : out0;
    const int b0 = tile * kAp4Tile;
    const int nb = min(kAp4Tile, n_blocks - b0);
    int tile_n = tile + s_tiles, tensor_n = tensor + s_tensors;
    if (tile_n >= tiles) { tile_n -= tiles; tensor_n++; }
    const bool more = tensor_n < n_tensors;

    // DFK2 and paged tiles: the per-lane offsets and the paged divisors are
    // re-formed every tile (a few instructions) instead of living in
    // registers across the loop, where the tile leaves no room for them.
    // DFK2 and paged tiles form the lane index where they use it (for the
    // loads here, again for the stores), not from a register held across
    // the tile
    const int lane_t = (kDfk2 || kPaged) ? opaque_lane() : lane;
    // R1 = first half of block `lane`, R2 = second half of block lane ^ 1
    uint32_t h1[32], h2[32];
    load_halves<kDfk2>(h1, h2, tensor ? in1 : in0, tensor ? sc1 : sc0, b0, nb, lane_t);
    // norm (reference order): block lane's chain over R1 here, handed to the
    // other lane of the pair, which continues over its R2
    float n1 = 0.0f;
#pragma unroll
    for (int k = 0; k < 32; k++) {
      const float lo = h2f(h1[k] & 0xffffu), hi = h2f(h1[k] >> 16);
      n1 = __builtin_fmaf(lo, lo, n1);
      n1 = __builtin_fmaf(hi, hi, n1);
    }
    float n2 = lane_dpp<0xB1>(n1);   // quad_perm [1,0,3,2]: block lane ^ 1's first-half partial
#pragma unroll
    for (int k = 0; k < 32; k++) {
      const float lo = h2f(h2[k] & 0xffffu), hi = h2f(h2[k] >> 16);
      n2 = __builtin_fmaf(lo, lo, n2);
      n2 = __builtin_fmaf(hi, hi, n2);
    }
    const float norm2 = __builtin_sqrtf(n2);   // block lane ^ 1
    const float inv2 = 1.0f / norm2;
    const float norm1 = lane_dpp<0xB1>(norm2);   // block lane
    const float inv1 = lane_dpp<0xB1>(inv2);
    // x * inv * sign (turboquant.cuh:141-149; the sign multiply is exact, so
    // it folds into the factor)
    float x1[64], x2[64];
#pragma unroll
    for (int e = 0; e < 64; e++) {
      x1[e] = __builtin_fmaf(h2f((e & 1) ? h1[e >> 1] >> 16 : h1[e >> 1] & 0xffffu),
                             sign_pos(e) ? inv1 : -inv1, 0.0f);
      x2[e] = __builtin_fmaf(h2f((e & 1) ? h2[e >> 1] >> 16 : h2[e >> 1] & 0xffffu),
                             sign_pos(64 + e) ? inv2 : -inv2, 0.0f);
    }
    // WHT stages 1 .. 32 (turboquant.cuh:50-59) on each half, then stage 64
    // across the pair
#pragma unroll
    for (int step = 1; step < 64; step <<= 1) {
#pragma unroll
      for (int i = 0; i < 64; i += 2 * step) {
#pragma unroll
        for (int j = i; j < i + step; j++) {
          const float a = x1[j], b = x1[j + step];
          x1[j] = a + b;
          x1[j + step] = a - b;
          const float c = x2[j], d = x2[j + step];
          x2[j] = c + d;
          x2[j + step] = c - d;
        }
      }
    }
    // stage 64 and the bins of block `lane`, eight chain steps at a time (a
    // group's outputs are binned as soon as they exist, which keeps the live
    // outputs to 32): words 0..5 from outputs 0..63, 6..11 from 64..127
    float y1[64], y2[64];
    uint32_t acc[12];
    {
      uint32_t a0[6] = {0u, 0u, 0u, 0u, 0u, 0u}, a1[6] = {0u, 0u, 0u, 0u, 0u, 0u};
      pair_stage8(x1, x2, y1, y2, 56);
      pair_stage8(x1, x2, y1, y2, 24);
      bin_steps<0, 8>(y1, q, a0);
      bin_steps<0, 8>(y2, q, a1);
      pair_stage8(x1, x2, y1, y2, 48);
      pair_stage8(x1, x2, y1, y2, 16);
      bin_steps<8, 8>(y1, q, a0);
      bin_steps<8, 8>(y2, q, a1);
      pair_stage8(x1, x2, y1, y2, 40);
      pair_stage8(x1, x2, y1, y2, 8);
      bin_steps<16, 8>(y1, q, a0);
      bin_steps<16, 8>(y2, q, a1);
      pair_stage8(x1, x2, y1, y2, 32);
      pair_stage8(x1, x2, y1, y2, 0);
      bin_steps<24, 8>(y1, q, a0);
      bin_steps<24, 8>(y2, q, a1);
      sign_fix<0, 3>(a0);
      sign_fix<3, 3>(a0 + 3);
      sign_fix<0, 3>(a1);
      sign_fix<3, 3>(a1 + 3);
      const bool keep = norm1 >= 1e-10f && norm1 < __builtin_inff();
#pragma unroll
      for (int w = 0; w < 6; w++) {
        acc[w] = keep ? a0[w] : 0u;
        acc[6 + w] = keep ? a1[w] : 0u;
      }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
    const int lane_s = (kDfk2 || kPaged) ? opaque_lane() : lane;

    if constexpr (kPaged) {
      // paged: each lane stores its block at the block's row
      PagedRows prt = pr;
      asm volatile("" : "+s"(prt.block_tokens), "+s"(prt.blocks_per_row), "+s"(prt.n_tok));
      if (lane_s < nb) {
        const long ob = paged_block(prt, (long)b0 + lane_s);
        if (ob >= 0) {
          uint32_t* dst = out + ob * 13;
          dst[0] = __float_as_uint(norm1);
#pragma unroll
          for (int w = 0; w < 12; w++) dst[1 + w] = acc[w];
        }
      }
    } else {
      // 4. stage the tile's 64 x 13 dwords, then store them contiguously
      uint32_t* ob = wl + lane_s * 13;
      ob[0] = __float_as_uint(norm1);
#pragma unroll
      for (int w = 0; w < 12; w++) ob[1 + w] = acc[w];
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
      // the resource spans the tile's nb * 52 bytes: stores past it are dropped
      const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc(
          out + (long)b0 * 13, 0, nb * 52, kBufferRsrcWord3);
#pragma unroll
      for (int j = 0; j < 13; j++)
        __builtin_amdgcn_raw_buffer_store_b32(wl[j * 64 + lane_s], rd, lane_s * 4, j * 256, 0);
    }
    if (!more) break;
    tile = tile_n;
    tensor = tensor_n;
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
  }
}

// ---------------------------------------------------------------------------
// Append of a few blocks (a decode step's new tokens): latency first.
//
// The lane-pair kernel gives each lane 128 elements, so a small append is one
// wave running ~2,000 dependent instructions.  Here a block is spread over a
// 16-lane DPP row, lane t holding elements 8t..8t+7 (one 16-byte load), and
// encoded by tq3_encode_row16 (tq3_encode.h): the norm's sequential sum runs
// through the row, the WHT's last four stages across it, and lanes 0..11
// gather the 12 code dwords, lane 12 storing the norm.
// Four blocks per wave, sixteen per workgroup; no persistent loop.
// ---------------------------------------------------------------------------
constexpr int kSmallThreads = 256;
// At most this many blocks (all tensors) take this kernel: measured K+V
// appends of n tokens (16 blocks each), small / lane-pair kernel: 1 token
// 2.6 / 6.6 us, 256 tokens 3.8 / 9.0, 1024 tokens 6.3 / 9.1, 2048 tokens
// 10.2 / 9.2.
constexpr long kSmallAppendBlocks = 16384;
constexpr int kSmallBlocksPerWg = kSmallThreads / 16;

template <bool kPaged>
__global__ __launch_bounds__(kSmallThreads) void tq3_append_small_kernel(
    const uint4* __restrict__ in0, uint32_t* __restrict__ out0, const uint4* __restrict__ in1,
    uint32_t* __restrict__ out1, int n_blocks, int n_tensors, PagedRows pr) {
  const int lane = threadIdx.x & 63;
  const int t = lane & 15;
  const long item = (long)blockIdx.x * kSmallBlocksPerWg + (threadIdx.x >> 4);
  const bool valid = item < (long)n_blocks * n_tensors;
  const int tensor = valid && item >= n_blocks ? 1 : 0;
  const long b = item - (long)tensor * n_blocks;
  const uint4* __restrict__ in = tensor ? in1 : in0;
  uint32_t* __restrict__ out = tensor ? out1 : out0;

  uint4 raw = make_uint4(0u, 0u, 0u, 0u);
  if (valid) raw = in[b * 16 + t];
  const uint32_t word = tq3_encode_row16(raw, lane);
  if (!valid || t > 12) return;
  long ob = b;
  if constexpr (kPaged) ob = paged_block(pr, b);
  if (ob < 0) return;
  uint32_t* dst = out + ob * 13;
  dst[t == 12 ? 0 : 1 + t] = word;
}

// ---------------------------------------------------------------------------
// Dequant (turboquant.cuh:169-200): half(((H*c)*rs)*sign*norm)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kCodecThreads) void tq3_dequant_kernel(
    const uint32_t* __restrict__ in, uint4* __restrict__ out, int n_blocks) {
  __shared__ uint32_t lds[kCodecWaves * kWaveLdsDw];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  uint32_t* wl = lds + wave * kWaveLdsDw;
  const long b0 = ((long)blockIdx.x * kCodecWaves + wave) * 64;
  if (b0 >= n_blocks) return;
  const int nb = (int)min<long>(64, n_blocks - b0);

  // 1. coalesced dword loads of 64 x 13 dwords into LDS
  const uint32_t* src = in + b0 * 13;
  const int n_dw = nb * 13;
#pragma unroll
  for (int j = 0; j < 13; j++) {
    const int idx = j * 64 + lane;
    if (idx < n_dw) wl[idx] = src[idx];
  }
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");

  uint32_t hw[64];
  if (lane < nb) {
    uint32_t w[13];
#pragma unroll
    for (int k = 0; k < 13; k++) w[k] = wl[lane * 13 + k];
    const float norm = __uint_as_float(w[0]);
    float x[128];
#pragma unroll
    for (int e = 0; e < 128; e++) {
      const int bit = 3 * e;
      const int q = bit >> 5, sh = bit & 31;
      uint32_t c = w[1 + q] >> sh;
      if (sh > 29) c |= w[2 + q] << (32 - sh);
      x[e] = kCentroids[c & 7u];
    }
    wht128_butterflies(x);
    const float rs = wht_scale();
#pragma unroll
    for (int k = 0; k < 64; k++) {
      float a = x[2 * k] * rs, b = x[2 * k + 1] * rs;
      a = sign_pos(2 * k) ? a : -a;
      b = sign_pos(2 * k + 1) ? b : -b;
      // The reference rounds v*norm to fp32 and then to fp16.  The empty asm
      // keeps the fp32 product, so the compiler cannot fuse multiply and
      // conversion into one fp16-rounding mixed FMA.
      float pa = a * norm, pb = b * norm;
      asm volatile("" : "+v"(pa), "+v"(pb));
      hw[k] = f2h(pa) | (f2h(pb) << 16);
    }
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
  if (lane < nb) {
#pragma unroll
    for (int k = 0; k < 16; k++)
      *reinterpret_cast<uint4*>(wl + lane * kInPitchDw + 4 * k) =
          make_uint4(hw[4 * k], hw[4 * k + 1], hw[4 * k + 2], hw[4 * k + 3]);
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
#pragma unroll
  for (int j = 0; j < 16; j++) {
    const int chunk = j * 64 + lane;
    const int blk = chunk >> 4, part = chunk & 15;
    if (blk < nb) out[(b0 + blk) * 16 + part] = *reinterpret_cast<const uint4*>(wl + blk * kInPitchDw + part * 4);
  }
}

// ---------------------------------------------------------------------------
// host launchers (validated by the C ABI layer)
// ---------------------------------------------------------------------------
hipError_t launch_tq3_append(const void* in0, void* out0, const void* in1, void* out1,
                             int n_blocks, int n_tensors, hipStream_t stream,
                             const PagedRows* paged, const uint16_t* sc0, const uint16_t* sc1) {
  // Persistent grid: three workgroups (12 waves) per CU, fewer when the work
  // list is shorter.
  static std::atomic<int> cus[64];
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return err;
  if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
  int n_cu = cus[dev].load(std::memory_order_relaxed);
  if (n_cu == 0) {
    err = hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev);
    if (err != hipSuccess) return err;
    n_cu = n_cu > 0 ? n_cu : 1;
    cus[dev].store(n_cu, std::memory_order_relaxed);
  }
  const PagedRows pr = paged ? *paged : PagedRows{};
  const long items = (long)n_blocks * n_tensors;
  if (sc0 == nullptr && items > 0 && items <= kSmallAppendBlocks) {
    const int grid = (int)((items + kSmallBlocksPerWg - 1) / kSmallBlocksPerWg);
    auto kernel = paged ? tq3_append_small_kernel<true> : tq3_append_small_kernel<false>;
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kSmallThreads), 0, stream, static_cast<const uint4*>(in0),
                       static_cast<uint32_t*>(out0), static_cast<const uint4*>(in1),
                       static_cast<uint32_t*>(out1), n_blocks, n_tensors, pr);
    return hipGetLastError();
  }
  const long tiles = ((long)n_blocks + kAp4Tile - 1) / kAp4Tile * n_tensors;
  const long wgs_needed = (tiles + kAp4Waves - 1) / kAp4Waves;
  const int grid = (int)std::min<long>(wgs_needed, 3L * n_cu);
  if (grid == 0) return hipSuccess;
  auto kernel = sc0 != nullptr ? (paged ? tq3_append4_kernel<true, true> : tq3_append4_kernel<true, false>)
                                : (paged ? tq3_append4_kernel<false, true> : tq3_append4_kernel<false, false>);
  hipLaunchKernelGGL(kernel, dim3(grid), dim3(kAp4Threads), 0, stream, static_cast<const uint4*>(in0),
                     static_cast<uint32_t*>(out0), static_cast<const uint4*>(in1),
                     static_cast<uint32_t*>(out1), n_blocks, n_tensors, pr, sc0, sc1);
  return hipGetLastError();
}

hipError_t launch_tq3_dequant(const void* in, void* out, int n_blocks, hipStream_t stream) {
  const int per_wg = 64 * kCodecWaves;
  dim3 grid((n_blocks + per_wg - 1) / per_wg);
  hipLaunchKernelGGL(tq3_dequant_kernel, grid, dim3(kCodecThreads), 0, stream,
                     static_cast<const uint32_t*>(in), static_cast<uint4*>(out), n_blocks);
  return hipGetLastError();
}

}  // namespace qkv
