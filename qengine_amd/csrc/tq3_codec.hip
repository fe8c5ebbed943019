// tq3_codec.hip -- TQ3 append (encode) and dequant kernels for gfx950.
//
// Reference arithmetic: turboquant.cuh:112-165 (encode) and 169-200 (decode).
//
// Layout on the GPU: one lane owns one 128-element block.  Waves are
// persistent: each takes 64-block tiles (16 KiB of fp16) in turn, with the
// coalesced 16-byte buffer loads of its next tile in flight into registers
// while it encodes the current one.  A tile passes through LDS at a 272-byte
// pitch (bank-conflict-free 16-byte reads per lane); each lane then runs the
// reference's sequential norm, unit scaling, random signs and 7-stage
// butterfly WHT in registers, bins the result against thresholds that fold
// the final x rs scaling in exactly, and the wave writes its 64 x 52-byte
// output through an LDS staging area with dword stores that cover whole cache
// lines.  Every float operation that feeds a code or a norm is the same
// single-rounding IEEE operation in the same order as the reference, so codes
// and norms are bit-identical.
#include <algorithm>
#include <atomic>

#include "qkv_device.h"
#include "qkv_launch.h"

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

// Encode one block held as 64 dwords of packed fp16 (element 2k in the low
// half of hw[k]).  Writes the 13 output dwords (norm, qs[0..47]) to o[].
//
// Instruction budget per element: one v_fma_mix for the norm, one for the
// scaling (fp16 operand converted inside the instruction), seven butterfly
// add/subs, one FMA that folds the sign, three compares into scalar lane
// masks and three shifts into the packed words (the sign bit directly, two
// mask bits), plus about 0.4 for the sign fix of the packed words.  Bit 0 of
// the code is formed from the compare masks on the scalar unit, which runs
// beside the vector ALU.
__device__ __forceinline__ void tq3_encode_block(const uint32_t (&hw)[64], uint32_t (&o)[13]) {
  // Sequential sum of squares in reference order (x^2 of an fp16 value is
  // exact in fp32, so an FMA gives the same result as mul+add).
  float nsq = 0.0f;
#pragma unroll
  for (int k = 0; k < 64; k++) {
    float lo = h2f(hw[k] & 0xffffu), hi = h2f(hw[k] >> 16);
    nsq = __builtin_fmaf(lo, lo, nsq);
    nsq = __builtin_fmaf(hi, hi, nsq);
  }
  const float norm = __builtin_sqrtf(nsq);
  const float inv = 1.0f / norm;
  float x[128];
#pragma unroll
  for (int k = 0; k < 64; k++) {
    // x * inv then * sign: the sign multiply is exact, so it folds into the
    // factor.  The +0 addend only changes the sign of an exact zero, which no
    // later sum or bin comparison can observe.
    x[2 * k] = __builtin_fmaf(h2f(hw[k] & 0xffffu), sign_pos(2 * k) ? inv : -inv, 0.0f);
    x[2 * k + 1] = __builtin_fmaf(h2f(hw[k] >> 16), sign_pos(2 * k + 1) ? inv : -inv, 0.0f);
  }
  wht128_butterflies(x);

  // Bins (sign-folded form, kFoldQBits): y = fma(w, -A, |w|), bit 2 = sign
  // bit of y, bits 1..0 from three compares of |y|.  Bit 3e+b of the 384-bit
  // code stream is bit b of element e; the words are filled by shifting bits
  // in from the top, highest element first, in two independent chains
  // (elements 127..64 fill words 11..6, elements 63..0 words 5..0) so that no
  // shift waits on the one before it.
  uint32_t acc[12];
#pragma unroll
  for (int w = 0; w < 12; w++) acc[w] = 0u;
  uint32_t q[3];
#pragma unroll
  for (int k = 0; k < 3; k++) q[k] = __builtin_amdgcn_readfirstlane(kFoldQBits[k]);
  const float neg_a = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(
                                                    __builtin_bit_cast(uint32_t, -kFoldA)));
#pragma unroll
  for (int i = 0; i < 64; i++) {
    const int ea = 127 - i, eb = 63 - i;
    const float ya = __builtin_fmaf(x[ea], neg_a, __builtin_fabsf(x[ea]));
    const float yb = __builtin_fmaf(x[eb], neg_a, __builtin_fabsf(x[eb]));
    uint64_t pa[2], pb[2];
    fold_planes2(ya, yb, q, pa, pb);
    shift_in_sign(acc[(3 * ea + 2) >> 5], ya);
    shift_in_sign(acc[(3 * eb + 2) >> 5], yb);
    shift_in(acc[(3 * ea + 1) >> 5], pa[0]);
    shift_in(acc[(3 * eb + 1) >> 5], pb[0]);
    shift_in(acc[(3 * ea) >> 5], pa[1]);
    shift_in(acc[(3 * eb) >> 5], pb[1]);
  }
  sign_fix<0, 6>(acc);
  sign_fix<6, 6>(acc + 6);
  // zero block (turboquant.cuh:133-140): norm stored, codes zero.  A block
  // with a non-finite norm (an inf or NaN element) has NaN WHT outputs, which
  // the reference bins to 0: its codes are zero as well.
  const bool keep = norm >= 1e-10f && norm < __builtin_inff();
  o[0] = __float_as_uint(norm);
#pragma unroll
  for (int w = 0; w < 12; w++) o[1 + w] = keep ? acc[w] : 0u;
}

// Output block of input block i for a paged append (PagedRows), or -1 when
// the row it maps to lies outside the pool (then nothing is written).
__device__ __forceinline__ long paged_block(const PagedRows& pr, long i) {
  const long tok = i / pr.blocks_per_row;
  const int j = (int)(i - tok * pr.blocks_per_row);
  const int s = (int)(tok / pr.n_tok), t = (int)(tok - (long)s * pr.n_tok);
  const long pos = (long)pr.positions[s] + t;
  if (pos < 0) return -1;
  const long b = pos / pr.block_tokens;
  if (b >= pr.max_blocks) return -1;
  const long row = (long)pr.block_tables[(long)s * pr.max_blocks + b] * pr.block_tokens +
                   (pos - b * pr.block_tokens);
  if (row < 0 || row >= pr.pool_rows) return -1;
  return row * pr.blocks_per_row + j;
}

// Issue the 16 coalesced 16-byte loads of one 64-block tile (blocks b0..b0+nb-1
// of `in`); chunk j*64+lane is 16-byte piece (chunk & 15) of block (chunk >> 4).
// The buffer resource spans exactly the tile's nb blocks, so chunks past the
// last block read zero: the loads carry no branches or clamps.
__device__ __forceinline__ void load_tile(uint32_t (&pre)[64], const uint4* __restrict__ in,
                                          long b0, int nb, int lane) {
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint4*>(in + b0 * 16), 0, nb * 256, kBufferRsrcWord3);
#pragma unroll
  for (int j = 0; j < 16; j++) {
    const u4_t v = __builtin_amdgcn_raw_buffer_load_b128(rs, lane * 16, j * 1024, 0);
    pre[4 * j] = v.x;
    pre[4 * j + 1] = v.y;
    pre[4 * j + 2] = v.z;
    pre[4 * j + 3] = v.w;
  }
}

// in: n_blocks*128 fp16 as uint4 (16 B aligned); out: n_blocks*13 dwords,
// or, when pr.block_tables is set, each block at its paged_block position.
// n_tensors (1 or 2) (in, out) pairs share one launch (K and V).
//
// Persistent waves: tile t (64 blocks) of the n_tensors * tiles work list is
// taken by wave t mod (total waves).  While a wave encodes one tile, the
// loads of its next tile are in flight into registers, so each wave overlaps
// its own HBM latency with its vector work.
__global__ __launch_bounds__(kCodecThreads, 2) void tq3_append_kernel(
    const uint4* __restrict__ in0, uint32_t* __restrict__ out0, const uint4* __restrict__ in1,
    uint32_t* __restrict__ out1, int n_blocks, int n_tensors, PagedRows pr) {
  __shared__ uint32_t lds[kCodecWaves * kWaveLdsDw];
  const int lane = threadIdx.x & 63;
  // wave-uniform: keeps the tile bookkeeping on the scalar unit
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  uint32_t* wl = lds + wave * kWaveLdsDw;
  const long tiles = ((long)n_blocks + 63) / 64;
  const long total = tiles * n_tensors;
  const long stride = (long)gridDim.x * kCodecWaves;
  long t = (long)blockIdx.x * kCodecWaves + wave;
  if (t >= total) return;  // whole wave idle

  uint32_t pre[64];
  {
    const long b0 = (t % tiles) * 64;
    load_tile(pre, t < tiles ? in0 : in1, b0, (int)min<long>(64, n_blocks - b0), lane);
  }
  for (;;) {
    const bool second = t >= tiles;
    uint32_t* __restrict__ out = second ? out1 : out0;
    const long b0 = (t % tiles) * 64;
    const int nb = (int)min<long>(64, n_blocks - b0);

    // 1. the prefetched tile into LDS (272-byte pitch: conflict-free reads;
    //    pieces of blocks past nb are zeros and are never read)
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const int chunk = j * 64 + lane;
      const int blk = chunk >> 4, part = chunk & 15;
      *reinterpret_cast<uint4*>(wl + blk * kInPitchDw + part * 4) =
          make_uint4(pre[4 * j], pre[4 * j + 1], pre[4 * j + 2], pre[4 * j + 3]);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");

    // 2. next tile's loads go out before this tile's vector work
    const long tn = t + stride;
    if (tn < total) {
      const long nb0 = (tn % tiles) * 64;
      load_tile(pre, tn < tiles ? in0 : in1, nb0, (int)min<long>(64, n_blocks - nb0), lane);
    }

    // 3. one lane per block
    uint32_t o[13];
    if (lane < nb) {
      uint32_t hw[64];
#pragma unroll
      for (int k = 0; k < 16; k++) {
        uint4 v = *reinterpret_cast<const uint4*>(wl + lane * kInPitchDw + 4 * k);
        hw[4 * k] = v.x;
        hw[4 * k + 1] = v.y;
        hw[4 * k + 2] = v.z;
        hw[4 * k + 3] = v.w;
      }
      tq3_encode_block(hw, o);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");

    if (pr.block_tables != nullptr) {
      // paged: each lane stores its block at its own row
      if (lane < nb) {
        const long ob = paged_block(pr, b0 + lane);
        if (ob >= 0) {
          uint32_t* dst = out + ob * 13;
#pragma unroll
          for (int k = 0; k < 13; k++) dst[k] = o[k];
        }
      }
    } else {
      // 4. stage 13 dwords per lane (odd pitch: conflict-free), then store the
      //    wave's contiguous 64*52 bytes with dword stores.
      if (lane < nb) {
#pragma unroll
        for (int k = 0; k < 13; k++) wl[lane * 13 + k] = o[k];
      }
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
      // the resource spans the tile's nb * 52 bytes: stores past it are dropped
      const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc(
          out + b0 * 13, 0, nb * 52, kBufferRsrcWord3);
#pragma unroll
      for (int j = 0; j < 13; j++)
        __builtin_amdgcn_raw_buffer_store_b32(wl[j * 64 + lane], rd, lane * 4, j * 256, 0);
    }
    if (tn >= total) break;
    t = tn;
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
  }
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
                             const PagedRows* paged) {
  // Persistent grid: two workgroups (8 waves) per CU, fewer when the work
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
  const long tiles = ((long)n_blocks + 63) / 64 * n_tensors;
  const long wgs_needed = (tiles + kCodecWaves - 1) / kCodecWaves;
  const int grid = (int)std::min<long>(wgs_needed, 2L * n_cu);
  if (grid == 0) return hipSuccess;
  const PagedRows pr = paged ? *paged : PagedRows{};
  hipLaunchKernelGGL(tq3_append_kernel, dim3(grid), dim3(kCodecThreads), 0, stream,
                     static_cast<const uint4*>(in0), static_cast<uint32_t*>(out0),
                     static_cast<const uint4*>(in1), static_cast<uint32_t*>(out1), n_blocks,
                     n_tensors, pr);
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
