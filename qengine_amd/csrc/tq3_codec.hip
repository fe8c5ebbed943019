// tq3_codec.hip -- TQ3 append (encode) and dequant kernels for gfx950.
//
// Reference arithmetic: turboquant.cuh:112-165 (encode) and 169-200 (decode).
//
// Layout on the GPU: one lane owns one 128-element block.  A wave stages its
// 64 input blocks (16 KiB of fp16) from HBM with coalesced 16-byte loads into
// LDS at a 272-byte pitch (bank-conflict-free 16-byte reads per lane), each
// lane then runs the reference's sequential norm, unit scaling, random signs,
// 7-stage butterfly WHT and 7-bound bin search in registers, and the wave
// writes its 64 x 52-byte output through an LDS staging area with dword
// stores that cover whole cache lines.  Every float operation is the same
// single-rounding IEEE operation in the same order as the reference, so
// codes and norms are bit-identical.
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

// Encode one block held as 64 dwords of packed fp16 (element 2k in the low
// half of hw[k]).  Writes the 13 output dwords (norm, qs[0..47]) to o[].
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
  o[0] = __float_as_uint(norm);
#pragma unroll
  for (int k = 1; k < 13; k++) o[k] = 0u;
  if (norm < 1e-10f) return;  // zero block: norm stored, codes zero

  const float inv = 1.0f / norm;
  float x[128];
#pragma unroll
  for (int k = 0; k < 64; k++) {
    // x * inv then * sign: the sign multiply is exact, so fold it into the factor.
    x[2 * k] = h2f(hw[k] & 0xffffu) * (sign_pos(2 * k) ? inv : -inv);
    x[2 * k + 1] = h2f(hw[k] >> 16) * (sign_pos(2 * k + 1) ? inv : -inv);
  }
  wht128_butterflies(x);
  const float rs = wht_scale();
#pragma unroll
  for (int e = 0; e < 128; e++) {
    uint32_t c = tq3_bin(x[e] * rs);
    const int bit = 3 * e;
    const int w = bit >> 5, sh = bit & 31;
    o[1 + w] |= c << sh;
    if (sh > 29) o[2 + w] |= c >> (32 - sh);
  }
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

// in: n_blocks*128 fp16 as uint4 (16 B aligned); out: n_blocks*13 dwords,
// or, when pr.block_tables is set, each block at its paged_block position.
// gridDim.y selects the (in, out) pair so K and V can share one launch.
__global__ __launch_bounds__(kCodecThreads) void tq3_append_kernel(
    const uint4* __restrict__ in0, uint32_t* __restrict__ out0, const uint4* __restrict__ in1,
    uint32_t* __restrict__ out1, int n_blocks, PagedRows pr) {
  __shared__ uint32_t lds[kCodecWaves * kWaveLdsDw];
  const uint4* __restrict__ in = blockIdx.y ? in1 : in0;
  uint32_t* __restrict__ out = blockIdx.y ? out1 : out0;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  uint32_t* wl = lds + wave * kWaveLdsDw;
  const long b0 = ((long)blockIdx.x * kCodecWaves + wave) * 64;  // first block of this wave
  if (b0 >= n_blocks) return;                                     // whole wave idle
  const int nb = (int)min<long>(64, n_blocks - b0);

  // 1. coalesced 16-byte loads of the wave's blocks into LDS
#pragma unroll
  for (int j = 0; j < 16; j++) {
    const int chunk = j * 64 + lane;  // 16-byte chunk within the wave's 16 KiB
    const int blk = chunk >> 4, part = chunk & 15;
    if (blk < nb) {
      uint4 v = in[(b0 + blk) * 16 + part];
      *reinterpret_cast<uint4*>(wl + blk * kInPitchDw + part * 4) = v;
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");

  // 2. one lane per block
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

  // paged: each lane stores its block at its own row
  if (pr.block_tables != nullptr) {
    if (lane < nb) {
      const long ob = paged_block(pr, b0 + lane);
      if (ob >= 0) {
        uint32_t* dst = out + ob * 13;
#pragma unroll
        for (int k = 0; k < 13; k++) dst[k] = o[k];
      }
    }
    return;
  }
  // 3. stage 13 dwords per lane (odd pitch: conflict-free), then store the
  //    wave's contiguous 64*52 bytes with dword stores.
  if (lane < nb) {
#pragma unroll
    for (int k = 0; k < 13; k++) wl[lane * 13 + k] = o[k];
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
  const int n_dw = nb * 13;
  uint32_t* dst = out + b0 * 13;
#pragma unroll
  for (int j = 0; j < 13; j++) {
    const int idx = j * 64 + lane;
    if (idx < n_dw) dst[idx] = wl[idx];
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
  const int per_wg = 64 * kCodecWaves;
  dim3 grid((n_blocks + per_wg - 1) / per_wg, n_tensors);
  const PagedRows pr = paged ? *paged : PagedRows{};
  hipLaunchKernelGGL(tq3_append_kernel, grid, dim3(kCodecThreads), 0, stream,
                     static_cast<const uint4*>(in0), static_cast<uint32_t*>(out0),
                     static_cast<const uint4*>(in1), static_cast<uint32_t*>(out1), n_blocks, pr);
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
