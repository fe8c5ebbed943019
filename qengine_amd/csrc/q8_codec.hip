// q8_codec.hip -- Q8_0 KV append and dequant kernels for gfx950.
//
// Reference arithmetic: attention.cuh:2587-2609 (encode), 2614-2626 (decode).
// Layout: 4 lanes per 32-element block, 8 fp16 (one 16-byte load) per lane, so
// a wave covers 16 blocks with fully coalesced loads; the block absmax is a
// 2-step xor reduction inside each lane quad (DPP).  amax/127, 1/scale and
// v*inv are the same IEEE single-rounding operations as the reference, with
// round-half-even to int and the [-128,127] clamp; the fp16 scale is written
// with a 16-bit store so the `pad` field keeps whatever the cache held.
#include "qkv_device.h"

// Bit-exact codec: no FMA contraction across the reference's separate roundings.
#pragma clang fp contract(off)

namespace qkv {

constexpr int kQ8Threads = 256;

__device__ __forceinline__ float quad_max(float v) {
  v = fmaxf(v, __shfl_xor(v, 1));
  v = fmaxf(v, __shfl_xor(v, 2));
  return v;
}

__device__ __forceinline__ uint32_t q8_code(float v, float inv) {
  // __float2int_rn: round half to even; v_cvt_i32_f32 maps NaN to 0.
  int q = (int)__builtin_rintf(v * inv);
  q = q > 127 ? 127 : q;
  q = q < -128 ? -128 : q;
  return (uint32_t)q & 0xffu;
}

// gridDim.y selects (in, out) so K and V can share one launch.  kDfk2: the
// input is DFK2 int8 rows (8 bytes per 8-element group) with one fp16 scale
// per 128 elements (sc0/sc1), each element first dequantized as
// dfki2_dequant_kernel does (model.cuh:149-159): half(float(q) * float(s)).
template <bool kDfk2>
__global__ __launch_bounds__(kQ8Threads) void q8_append_kernel(
    const void* __restrict__ in0, uint8_t* __restrict__ out0, const void* __restrict__ in1,
    uint8_t* __restrict__ out1, int n_blocks, const uint16_t* __restrict__ sc0,
    const uint16_t* __restrict__ sc1) {
  uint8_t* __restrict__ out = blockIdx.y ? out1 : out0;
  const long g = (long)blockIdx.x * kQ8Threads + threadIdx.x;  // 8-element group
  const long blk = g >> 2;
  const int part = (int)(g & 3);
  const bool live = blk < n_blocks;
  float v[8];
  if constexpr (kDfk2) {
    const uint2* __restrict__ in = static_cast<const uint2*>(blockIdx.y ? in1 : in0);
    const uint16_t* __restrict__ sc = blockIdx.y ? sc1 : sc0;
    const uint2 w = live ? in[g] : make_uint2(0, 0);
    const float s = live ? h2f(sc[g >> 4]) : 0.0f;   // 16 groups of 8 per scale
    const uint32_t ww[2] = {w.x, w.y};
#pragma unroll
    for (int k = 0; k < 8; k++)
      v[k] = h2f(f2h((float)(int8_t)((ww[k >> 2] >> (8 * (k & 3))) & 0xffu) * s));
  } else {
    const uint4* __restrict__ in = static_cast<const uint4*>(blockIdx.y ? in1 : in0);
    const uint4 w = live ? in[g] : make_uint4(0, 0, 0, 0);
    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
      v[2 * k] = h2f(ww[k] & 0xffffu);
      v[2 * k + 1] = h2f(ww[k] >> 16);
    }
  }
  float amax = fabsf(v[0]);
#pragma unroll
  for (int i = 1; i < 8; i++) amax = fmaxf(amax, fabsf(v[i]));
  amax = quad_max(amax);
  const float scale = amax / 127.0f;
  const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) lo |= q8_code(v[i], inv) << (8 * i);
#pragma unroll
  for (int i = 0; i < 4; i++) hi |= q8_code(v[4 + i], inv) << (8 * i);
  if (live) {
    uint8_t* b = out + blk * kQ8BlockBytes;
    uint32_t* bw = reinterpret_cast<uint32_t*>(b + 8 * part);  // 36-byte blocks: 4-byte aligned
    bw[0] = lo;
    bw[1] = hi;
    if (part == 0) *reinterpret_cast<uint16_t*>(b + 34) = (uint16_t)f2h(scale);
  }
}

__global__ __launch_bounds__(kQ8Threads) void q8_dequant_kernel(const uint8_t* __restrict__ in,
                                                                uint4* __restrict__ out,
                                                                int n_blocks) {
  const long g = (long)blockIdx.x * kQ8Threads + threadIdx.x;
  const long blk = g >> 2;
  const int part = (int)(g & 3);
  if (blk >= n_blocks) return;
  const uint8_t* b = in + blk * kQ8BlockBytes;
  const uint32_t* bw = reinterpret_cast<const uint32_t*>(b + 8 * part);
  const uint2 q = make_uint2(bw[0], bw[1]);
  const float s = h2f(*reinterpret_cast<const uint16_t*>(b + 34));
  uint32_t o[4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const uint32_t word = k < 2 ? q.x : q.y;
    const int sh = 16 * (k & 1);
    const float a = (float)(int8_t)((word >> sh) & 0xffu);
    const float c = (float)(int8_t)((word >> (sh + 8)) & 0xffu);
    o[k] = f2h(a * s) | (f2h(c * s) << 16);
  }
  out[g] = make_uint4(o[0], o[1], o[2], o[3]);
}

hipError_t launch_q8_append(const void* in0, void* out0, const void* in1, void* out1,
                            int n_blocks, int n_tensors, hipStream_t stream,
                            const uint16_t* sc0, const uint16_t* sc1) {
  const long groups = (long)n_blocks * 4;
  dim3 grid((unsigned)((groups + kQ8Threads - 1) / kQ8Threads), n_tensors);
  if (sc0 != nullptr)
    hipLaunchKernelGGL(q8_append_kernel<true>, grid, dim3(kQ8Threads), 0, stream, in0,
                       static_cast<uint8_t*>(out0), in1, static_cast<uint8_t*>(out1), n_blocks,
                       sc0, sc1);
  else
    hipLaunchKernelGGL(q8_append_kernel<false>, grid, dim3(kQ8Threads), 0, stream, in0,
                       static_cast<uint8_t*>(out0), in1, static_cast<uint8_t*>(out1), n_blocks,
                       nullptr, nullptr);
  return hipGetLastError();
}

// dfki2_dequant_kernel (model.cuh:149-159): 8 elements per thread.
__global__ __launch_bounds__(kQ8Threads) void dfk2_dequant_kernel(
    const uint2* __restrict__ q, const uint16_t* __restrict__ sc, uint4* __restrict__ out,
    long n_groups) {
  const long g = (long)blockIdx.x * kQ8Threads + threadIdx.x;
  if (g >= n_groups) return;
  const uint2 w = q[g];
  const float s = h2f(sc[g >> 4]);
  const uint32_t ww[2] = {w.x, w.y};
  uint32_t o[4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const uint32_t word = ww[k >> 1];
    const int sh = 16 * (k & 1);
    o[k] = f2h((float)(int8_t)((word >> sh) & 0xffu) * s) |
           (f2h((float)(int8_t)((word >> (sh + 8)) & 0xffu) * s) << 16);
  }
  out[g] = make_uint4(o[0], o[1], o[2], o[3]);
}

hipError_t launch_dfk2_dequant(const void* q, const uint16_t* sc, void* out, long n_elems,
                               hipStream_t stream) {
  const long groups = n_elems / 8;
  if (groups == 0) return hipSuccess;
  hipLaunchKernelGGL(dfk2_dequant_kernel, dim3((unsigned)((groups + kQ8Threads - 1) / kQ8Threads)),
                     dim3(kQ8Threads), 0, stream, static_cast<const uint2*>(q), sc,
                     static_cast<uint4*>(out), groups);
  return hipGetLastError();
}

hipError_t launch_q8_dequant(const void* in, void* out, int n_blocks, hipStream_t stream) {
  const long groups = (long)n_blocks * 4;
  dim3 grid((unsigned)((groups + kQ8Threads - 1) / kQ8Threads));
  hipLaunchKernelGGL(q8_dequant_kernel, grid, dim3(kQ8Threads), 0, stream,
                     static_cast<const uint8_t*>(in), static_cast<uint4*>(out), n_blocks);
  return hipGetLastError();
}

}  // namespace qkv
