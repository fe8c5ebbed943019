// read_bench.hip -- the streaming-read kernels behind bench.py's HBM read
// peak and single-launch read floor (libqkv_bench.so; not part of libqkv.so).
#include <hip/hip_runtime.h>

#include <algorithm>

#include "qkv_bench.h"

namespace qkv {
namespace {

// Streaming read of `bytes` (a multiple of 64): every 16-byte piece loaded
// once by a grid-stride loop; the xor of the data is written only if it
// equals a value no test buffer produces, so no store traffic is added and
// the loads cannot be elided.  The measurement the reference makes with its
// bandwidth tool (tools/bench_hbm_bandwidth.cu k_read_f4).
__global__ __launch_bounds__(256) void stream_read_kernel(const uint4* __restrict__ p, size_t n4,
                                                          uint32_t* __restrict__ sink) {
  const size_t stride = (size_t)gridDim.x * 256;
  uint32_t acc = 0u;
  for (size_t i = blockIdx.x * 256ul + threadIdx.x; i < n4; i += stride) {
    const uint4 a = p[i];
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  if (acc == 0x9E3779B9u) sink[0] = acc;
}

// Short reads (up to kShortRead bytes, e.g. one decode layer's cache): one
// 8 KB piece per workgroup, both loads of a thread issued before either is
// used, so the launch costs one memory round trip plus the transfer.
constexpr size_t kShortRead = 64ul << 20;
__global__ __launch_bounds__(256) void stream_read_short_kernel(const uint4* __restrict__ p, size_t n4,
                                                                uint32_t* __restrict__ sink) {
  const size_t i = blockIdx.x * 512ul + threadIdx.x;
  const uint4 a = i < n4 ? p[i] : make_uint4(0, 0, 0, 0);
  const uint4 b = i + 256 < n4 ? p[i + 256] : make_uint4(0, 0, 0, 0);
  const uint32_t acc = a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w;
  if (acc == 0x9E3779B9u) sink[0] = acc;
}

hipError_t launch_stream_read(const void* p, size_t bytes, uint32_t* sink, hipStream_t stream) {
  const size_t n4 = bytes / 16;
  if (bytes <= kShortRead) {
    hipLaunchKernelGGL(stream_read_short_kernel, dim3((unsigned)((n4 + 511) / 512)), dim3(256), 0, stream,
                       static_cast<const uint4*>(p), n4, sink);
    return hipGetLastError();
  }
  const unsigned blocks = (unsigned)std::min<size_t>((n4 + 255) / 256, 2048);
  hipLaunchKernelGGL(stream_read_kernel, dim3(blocks), dim3(256), 0, stream,
                     static_cast<const uint4*>(p), n4, sink);
  return hipGetLastError();
}

}  // namespace
}  // namespace qkv

extern "C" int qkv_hbm_read_bench(const void* buf, size_t bytes, uint32_t* sink, hipStream_t stream) {
  if (bytes == 0) return QKV_OK;
  if (bytes % 64) return QKV_ERR_INVALID;
  if (!buf || !sink) return QKV_ERR_NULL;
  if (reinterpret_cast<uintptr_t>(buf) % 16 || reinterpret_cast<uintptr_t>(sink) % 4) return QKV_ERR_ALIGN;
  return qkv::launch_stream_read(buf, bytes, sink, stream) == hipSuccess ? QKV_OK : QKV_ERR_LAUNCH;
}
