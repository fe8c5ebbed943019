// attn_merge.hip -- log-sum-exp merge of split partials (reference layout).
//
// Reference: flash_attn_split_merge (attention.cuh:1837-1891): M = max over
// splits; splits with non-finite m or l <= 0 are skipped; out = sum w*o /
// sum w*l with w = exp(m_s - M), 0 when the sum is 0; fp16 output
// [t][q_head][256].  One workgroup per (q head, t), one thread per dim.
#include <algorithm>

#include "attn_common.h"
#include "qkv_launch.h"
#include "qkv_device.h"

namespace qkv {

__global__ __launch_bounds__(256) void split_merge_kernel(const float* __restrict__ pm,
                                                          const float* __restrict__ pl,
                                                          const float* __restrict__ po,
                                                          uint16_t* __restrict__ out, int num_q,
                                                          int sub_n_max, int k_splits) {
  const int qh = blockIdx.x, t = blockIdx.y, d = threadIdx.x;
  const long base = ((long)qh * sub_n_max + t) * k_splits;
  float M = -INFINITY;
  for (int s = 0; s < k_splits; s++) M = fmaxf(M, pm[base + s]);
  float L = 0.f, o = 0.f;
  for (int s = 0; s < k_splits; s++) {
    const float ms = pm[base + s], ls = pl[base + s];
    if (!__builtin_isfinite(ms) || ls <= 0.0f) continue;
    const float w = __expf(ms - M);
    L += w * ls;
    o += w * po[(base + s) * 256 + d];
  }
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  out[((long)t * num_q + qh) * 256 + d] = (uint16_t)f2h(o * inv);
}

hipError_t launch_split_merge(const float* m, const float* l, const float* o, uint16_t* out,
                              int num_q, int sub_n, int sub_n_max, int k_splits,
                              hipStream_t stream) {
  dim3 grid(num_q, sub_n);
  hipLaunchKernelGGL(split_merge_kernel, grid, dim3(256), 0, stream, m, l, o, out, num_q,
                     sub_n_max, k_splits);
  return hipGetLastError();
}

// Zero-fill by a kernel, so that a caller that captures the reset into a HIP
// graph records a kernel node rather than a memset node.
__global__ __launch_bounds__(256) void fill_zero_kernel(uint32_t* __restrict__ p, size_t n_words) {
  for (size_t i = blockIdx.x * 256ul + threadIdx.x; i < n_words; i += (size_t)gridDim.x * 256)
    p[i] = 0u;
}

hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t stream) {
  const size_t n = bytes / 4;
  const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(fill_zero_kernel, dim3(blocks), dim3(256), 0, stream,
                     static_cast<uint32_t*>(p), n);
  return hipGetLastError();
}

// The health word of a fast-path workspace (header word kWsErrorWord) turned
// into a status and stored to `status` (device memory, or host memory the
// device can write) by one thread: ok_value while the word is 0, else
// timeout_value.  Stream-ordered, no host synchronization.
__global__ __launch_bounds__(64) void ws_status_kernel(const int* __restrict__ header, int* status,
                                                       int ok_value, int timeout_value) {
  if (threadIdx.x == 0) {
    const int w = __hip_atomic_load(header + kWsErrorWord, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *status = w == 0 ? ok_value : timeout_value;
  }
}

hipError_t launch_ws_status(const void* workspace, int* status, int ok_value, int timeout_value,
                            hipStream_t stream) {
  hipLaunchKernelGGL(ws_status_kernel, dim3(1), dim3(64), 0, stream, static_cast<const int*>(workspace),
                     status, ok_value, timeout_value);
  return hipGetLastError();
}

}  // namespace qkv
