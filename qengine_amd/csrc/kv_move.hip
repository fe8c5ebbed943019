// kv_move.hip -- token-row moves inside one slot of a packed KV cache (gfx950).
//
// Reference: kv_move_token (model.cuh:7430-7471): for an accepted token the K
// and V rows (blocks_per_token blocks) at from_pos are copied to to_pos inside
// the slot, two device copies per token and layer.  Here one launch moves a
// whole list of tokens of one layer.  When no row is written by one move and
// read or written by another, every (move, K/V) pair is an independent
// workgroup; otherwise one workgroup performs the moves in list order with a
// barrier between them, which is the reference's sequential result.
#include <algorithm>
#include <type_traits>

#include "qkv_launch.h"

namespace qkv {

constexpr int kMoveThreads = 256;

// Copy one row of row_bytes (a multiple of 4) from row src to row dst.
__device__ __forceinline__ void copy_row(uint8_t* base, uint32_t row_bytes, long src, long dst) {
  const uint32_t* s = reinterpret_cast<const uint32_t*>(base + src * row_bytes);
  uint32_t* d = reinterpret_cast<uint32_t*>(base + dst * row_bytes);
  for (uint32_t i = threadIdx.x; i < row_bytes / 4; i += kMoveThreads) d[i] = s[i];
}

// workgroup (i, kv): move i of the K rows (kv 0) or the V rows (kv 1)
__global__ __launch_bounds__(kMoveThreads) void kv_move_parallel_kernel(MoveArgs a) {
  const int i = blockIdx.x;
  if (a.from[i] == a.to[i]) return;
  if (blockIdx.y == 0)
    copy_row(a.k, a.k_row_bytes, a.slot_row0 + a.from[i], a.slot_row0 + a.to[i]);
  else
    copy_row(a.v, a.v_row_bytes, a.slot_row0 + a.from[i], a.slot_row0 + a.to[i]);
}

// one workgroup, the moves in list order
__global__ __launch_bounds__(kMoveThreads) void kv_move_ordered_kernel(MoveArgs a) {
  for (int i = 0; i < a.n; i++) {
    if (a.from[i] != a.to[i]) {
      copy_row(a.k, a.k_row_bytes, a.slot_row0 + a.from[i], a.slot_row0 + a.to[i]);
      copy_row(a.v, a.v_row_bytes, a.slot_row0 + a.from[i], a.slot_row0 + a.to[i]);
    }
    __syncthreads();   // this move's stores are seen by the next move's loads
  }
}

hipError_t launch_kv_move(const MoveArgs& a, bool ordered, hipStream_t stream) {
  if (ordered)
    hipLaunchKernelGGL(kv_move_ordered_kernel, dim3(1), dim3(kMoveThreads), 0, stream, a);
  else
    hipLaunchKernelGGL(kv_move_parallel_kernel, dim3(a.n, 2), dim3(kMoveThreads), 0, stream, a);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Slot snapshot / restore over a paged pool.  The reference copies a slot's
// first N rows of K and V between the contiguous cache and pinned host memory
// (save_prefix_snapshot / restore_snapshot_into_slot, model.cuh:3314-3459).
// With a paged pool the slot's logical row r lives at pool row
// table[r / block_tokens] * block_tokens + r % block_tokens; these kernels
// gather those rows into a flat [N][row] buffer (which the caller copies to
// the host as the reference does) and scatter a flat buffer back.  One thread
// per 16 bytes (rows are multiples of 16 bytes) or per dword otherwise.
// ---------------------------------------------------------------------------
template <int UNIT, bool SCATTER>
__global__ __launch_bounds__(256) void kv_page_copy_kernel(PageCopyArgs a) {
  typedef typename std::conditional<UNIT == 16, uint4, uint32_t>::type unit_t;
  const int t = blockIdx.y;
  const uint32_t row_units = a.row_bytes[t] / UNIT;
  const long g = (long)blockIdx.x * 256 + threadIdx.x;
  if (g >= (long)a.n_rows * row_units) return;
  const long r = g / row_units;
  const uint32_t c = (uint32_t)(g - r * row_units);
  const long b = r / a.block_tokens;
  long prow = -1;
  if (b < a.max_blocks) {
    const long e = a.table[b];
    prow = e < 0 ? -1 : e * a.block_tokens + (r - b * a.block_tokens);
    if (prow >= a.pool_rows) prow = -1;
  }
  unit_t* flat = reinterpret_cast<unit_t*>(a.flat[t] + r * a.row_bytes[t]) + c;
  if (SCATTER) {
    if (prow >= 0)
      reinterpret_cast<unit_t*>(a.pool[t] + prow * a.row_bytes[t])[c] = *flat;
  } else {
    *flat = prow >= 0 ? reinterpret_cast<const unit_t*>(a.pool[t] + prow * a.row_bytes[t])[c]
                      : unit_t{};
  }
}

hipError_t launch_kv_page_copy(const PageCopyArgs& a, bool scatter, hipStream_t stream) {
  const bool wide = a.row_bytes[0] % 16 == 0 && (a.n_tensors < 2 || a.row_bytes[1] % 16 == 0) &&
                    a.aligned16;
  const uint32_t unit = wide ? 16 : 4;
  uint32_t max_units = a.row_bytes[0] / unit;
  if (a.n_tensors == 2) max_units = std::max(max_units, a.row_bytes[1] / unit);
  const long total = (long)a.n_rows * max_units;
  const dim3 grid((unsigned)((total + 255) / 256), a.n_tensors);
  if (wide && scatter)
    hipLaunchKernelGGL((kv_page_copy_kernel<16, true>), grid, dim3(256), 0, stream, a);
  else if (wide)
    hipLaunchKernelGGL((kv_page_copy_kernel<16, false>), grid, dim3(256), 0, stream, a);
  else if (scatter)
    hipLaunchKernelGGL((kv_page_copy_kernel<4, true>), grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((kv_page_copy_kernel<4, false>), grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace qkv
