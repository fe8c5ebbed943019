// kv_move.hip -- token-row moves inside one slot of a packed KV cache (gfx950).
//
// Reference: kv_move_token (model.cuh:7430-7471): for an accepted token the K
// and V rows (blocks_per_token blocks) at from_pos are copied to to_pos inside
// the slot, two device copies per token and layer.  Here one launch moves a
// whole list of tokens of one layer.  When no row is written by one move and
// read or written by another, every (move, K/V) pair is an independent
// workgroup; otherwise one workgroup performs the moves in list order with a
// barrier between them, which is the reference's sequential result.
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

}  // namespace qkv
