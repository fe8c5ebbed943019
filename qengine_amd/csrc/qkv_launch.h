// qkv_launch.h -- host launchers of the gfx950 kernels (internal; the public
// surface is include/qkv.h).  Arguments are validated by qkv_api.cpp.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qkv {

// Row mapping of a paged append: input block i (token i / blocks_per_row,
// slot token / n_tok, position positions[slot] + token % n_tok) goes to
// pool row block_tables[slot * max_blocks + pos / block_tokens] *
// block_tokens + pos % block_tokens; rows outside [0, pool_rows) are skipped.
struct PagedRows {
  const int32_t* block_tables;
  const int32_t* positions;
  int max_blocks, block_tokens, blocks_per_row, n_tok;
  long pool_rows;
};

hipError_t launch_tq3_append(const void* in0, void* out0, const void* in1, void* out1,
                             int n_blocks, int n_tensors, hipStream_t stream,
                             const PagedRows* paged = nullptr);
hipError_t launch_tq3_dequant(const void* in, void* out, int n_blocks, hipStream_t stream);
hipError_t launch_q8_append(const void* in0, void* out0, const void* in1, void* out1,
                            int n_blocks, int n_tensors, hipStream_t stream);
hipError_t launch_q8_dequant(const void* in, void* out, int n_blocks, hipStream_t stream);

}  // namespace qkv
