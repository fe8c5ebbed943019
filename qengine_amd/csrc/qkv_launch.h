// qkv_launch.h -- host launchers of the gfx950 kernels (internal; the public
// surface is include/qkv.h).  Arguments are validated by qkv_api.cpp.
#pragma once
#include <hip/hip_runtime.h>

namespace qkv {

hipError_t launch_tq3_append(const void* in0, void* out0, const void* in1, void* out1,
                             int n_blocks, int n_tensors, hipStream_t stream);
hipError_t launch_tq3_dequant(const void* in, void* out, int n_blocks, hipStream_t stream);
hipError_t launch_q8_append(const void* in0, void* out0, const void* in1, void* out1,
                            int n_blocks, int n_tensors, hipStream_t stream);
hipError_t launch_q8_dequant(const void* in, void* out, int n_blocks, hipStream_t stream);

}  // namespace qkv
