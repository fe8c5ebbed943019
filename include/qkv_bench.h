/* qkv_bench.h -- measurement helper of the benchmark (libqkv_bench.so), kept
 * out of the product library libqkv.so.  Status codes are those of qkv.h. */
#ifndef QKV_BENCH_H
#define QKV_BENCH_H

#include <stddef.h>
#include <stdint.h>

#include "qkv.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Measurement helper, not a cache operation: one streaming read of `bytes`
 * (a multiple of 64) from device memory, each byte once, nothing stored
 * (sink, one dword, is written only for a data pattern no caller produces).
 * Timed around a buffer larger than the 256 MB Infinity Cache it gives the
 * sustained read bandwidth the decode's HBM fraction is also quoted against;
 * the reference measures the same with tools/bench_hbm_bandwidth.cu
 * (k_read_f4, lines 45-57). */
int qkv_hbm_read_bench(const void* buf, size_t bytes, uint32_t* sink, hipStream_t stream);

/* Measurement helper, not a cache operation: `workgroups` workgroups of 8
 * waves, each wave issuing 16 x iters v_mfma_f32_32x32x16_f16 (32,768 flops
 * each) on pseudo-random fp16 operands that rotate over four sets, nothing
 * stored (sink, one float, is written only for a value no run produces).
 * Timed over a few milliseconds it gives the fp16 matrix rate the part
 * sustains on data-like operands, the ceiling the prefill's MFMA fraction is
 * also quoted against. */
int qkv_mfma_rate_bench(int workgroups, int iters, float* sink, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* QKV_BENCH_H */
