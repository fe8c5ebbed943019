/*
 * qkv_caller.c -- a compiled C (and C++) caller of include/qkv.h, used by
 * tests/test_gpu_c_caller.py.  It links libqkv.so and issues one TQ3 decode
 * step the way the reference's QwenModel launches it:
 *   - append of the cached tokens' K and V (the prefill's cache build),
 *   - append of the new token's K, then V, at row start_pos of the slot
 *     (model.cuh:2316-2333: two tq3_quantize_kernel launches),
 *   - split-K decode over the slot base, sub_n 1, sub_n_max 16, K_SPLITS 8,
 *     then the merge written in place over the query buffer
 *     (model.cuh:2472-2491),
 *   - and the single-launch fast path qkv_decode_attn_tq3 on the same inputs.
 *
 * usage: qkv_caller IN OUT
 *   IN : int32 n_ctx, num_q, num_kv; fp16 K[n_ctx+1][num_kv][256],
 *        V[n_ctx+1][num_kv][256], q[num_q][256]   (the new token is row n_ctx)
 *   OUT: fp16 merged[num_q][256], fp16 fast[num_q][256],
 *        K cache then V cache ((n_ctx+1) * num_kv * 2 blocks of 52 bytes each)
 * Exit status 0 on success; every library status is checked.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "qkv.h"

#define HD 256

static int fail(const char* what, int st) {
  fprintf(stderr, "qkv_caller: %s failed: %d (%s)\n", what, st, qkv_status_string(st));
  return 1;
}

#define CHECK_QKV(call)                      \
  do {                                       \
    int st_ = (call);                        \
    if (st_ != QKV_OK) return fail(#call, st_); \
  } while (0)

#define CHECK_HIP(call)                                                         \
  do {                                                                          \
    hipError_t e_ = (call);                                                     \
    if (e_ != hipSuccess) {                                                     \
      fprintf(stderr, "qkv_caller: %s: %s\n", #call, hipGetErrorString(e_));    \
      return 1;                                                                 \
    }                                                                           \
  } while (0)

static void* read_all(const char* path, size_t* n) {
  FILE* f = fopen(path, "rb");
  void* buf;
  long len;
  if (!f) return NULL;
  fseek(f, 0, SEEK_END);
  len = ftell(f);
  fseek(f, 0, SEEK_SET);
  buf = malloc((size_t)len);
  if (buf && fread(buf, 1, (size_t)len, f) != (size_t)len) {
    free(buf);
    buf = NULL;
  }
  fclose(f);
  *n = (size_t)len;
  return buf;
}

int main(int argc, char** argv) {
  size_t in_bytes = 0;
  const int32_t* hdr;
  int n_ctx, num_q, num_kv, bpt, k_splits = 8, sub_n_max = 16;
  size_t kv_elems, q_elems, cache_blocks;
  const uint16_t *hk, *hv, *hq;
  uint16_t *dk, *dv, *dq_split, *dq, *dout;
  qkv_block_tq3 *kc, *vc;
  float *pm, *pl, *po;
  void* ws;
  size_t ws_bytes;
  uint16_t* res;
  FILE* f;
  unsigned char* in;
  hipStream_t s;

  if (argc != 3) {
    fprintf(stderr, "usage: qkv_caller IN OUT\n");
    return 2;
  }
  in = (unsigned char*)read_all(argv[1], &in_bytes);
  if (!in || in_bytes < 12) {
    fprintf(stderr, "qkv_caller: cannot read %s\n", argv[1]);
    return 1;
  }
  hdr = (const int32_t*)in;
  n_ctx = hdr[0];
  num_q = hdr[1];
  num_kv = hdr[2];
  bpt = num_kv * HD / 128;
  kv_elems = (size_t)(n_ctx + 1) * num_kv * HD;
  q_elems = (size_t)num_q * HD;
  if (in_bytes != 12 + 2 * (2 * kv_elems + q_elems)) {
    fprintf(stderr, "qkv_caller: %s has %zu bytes, the header implies %zu\n", argv[1], in_bytes,
            12 + 2 * (2 * kv_elems + q_elems));
    return 1;
  }
  hk = (const uint16_t*)(in + 12);
  hv = hk + kv_elems;
  hq = hv + kv_elems;
  cache_blocks = (size_t)(n_ctx + 1) * bpt;

  CHECK_QKV(qkv_tq3_init(0));
  CHECK_HIP(hipSetDevice(0));
  CHECK_HIP(hipStreamCreate(&s));
  CHECK_HIP(hipMalloc((void**)&dk, kv_elems * 2));
  CHECK_HIP(hipMalloc((void**)&dv, kv_elems * 2));
  CHECK_HIP(hipMalloc((void**)&dq_split, q_elems * 2));
  CHECK_HIP(hipMalloc((void**)&dq, q_elems * 2));
  CHECK_HIP(hipMalloc((void**)&dout, q_elems * 2));
  CHECK_HIP(hipMalloc((void**)&kc, cache_blocks * sizeof(qkv_block_tq3)));
  CHECK_HIP(hipMalloc((void**)&vc, cache_blocks * sizeof(qkv_block_tq3)));
  /* the reference zero-fills its caches (model.cuh:1914-1920) */
  CHECK_HIP(hipMemset(kc, 0, cache_blocks * sizeof(qkv_block_tq3)));
  CHECK_HIP(hipMemset(vc, 0, cache_blocks * sizeof(qkv_block_tq3)));
  CHECK_HIP(hipMalloc((void**)&pm, (size_t)num_q * sub_n_max * k_splits * sizeof(float)));
  CHECK_HIP(hipMalloc((void**)&pl, (size_t)num_q * sub_n_max * k_splits * sizeof(float)));
  CHECK_HIP(hipMalloc((void**)&po, (size_t)num_q * sub_n_max * k_splits * HD * sizeof(float)));
  ws_bytes = qkv_decode_attn_tq3_workspace_bytes(num_q, num_kv, 1, n_ctx + 1);
  if (ws_bytes == 0) return fail("qkv_decode_attn_tq3_workspace_bytes", QKV_ERR_INVALID);
  CHECK_HIP(hipMalloc(&ws, ws_bytes));
  CHECK_HIP(hipMemset(ws, 0, ws_bytes));
  CHECK_HIP(hipMemcpy(dk, hk, kv_elems * 2, hipMemcpyHostToDevice));
  CHECK_HIP(hipMemcpy(dv, hv, kv_elems * 2, hipMemcpyHostToDevice));
  CHECK_HIP(hipMemcpy(dq_split, hq, q_elems * 2, hipMemcpyHostToDevice));
  CHECK_HIP(hipMemcpy(dq, hq, q_elems * 2, hipMemcpyHostToDevice));

  /* cache build: rows 0 .. n_ctx-1 */
  if (n_ctx > 0) {
    CHECK_QKV(qkv_tq3_append(dk, kc, n_ctx * bpt, s));
    CHECK_QKV(qkv_tq3_append(dv, vc, n_ctx * bpt, s));
  }
  /* decode step: the new token's K, then V, at row n_ctx (kv_slot) */
  CHECK_QKV(qkv_tq3_append(dk + (size_t)n_ctx * num_kv * HD, kc + (size_t)n_ctx * bpt, bpt, s));
  CHECK_QKV(qkv_tq3_append(dv + (size_t)n_ctx * num_kv * HD, vc + (size_t)n_ctx * bpt, bpt, s));
  /* split-K decode (query row start_pos = n_ctx sees keys 0..n_ctx), merged in place */
  CHECK_QKV(qkv_attn_split_tq3(dq_split, kc, vc, pm, pl, po, num_q, num_kv, HD, n_ctx, 1, sub_n_max,
                               n_ctx + 1, 1.0f / 16.0f, k_splits, 0, 0, NULL, s));
  CHECK_QKV(qkv_attn_split_merge(pm, pl, po, dq_split, num_q, num_kv, HD, 1, sub_n_max, k_splits, s));
  /* the single-launch fast path */
  CHECK_QKV(qkv_decode_attn_tq3(dq, kc, vc, dout, num_q, num_kv, HD, n_ctx, 1, 1.0f / 16.0f, 0, 0,
                                NULL, ws, ws_bytes, s));
  CHECK_HIP(hipStreamSynchronize(s));
  CHECK_QKV(qkv_decode_workspace_status(ws, s));

  res = (uint16_t*)malloc(2 * q_elems * 2 + 2 * cache_blocks * sizeof(qkv_block_tq3));
  if (!res) return 1;
  CHECK_HIP(hipMemcpy(res, dq_split, q_elems * 2, hipMemcpyDeviceToHost));
  CHECK_HIP(hipMemcpy(res + q_elems, dout, q_elems * 2, hipMemcpyDeviceToHost));
  CHECK_HIP(hipMemcpy((unsigned char*)(res + 2 * q_elems), kc, cache_blocks * sizeof(qkv_block_tq3),
                      hipMemcpyDeviceToHost));
  CHECK_HIP(hipMemcpy((unsigned char*)(res + 2 * q_elems) + cache_blocks * sizeof(qkv_block_tq3), vc,
                      cache_blocks * sizeof(qkv_block_tq3), hipMemcpyDeviceToHost));
  f = fopen(argv[2], "wb");
  if (!f) return 1;
  if (fwrite(res, 1, 2 * q_elems * 2 + 2 * cache_blocks * sizeof(qkv_block_tq3), f) !=
      2 * q_elems * 2 + 2 * cache_blocks * sizeof(qkv_block_tq3)) {
    fclose(f);
    return 1;
  }
  fclose(f);
  CHECK_HIP(hipFree(dk));
  CHECK_HIP(hipFree(dv));
  CHECK_HIP(hipFree(dq_split));
  CHECK_HIP(hipFree(dq));
  CHECK_HIP(hipFree(dout));
  CHECK_HIP(hipFree(kc));
  CHECK_HIP(hipFree(vc));
  CHECK_HIP(hipFree(pm));
  CHECK_HIP(hipFree(pl));
  CHECK_HIP(hipFree(po));
  CHECK_HIP(hipFree(ws));
  CHECK_HIP(hipStreamDestroy(s));
  free(res);
  free(in);
  printf("qkv_caller: ok (n_ctx %d, num_q %d, num_kv %d)\n", n_ctx, num_q, num_kv);
  return 0;
}
