// sparse_tq3.hip -- block selection for the block-sparse TQ3 verify (gfx950).
//
// Reference: the verify path of model.cuh:4589-4662 keeps per kv head a pool
// of 64-token block signatures over the TQ3 key cache (mean and sign-
// preserving max-abs of the dequantized keys, tq3_kpool_ms_update_kern,
// attention.cuh:2445-2533), scores every block for each verify query
// against the GQA-mean query, max(q.mean, beta * q.maxabs), and keeps the
// top_k blocks (build_block_index_ms_kern, sparse_attn/sparse_index.cuh:
// 214-330).  The attention over the selected blocks is tq3_attn_kernel<2>.
//
// Both kernels here reproduce the reference's values exactly: the keys are
// dequantized bit for bit (tq3_dequant_exact8), the signature sums run in the
// reference's order, the block scores sum exact fp16 x fp16 products pairwise
// in the reference's order, and the selection is the reference's repeated
// argmax (highest score, lower block index on ties), sorted ascending.
#include <algorithm>

#include "attn_common.h"
#include "qkv_device.h"
#include "qkv_launch.h"

// the signature and score sums keep the reference's separate roundings
#pragma clang fp contract(off)

namespace qkv {

constexpr int kSpThreads = 256;
constexpr int kSpHD = 256;
constexpr int kPoolPitch = kSpHD * 2 + 16;   // bytes per staged key row (fp16)

// One workgroup per (kv head, position block n = blk_lo + i): the block's up
// to 64 key rows are dequantized into LDS (16 lanes per 128-element TQ3
// block), then thread c reduces dimension c over the rows in position order.
__global__ __launch_bounds__(kSpThreads) void tq3_kpool_kernel(KpoolArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t rows[64 * kPoolPitch];
  const int n_upd = a.cur_blocks - a.blk_lo;
  const int h = blockIdx.x / n_upd;
  const int n = a.blk_lo + (int)(blockIdx.x - h * n_upd);
  const int t_lo = n * a.bsn;
  const int t_hi = min(t_lo + a.bsn, a.total_kv);
  const int n_pos = t_hi - t_lo;   // >= 1: n < cur_blocks
  const int tid = threadIdx.x;
  const int part = tid & 15, lane = tid & 63;
  // units (position, 128-block): 16 per pass of the workgroup
  for (int u = tid >> 4; u < 2 * n_pos; u += kSpThreads / 16) {
    const int pos = u >> 1, blk = u & 1;
    const uint8_t* src = reinterpret_cast<const uint8_t*>(a.k) +
                         ((uint64_t)(uint32_t)(t_lo + pos) * (uint32_t)a.num_kv + h) * 104u +
                         blk * 52u;
    uint32_t pk[4];
    tq3_dequant_exact8(src, part, lane, pk);
    *reinterpret_cast<uint4*>(rows + pos * kPoolPitch + (blk * 128 + part * 8) * 2) =
        make_uint4(pk[0], pk[1], pk[2], pk[3]);
  }
  __syncthreads();
  const int c = tid;   // 256 threads: one dimension each
  float sum = 0.0f, best_mag = 0.0f, best_val = 0.0f;
  for (int pos = 0; pos < n_pos; pos++) {
    const float x = h2f(*reinterpret_cast<const uint16_t*>(rows + pos * kPoolPitch + c * 2));
    sum += x;
    const float m = fabsf(x);
    if (m > best_mag) {
      best_mag = m;
      best_val = x;
    }
  }
  const long ob = ((long)h * a.stride + n) * kSpHD + c;
  a.k_pool[ob] = (uint16_t)f2h(sum / (float)n_pos);
  a.k_pool_max[ob] = (uint16_t)f2h(best_val);
}

// (value, index) order of the selection: higher value first, then lower index;
// index -1 (nothing) last
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  return i >= 0 && (bi < 0 || v > bv || (v == bv && i < bi));
}

// One workgroup per (kv head, verify query t).  Dynamic LDS: the scores of
// the n_blocks blocks.
__global__ __launch_bounds__(kSpThreads) void block_index_kernel(BlockIndexArgs a) {
  extern __shared__ float sc[];
  __shared__ float qa[kSpHD];
  __shared__ float wv[kSpThreads / 64];
  __shared__ int wi[kSpThreads / 64];
  const int h = blockIdx.x % a.num_kv;
  const int t = blockIdx.x / a.num_kv;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int gqa = a.num_q / a.num_kv;
  {
    // GQA-mean query, rounded to fp16 (sparse_index.cuh:243-252)
    const float inv_g = 1.0f / (float)gqa;
    float s = 0.0f;
    for (int g = 0; g < gqa; g++)
      s += h2f(a.q[((long)t * a.num_q + h * gqa + g) * kSpHD + tid]);
    qa[tid] = h2f(f2h(s * inv_g));
  }
  __syncthreads();
  const int causal_max = (a.start_pos + t) / a.bsn;
  for (int n = tid; n < a.n_blocks; n += kSpThreads) {
    const uint32_t* mn = reinterpret_cast<const uint32_t*>(a.k_pool + ((long)h * a.stride + n) * kSpHD);
    const uint32_t* mx =
        reinterpret_cast<const uint32_t*>(a.k_pool_max + ((long)h * a.stride + n) * kSpHD);
    float s_mean = 0.0f, s_max = 0.0f;
    for (int c2 = 0; c2 < kSpHD / 2; c2++) {
      const uint32_t m2 = mn[c2], x2 = mx[c2];
      const float q0 = qa[2 * c2], q1 = qa[2 * c2 + 1];
      s_mean += q0 * h2f(m2 & 0xffffu) + q1 * h2f(m2 >> 16);
      s_max += q0 * h2f(x2 & 0xffffu) + q1 * h2f(x2 >> 16);
    }
    const float s = fmaxf(s_mean, a.beta * s_max);
    sc[n] = n > causal_max ? -INFINITY : s;
  }
  __syncthreads();
  int32_t* row = a.block_index + ((long)h * a.sub_n_max + t) * a.top_k;
  int k = 0;
  for (; k < a.top_k; k++) {
    float bv = -INFINITY;
    int bi = -1;
    for (int n = tid; n < a.n_blocks; n += kSpThreads) {
      const float v = sc[n];
      if (v > bv) {   // strict: never a -inf or NaN score; lowest n of this thread's subset
        bv = v;
        bi = n;
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const float ov = __shfl_xor(bv, off);
      const int oi = __shfl_xor(bi, off);
      if (better(ov, oi, bv, bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if (lane == 0) {
      wv[wave] = bv;
      wi[wave] = bi;
    }
    __syncthreads();
    bv = wv[0];
    bi = wi[0];
#pragma unroll
    for (int w = 1; w < kSpThreads / 64; w++)
      if (better(wv[w], wi[w], bv, bi)) {
        bv = wv[w];
        bi = wi[w];
      }
    __syncthreads();   // every thread has read wv / wi before the next pick
    if (bi < 0) break;
    if (tid == 0) {
      row[k] = bi;
      sc[bi] = -INFINITY;
    }
    __syncthreads();
  }
  if (tid == 0) {
    for (int kk = k; kk < a.top_k; kk++) row[kk] = -1;
    for (int i = 1; i < k; i++) {   // ascending
      const int32_t x = row[i];
      int j = i;
      while (j > 0 && row[j - 1] > x) {
        row[j] = row[j - 1];
        j--;
      }
      row[j] = x;
    }
  }
}

hipError_t launch_tq3_kpool(const KpoolArgs& a, hipStream_t stream) {
  const int n_upd = a.cur_blocks - a.blk_lo;
  if (n_upd <= 0) return hipSuccess;
  hipLaunchKernelGGL(tq3_kpool_kernel, dim3((unsigned)(a.num_kv * n_upd)), dim3(kSpThreads), 0,
                     stream, a);
  return hipGetLastError();
}

hipError_t launch_block_index(const BlockIndexArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL(block_index_kernel, dim3((unsigned)(a.num_kv * a.sub_n)), dim3(kSpThreads),
                     (size_t)a.n_blocks * 4, stream, a);
  return hipGetLastError();
}

}  // namespace qkv
