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
// The kernels here reproduce the reference's values exactly: the keys are
// dequantized bit for bit (tq3_group_dequant), the signature sums run in the
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
  __shared__ float cent[8];
  const int n_upd = a.cur_blocks - a.blk_lo;
  const int h = blockIdx.x / n_upd;
  const int n = a.blk_lo + (int)(blockIdx.x - h * n_upd);
  const int t_lo = n * a.bsn;
  const int t_hi = min(t_lo + a.bsn, a.total_kv);
  const int n_pos = t_hi - t_lo;   // >= 1: n < cur_blocks
  const int tid = threadIdx.x;
  const int part = tid & 15;
  tq3_centroid_table(cent, tid);
  const Tq3LaneConst lc = tq3_lane_const(part);
  // units (position, 128-block): 16 per pass of the workgroup, at most 8
  // passes (64 rows); every pass's loads are issued before the first is used
  constexpr int kPasses = 2 * 64 / (kSpThreads / 16);
  Tq3Group gr[kPasses];
#pragma unroll
  for (int p = 0; p < kPasses; p++) {
    const int u0 = (tid >> 4) + p * (kSpThreads / 16);
    const int u = u0 < 2 * n_pos ? u0 : 0;   // a unit past the block's rows re-reads unit 0
    const uint8_t* src = reinterpret_cast<const uint8_t*>(a.k) +
                         ((uint64_t)(uint32_t)(t_lo + (u >> 1)) * (uint32_t)a.num_kv + h) * 104u +
                         (u & 1) * 52u;
    gr[p] = tq3_group_load(src, part);
  }
  __syncthreads();   // the centroid table
#pragma unroll
  for (int p = 0; p < kPasses; p++) {
    const int u = (tid >> 4) + p * (kSpThreads / 16);
    if (u < 2 * n_pos) {   // uniform over the unit's 16 lanes (lane exchange inside)
      const int pos = u >> 1, blk = u & 1;
      uint32_t pk[4];
      tq3_group_dequant(gr[p], part, cent, lc, pk);
      *reinterpret_cast<uint4*>(rows + pos * kPoolPitch + (blk * 128 + part * 8) * 2) =
          make_uint4(pk[0], pk[1], pk[2], pk[3]);
    }
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

constexpr int kScBlocks = 32;          // blocks scored per workgroup
constexpr int kScQueries = 8;          // queries scored per workgroup
constexpr int kScPitchDw = 129;        // staged pool row: 128 dwords + 1 (conflict-free lanes)

// Block scores, one workgroup per (kv head, 32 blocks, 8 queries).  The
// blocks' mean and max-abs rows are staged in LDS; the GQA-mean queries
// (fp16-rounded, as the reference forms them, sparse_index.cuh:243-252) sit in
// LDS as fp16 pairs; thread (t, b) runs block b's two dot products for query
// t over the 128 pairs in the reference's order: each pair's products are
// exact and their sum is rounded once (an FMA onto the other exact product),
// then added to the running fp32 sum.  (v_dot2_f32_f16 does not give that
// rounding.)  Scores (-inf past the
// query's causal block) go to the workspace [num_kv][sub_n][n_blocks].
__global__ __launch_bounds__(kSpThreads) void block_score_kernel(BlockIndexArgs a, float* scores) {
  __shared__ uint32_t rows_mean[kScBlocks * kScPitchDw];
  __shared__ uint32_t rows_max[kScBlocks * kScPitchDw];
  __shared__ uint32_t qa2[kScQueries * kSpHD / 2];   // fp16 pairs
  const int nb_wg = (a.n_blocks + kScBlocks - 1) / kScBlocks;
  const int nq_wg = (a.sub_n + kScQueries - 1) / kScQueries;
  const int qg = blockIdx.x % nq_wg, r = blockIdx.x / nq_wg;
  const int h = r / nb_wg, b0 = (r - h * nb_wg) * kScBlocks, t0 = qg * kScQueries;
  const int nt = min(kScQueries, a.sub_n - t0);
  const int tid = threadIdx.x;
  const int gqa = a.num_q / a.num_kv;
  // Every load of the staging and of the query is issued before the first
  // one is used (one memory round trip for the workgroup's inputs).
  // 32 blocks x {mean, max} x 512 B: 2048 16-byte pieces, 8 per thread
  // (blocks past the pool's end are read at its last block and zeroed)
  static_assert(kScBlocks * 64 == 8 * kSpThreads, "8 staging pieces per thread");
  uint4 pv[8];
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const int piece = tid + k * kSpThreads;
    const int b = piece >> 6, w = piece & 63;   // w < 32: mean, else max; 8 dims each
    const int nbk = min(b0 + b, a.n_blocks - 1);
    pv[k] = *reinterpret_cast<const uint4*>((w < 32 ? a.k_pool : a.k_pool_max) +
                                            ((long)h * a.stride + nbk) * kSpHD + (w & 31) * 8);
  }
  // GQA-mean query pairs: thread i < nt * 128 forms pair c of query tq from
  // the 8 (or gqa) heads' fp16 pairs, loaded together (heads past gqa re-read
  // the last head and are not added)
  static_assert(kScQueries * kSpHD / 2 == 4 * kSpThreads, "4 query pairs per thread");
  uint32_t qv[4][8];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int i = min(tid + k * kSpThreads, nt * kSpHD / 2 - 1);
    const int tq = i / (kSpHD / 2), c = 2 * (i - tq * (kSpHD / 2));
#pragma unroll
    for (int g = 0; g < 8; g++)
      qv[k][g] = *reinterpret_cast<const uint32_t*>(
          a.q + ((long)(t0 + tq) * a.num_q + h * gqa + min(g, gqa - 1)) * kSpHD + c);
  }
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const int piece = tid + k * kSpThreads;
    const int b = piece >> 6, w = piece & 63;
    const uint4 v = b0 + b < a.n_blocks ? pv[k] : make_uint4(0u, 0u, 0u, 0u);
    uint32_t* d = (w < 32 ? rows_mean : rows_max) + b * kScPitchDw + (w & 31) * 4;
    d[0] = v.x;
    d[1] = v.y;
    d[2] = v.z;
    d[3] = v.w;
  }
  const float inv_g = a.inv_gqa;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int i = tid + k * kSpThreads;
    if (i < nt * kSpHD / 2) {
      float s0 = 0.0f, s1 = 0.0f;   // heads in order (the reference's sum)
#pragma unroll
      for (int g = 0; g < 8; g++)
        if (g < gqa) {
          s0 += h2f(qv[k][g] & 0xffffu);
          s1 += h2f(qv[k][g] >> 16);
        }
      // the reference rounds s * (1/GQA) to fp32, then to fp16: the empty asm
      // keeps the fp32 product (no fused fp16-rounding mixed FMA)
      float p0 = s0 * inv_g, p1 = s1 * inv_g;
      asm volatile("" : "+v"(p0), "+v"(p1));
      qa2[i] = f2h(p0) | (f2h(p1) << 16);
    }
  }
  __syncthreads();
  // thread -> (query tq, block b): 32 lanes of a wave are the 32 blocks of one query
  const int tq = tid / kScBlocks, b = tid - tq * kScBlocks;
  if (tq < nt) {
    const uint32_t* mn = rows_mean + b * kScPitchDw;
    const uint32_t* mx = rows_max + b * kScPitchDw;
    const uint32_t* q = qa2 + tq * (kSpHD / 2);
    float s_mean = 0.0f, s_max = 0.0f;
#pragma unroll 16
    for (int c2 = 0; c2 < kSpHD / 2; c2++) {
      const uint32_t qw = q[c2], m2 = mn[c2], x2 = mx[c2];
      const float q0 = h2f(qw & 0xffffu), q1 = h2f(qw >> 16);
      s_mean += __builtin_fmaf(q0, h2f(m2 & 0xffffu), q1 * h2f(m2 >> 16));
      s_max += __builtin_fmaf(q0, h2f(x2 & 0xffffu), q1 * h2f(x2 >> 16));
    }
    const int n = b0 + b, t = t0 + tq;
    if (n < a.n_blocks) {
      const float sc = fmaxf(s_mean, a.beta * s_max);
      scores[((long)h * a.sub_n + t) * a.n_blocks + n] = n > (a.start_pos + t) / a.bsn ? -INFINITY : sc;
    }
  }
}

// Selection, one workgroup per (kv head, query t).  The reference's repeated
// argmax (ties to the lower block, -inf and NaN never chosen, -1 padding)
// picks the first top_k blocks in the order (score descending, block
// ascending), and its list is then sorted ascending: it is that set.  It is
// found without sorting by a radix select on an order-preserving 32-bit key
// of the score (-0 and +0 equal):
//   1. four 8-bit passes narrow the key T of the top_k-th pick (a 256-bin
//      histogram of the keys that share the digits found so far, and a
//      suffix scan over the bins);
//   2. the picks are the blocks with key > T and the lowest-numbered `need`
//      blocks with key == T (a block-wide scan in block order);
//   3. a second scan gives each pick its place in the ascending list.
// Each thread owns a contiguous run of blocks.
constexpr int kTkThreads = 256;

__device__ __forceinline__ uint32_t order_key(float v) {
  const uint32_t b = __float_as_uint(v == 0.0f ? 0.0f : v);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ bool pickable(float v) { return v > -INFINITY; }   // false for NaN

// Exclusive scan of v over the workgroup (block order = thread order), and the total.
__device__ __forceinline__ int block_scan(int v, int* wtot, int& total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int inc = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int u = __shfl_up(inc, d, 64);
    if (lane >= d) inc += u;
  }
  if (lane == 63) wtot[wave] = inc;
  __syncthreads();
  int off = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kTkThreads / 64; w++) {
    const int x = wtot[w];
    off += w < wave ? x : 0;
    tot += x;
  }
  __syncthreads();
  total = tot;
  return off + inc - v;
}

// Rows of up to kSelLdsKeys blocks are read once and keep their keys in LDS
// for all passes; longer rows read the scores from the workspace in every pass.
constexpr int kSelLdsKeys = 8192;
__global__ __launch_bounds__(kTkThreads) void block_select_kernel(BlockIndexArgs a, const float* scores) {
  __shared__ uint32_t keys_s[kSelLdsKeys];
  __shared__ int hist[256];
  __shared__ int wtot[kTkThreads / 64];
  __shared__ int found[2];
  const int h = blockIdx.x % a.num_kv, t = blockIdx.x / a.num_kv;
  const int tid = threadIdx.x;
  const float* src = scores + ((long)h * a.sub_n + t) * a.n_blocks;
  int32_t* row = a.block_index + ((long)h * a.sub_n_max + t) * a.top_k;
  const int per = (a.n_blocks + kTkThreads - 1) / kTkThreads;
  const int i0 = min(tid * per, a.n_blocks), i1 = min(i0 + per, a.n_blocks);
  // key of block i: the order key of a pickable score, 0 otherwise (every
  // pickable score, > -inf and not NaN, has a key above 0x007FFFFF)
  const bool staged = a.n_blocks <= kSelLdsKeys;
  auto key_from = [](float v) -> uint32_t { return pickable(v) ? order_key(v) : 0u; };
  if (staged) {
    for (int i = tid; i < a.n_blocks; i += kTkThreads) keys_s[i] = key_from(src[i]);
    __syncthreads();
  }
  auto key_at = [&](int i) -> uint32_t { return staged ? keys_s[i] : key_from(src[i]); };

  int n_ok = 0;
  for (int i = i0; i < i1; i++) n_ok += key_at(i) != 0u;
  int total;
  (void)block_scan(n_ok, wtot, total);
  const bool all = total <= a.top_k;   // every pickable block is picked
  uint32_t T = 0u;
  int need = 0;
  if (!all) {
    uint32_t prefix = 0u, mask = 0u;
    int kk = a.top_k;   // rank of the pick sought among the keys sharing `prefix`
    for (int shift = 24; shift >= 0; shift -= 8) {
      hist[tid] = 0;
      __syncthreads();
      for (int i = i0; i < i1; i++) {
        const uint32_t key = key_at(i);
        if (key != 0u && (key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1);
      }
      __syncthreads();
      // suffix sums: thread tid takes bin 255 - tid
      const int c = hist[255 - tid];
      int tot;
      const int above = block_scan(c, wtot, tot);   // keys in bins above 255 - tid
      if (above < kk && above + c >= kk) {
        found[0] = 255 - tid;
        found[1] = kk - above;
      }
      __syncthreads();
      prefix |= (uint32_t)found[0] << shift;
      mask |= 255u << shift;
      kk = found[1];
      __syncthreads();
    }
    T = prefix;
    need = kk;   // picks among the blocks whose key is exactly T
  }
  // picks, in block order
  int n_eq = 0;
  if (!all)
    for (int i = i0; i < i1; i++) n_eq += key_at(i) == T;
  int tot_eq;
  int eq_rank = block_scan(n_eq, wtot, tot_eq);
  int n_pick = 0;
  for (int i = i0; i < i1; i++) {
    const uint32_t key = key_at(i);
    if (key == 0u) continue;
    if (all || key > T) {
      n_pick++;
    } else if (key == T) {
      n_pick += eq_rank < need;
      eq_rank++;
    }
  }
  int n_total;
  int pos = block_scan(n_pick, wtot, n_total);
  eq_rank -= n_eq;   // back to this thread's first equal key
  for (int i = i0; i < i1; i++) {
    const uint32_t key = key_at(i);
    if (key == 0u) continue;
    bool pick = all || key > T;
    if (!all && key == T) {
      pick = eq_rank < need;
      eq_rank++;
    }
    if (pick) row[pos++] = i;
  }
  for (int j = n_total + tid; j < a.top_k; j += kTkThreads) row[j] = -1;
}

hipError_t launch_tq3_kpool(const KpoolArgs& a, hipStream_t stream) {
  const int n_upd = a.cur_blocks - a.blk_lo;
  if (n_upd <= 0) return hipSuccess;
  hipLaunchKernelGGL(tq3_kpool_kernel, dim3((unsigned)(a.num_kv * n_upd)), dim3(kSpThreads), 0,
                     stream, a);
  return hipGetLastError();
}

hipError_t launch_block_index(const BlockIndexArgs& a, float* scores, hipStream_t stream) {
  const int nb_wg = (a.n_blocks + kScBlocks - 1) / kScBlocks;
  const int nq_wg = (a.sub_n + kScQueries - 1) / kScQueries;
  if (nb_wg == 0 || nq_wg == 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(block_score_kernel, dim3((unsigned)(a.num_kv * nb_wg * nq_wg)), dim3(kSpThreads), 0,
                     stream, a, scores);
  hipLaunchKernelGGL(block_select_kernel, dim3((unsigned)(a.num_kv * a.sub_n)), dim3(kTkThreads), 0,
                     stream, a, static_cast<const float*>(scores));
  return hipGetLastError();
}

}  // namespace qkv
