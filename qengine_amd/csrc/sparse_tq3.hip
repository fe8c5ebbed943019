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

constexpr int kScBlocks = 64;          // blocks scored per workgroup
constexpr int kScPitchDw = 129;        // staged pool row: 128 dwords + 1 (conflict-free lanes)

// Block scores for every verify query of a kv head: one workgroup per (kv
// head, 64 blocks).  The blocks' mean and max-abs rows are staged in LDS once
// and scored against all sub_n GQA-mean queries (fp16-rounded, as the
// reference forms them, sparse_index.cuh:243-252); thread (t, b) runs block
// b's two dot products for query t over the 128 half2 pairs in the
// reference's order.  Scores (-inf past the query's causal block) go to the
// workspace [num_kv][sub_n][n_blocks].
__global__ __launch_bounds__(kSpThreads) void block_score_kernel(BlockIndexArgs a, float* scores) {
  __shared__ uint32_t rows_mean[kScBlocks * kScPitchDw];
  __shared__ uint32_t rows_max[kScBlocks * kScPitchDw];
  __shared__ float qa[16 * kSpHD];   // up to 16 queries per pass
  const int nb_wg = (a.n_blocks + kScBlocks - 1) / kScBlocks;
  const int h = blockIdx.x / nb_wg, b0 = (blockIdx.x - h * nb_wg) * kScBlocks;
  const int tid = threadIdx.x;
  const int gqa = a.num_q / a.num_kv;
  // stage 64 blocks x {mean, max} x 512 B: 4096 16-byte pieces, 16 per thread
  for (int piece = tid; piece < kScBlocks * 64; piece += kSpThreads) {
    const int b = piece >> 6, w = piece & 63;   // w < 32: mean, else max; 8 dims each
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (b0 + b < a.n_blocks)
      v = *reinterpret_cast<const uint4*>((w < 32 ? a.k_pool : a.k_pool_max) +
                                          ((long)h * a.stride + b0 + b) * kSpHD + (w & 31) * 8);
    uint32_t* d = (w < 32 ? rows_mean : rows_max) + b * kScPitchDw + (w & 31) * 4;
    d[0] = v.x;
    d[1] = v.y;
    d[2] = v.z;
    d[3] = v.w;
  }
  const float inv_g = 1.0f / (float)gqa;
  for (int t0 = 0; t0 < a.sub_n; t0 += 16) {
    const int nt = min(16, a.sub_n - t0);
    __syncthreads();   // staging done / the previous pass is done with qa
    for (int i = tid; i < nt * kSpHD; i += kSpThreads) {
      const int tq = i / kSpHD, c = i - tq * kSpHD;
      float s = 0.0f;
      for (int g = 0; g < gqa; g++)
        s += h2f(a.q[((long)(t0 + tq) * a.num_q + h * gqa + g) * kSpHD + c]);
      qa[tq * kSpHD + c] = h2f(f2h(s * inv_g));
    }
    __syncthreads();
    // thread -> (query tq, block b): a wave's 64 lanes are 64 blocks of one query
    for (int pr = tid; pr < nt * kScBlocks; pr += kSpThreads) {
      const int tq = pr / kScBlocks, b = pr - tq * kScBlocks;
      const uint32_t* mn = rows_mean + b * kScPitchDw;
      const uint32_t* mx = rows_max + b * kScPitchDw;
      const float* q = qa + tq * kSpHD;
      float s_mean = 0.0f, s_max = 0.0f;
#pragma unroll 8
      for (int c2 = 0; c2 < kSpHD / 2; c2++) {
        const uint32_t m2 = mn[c2], x2 = mx[c2];
        const float q0 = q[2 * c2], q1 = q[2 * c2 + 1];
        s_mean += q0 * h2f(m2 & 0xffffu) + q1 * h2f(m2 >> 16);
        s_max += q0 * h2f(x2 & 0xffffu) + q1 * h2f(x2 >> 16);
      }
      const int n = b0 + b, t = t0 + tq;
      if (n < a.n_blocks) {
        const float s = fmaxf(s_mean, a.beta * s_max);
        scores[((long)h * a.sub_n + t) * a.n_blocks + n] = n > (a.start_pos + t) / a.bsn ? -INFINITY : s;
      }
    }
  }
}

// (value, index) order of the selection: higher value first, then lower index;
// index -1 (nothing) last
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  return i >= 0 && (bi < 0 || v > bv || (v == bv && i < bi));
}

// Selection, one wave per (kv head, query t): lane l keeps the best (score,
// block) of blocks l, l + 64, ...; each pick is the wave's best pair, after
// which its lane rescans its blocks; then the picks are sorted ascending (by
// rank across the lanes, or in LDS past 64 picks) and padded with -1.  The result is the reference's repeated argmax.  Lanes hold
// their blocks' scores in registers when there are at most 64 * kSelRegs
// blocks, in LDS otherwise.
constexpr int kSelRegs = 40;

// One step of a wave argmax under `better`: the (score, block) pair of the
// DPP source lane replaces the lane's own when it is better.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ void argmax_step(float& v, int& i) {
  const float ov = dpp_f<CTRL, ROW_MASK>(v);
  const int oi = __builtin_amdgcn_update_dpp(i, i, CTRL, ROW_MASK, 0xf, false);
  if (better(ov, oi, v, i)) {
    v = ov;
    i = oi;
  }
}

// The wave's best pair, in every lane (the reduction of wave_max: quad swaps,
// row rotations, row broadcasts, the result in lane 63).
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
  argmax_step<0xB1>(v, i);
  argmax_step<0x4E>(v, i);
  argmax_step<0x124>(v, i);
  argmax_step<0x128>(v, i);
  argmax_step<0x142, 0xa>(v, i);
  argmax_step<0x143, 0xc>(v, i);
  v = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
  i = __builtin_amdgcn_readlane(i, 63);
}
template <bool REGS>
__global__ __launch_bounds__(64) void block_select_kernel(BlockIndexArgs a, const float* scores) {
  extern __shared__ float sc_lds[];
  const int h = blockIdx.x % a.num_kv, t = blockIdx.x / a.num_kv;
  const int lane = threadIdx.x;
  const float* src = scores + ((long)h * a.sub_n + t) * a.n_blocks;
  float r[REGS ? kSelRegs : 1];
  if constexpr (REGS) {
#pragma unroll
    for (int j = 0; j < kSelRegs; j++) {
      const int n = lane + 64 * j;
      r[j] = n < a.n_blocks ? src[n] : -INFINITY;
    }
  } else {
    for (int n = lane; n < a.n_blocks; n += 64) sc_lds[n] = src[n];
  }
  auto lane_best = [&](float& bv, int& bi) {
    bv = -INFINITY;
    bi = -1;
    if constexpr (REGS) {
#pragma unroll
      for (int j = 0; j < kSelRegs; j++)
        if (r[j] > bv) {   // strict: never -inf or NaN; ascending blocks keep the lower one
          bv = r[j];
          bi = lane + 64 * j;
        }
    } else {
      for (int n = lane; n < a.n_blocks; n += 64) {
        const float v = sc_lds[n];
        if (v > bv) {
          bv = v;
          bi = n;
        }
      }
    }
  };
  float lv;
  int li;
  lane_best(lv, li);
  int32_t* row = a.block_index + ((long)h * a.sub_n_max + t) * a.top_k;
  // picks: lane k holds pick k when top_k <= 64, else an LDS list after the scores
  int* picks = reinterpret_cast<int*>(sc_lds + (REGS ? 0 : a.n_blocks));
  int mine = -1;
  int k = 0;
  for (; k < a.top_k; k++) {
    float bv = lv;
    int bi = li;
    wave_argmax(bv, bi);
    if (bi < 0) break;   // wave-uniform
    if (a.top_k <= 64) {
      if (lane == k) mine = bi;
    } else if (lane == 0) {
      picks[k] = bi;
    }
    if (lane == (bi & 63)) {
      if constexpr (REGS) {
#pragma unroll
        for (int j = 0; j < kSelRegs; j++)
          if (lane + 64 * j == bi) r[j] = -INFINITY;
      } else {
        sc_lds[bi] = -INFINITY;
      }
      lane_best(lv, li);
    }
  }
  if (a.top_k <= 64) {
    // ascending: each pick's rank among the k picks (block indices are distinct)
    int rank = 0;
    for (int j = 0; j < k; j++) rank += __builtin_amdgcn_readlane(mine, j) < mine;
    if (lane < k) row[rank] = mine;
    else if (lane < a.top_k) row[lane] = -1;
  } else if (lane == 0) {
    for (int i = 1; i < k; i++) {   // ascending, in LDS
      const int x = picks[i];
      int j = i;
      while (j > 0 && picks[j - 1] > x) {
        picks[j] = picks[j - 1];
        j--;
      }
      picks[j] = x;
    }
    for (int i = 0; i < a.top_k; i++) row[i] = i < k ? picks[i] : -1;
  }
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
  if (nb_wg == 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(block_score_kernel, dim3((unsigned)(a.num_kv * nb_wg)), dim3(kSpThreads), 0,
                     stream, a, scores);
  const size_t pick_lds = a.top_k > 64 ? (size_t)a.top_k * 4 : 0;
  if (a.n_blocks <= 64 * kSelRegs)
    hipLaunchKernelGGL(block_select_kernel<true>, dim3((unsigned)(a.num_kv * a.sub_n)), dim3(64),
                       pick_lds, stream, a, static_cast<const float*>(scores));
  else
    hipLaunchKernelGGL(block_select_kernel<false>, dim3((unsigned)(a.num_kv * a.sub_n)), dim3(64),
                       (size_t)a.n_blocks * 4 + pick_lds, stream, a, static_cast<const float*>(scores));
  return hipGetLastError();
}

}  // namespace qkv
