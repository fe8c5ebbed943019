// attn_q8.hip -- split-K flash decode over the Q8_0 KV cache (gfx950).
//
// Reference semantics: flash_attn_chunk_fused_split_q8 (attention.cuh:2633-2801).
// Query t (absolute position start_pos + t) attends keys [0, start_pos + t] of
// split z's range [z*tps*32, min((z+1)*tps*32, start_pos + t + 1)),
// tps = ceil(ceil(active_end_max/32)/k_splits).  K and V elements decode to
// half(q*d); scores are fp32 sums of fp16 products times `scale`; online
// softmax; the split writes its unnormalised partials (m in natural-log
// units, l, o[256]) in the reference layout.  Merged by attn_merge.hip.
//
// Design (not the reference's): one workgroup of 4 waves per (kv head,
// query, split); each wave takes 32-key tiles.
//   scores  v_mfma_f32_16x16x32_f16 with A = keys (16 per MFMA) decoded in
//           registers from 72 contiguous bytes per lane (two whole Q8 blocks:
//           lane k-group g owns blocks 2g and 2g+1, so the reduction order
//           over dims is permuted identically in both operands) and B = the
//           fp16 query.  D rows = keys, D cols = heads.
//   softmax online per head, base 2, the head's max over the 4 rows through
//           gfx950 row swaps.
//   values  A = the lane's own probabilities (fp16), B = 8 keys x 1 dim.
//           Value rows are staged in LDS as [dim quad][key] dwords plus
//           [block][key] scales; a lane reads one dim quad of 8 keys and
//           decodes it into the B operands of 4 MFMA tiles (tile 4a+e,
//           column n = dim 64a + 4n + e).
// Split API (MODE 1): one workgroup per reference split, partials in the
// reference layout.  Fast path (MODE 0): 128-key chunks (one 32-key tile per
// wave, or a multiple), tagged records and designated mergers in the same
// launch (attn_fastmerge.h); values are not rotated, so the merge ends with a
// plain fp16 store.
// Mixed formats (VTQ3: keys Q8_0, values TQ3, the reference's TQ_KEYS_Q8
// mode, model.cuh:1735-1748, 2323-2333, 2574-2588): the same scores; values
// accumulate sum_t p_t norm_t c[idx_t] in rotated coordinates as in
// attn_tq3.hip (A = p*norm per 128-block, B = centroid pairs from a per-lane
// 64-entry LDS table), and the mergers rotate each output block back.  The
// reference has no fused kernel for this mode: it dequantizes K to fp16 and
// runs the unfused score, softmax and TQ3 value kernels.
#include "qkv_device.h"
#include "attn_common.h"
#include "attn_fastmerge.h"

namespace qkv {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kTile = 32;                      // keys per wave tile
constexpr int kHD = 256;
constexpr int kRowBytes = 288;                 // one kv head of one token: 8 blocks x 36 B
constexpr int kPitch = kTile + 4;              // dwords per staged row of 32 keys

// per-wave staging (dwords): value code quads [64][kPitch], value scales
// [8][kPitch], per-head rescale [16]
constexpr int kStCodes = 0;
constexpr int kStScale = 64 * kPitch;
constexpr int kStCorr = 72 * kPitch;
constexpr int kStageBytes = (72 * kPitch + 16) * 4;
constexpr int kLdsStage = 0;
constexpr int kLdsTotalTile = kLdsStage + kWaves * kStageBytes;
// merge area (aliases the staging): [wave][8 rows][256] f32, then scalars
constexpr int kLdsMergeO = 0;
constexpr int kLdsMergeML = kLdsMergeO + kWaves * 8 * kHD * 4;
constexpr int kLdsMergeEnd = kLdsMergeML + 256 * 4;
constexpr int kLdsTotal = kLdsMergeEnd > kLdsTotalTile ? kLdsMergeEnd : kLdsTotalTile;
// mixed formats: centroid-pair table (entry E = codes E & 7, E >> 3 of lane L
// at byte E * 256 + 4 * L, so each lane reads its own bank), then per-wave
// staging (dwords): value code groups [block j][group g][kPitch] (3 bytes of
// codes, dword-expanded), value block norms [j][kPitch], per-head rescale [16]
constexpr int kTq3RowBytes = 104;              // one kv head of one token: 2 blocks x 52 B
constexpr int kMxStCodes = 0;
constexpr int kMxStNorm = 32 * kPitch;
constexpr int kMxStCorr = 34 * kPitch;
constexpr int kMxStageBytes = (34 * kPitch + 16) * 4;
constexpr int kMxLdsLut = 0;
constexpr int kMxLdsStage = 64 * 64 * 4;
constexpr int kMxLdsTotalTile = kMxLdsStage + kWaves * kMxStageBytes;
constexpr int kMxLdsTotal = kLdsMergeEnd > kMxLdsTotalTile ? kLdsMergeEnd : kMxLdsTotalTile;
constexpr int kMlW0 = 0, kMlLw0 = 8 * kWaves;   // merge scalars: m[w][8], l[w][8], M[8], L[8]
constexpr int kMlM = 16 * kWaves, kMlL = 16 * kWaves + 8;
static_assert(kMlL + 8 <= 256, "merge scalars must fit the ML area");
static_assert(kMlL + 8 <= 256, "merge scalars must fit the ML area");
static_assert(kLdsMergeO + MergeLayout<kThreads>::kRedFloats * 4 <= kLdsMergeML,
              "merger reduction must fit the merge area");

struct TileQ8 {
  uint32_t k[2][18];   // key 16g+col: blocks 2*row and 2*row+1 (qs, pad|d, qs, pad|d)
  u4_t v[9];           // key ts + (lane & 31): blocks 4*(lane>>5) .. +3 (36 dwords);
                       // TQ3 values: 128-block lane>>5 (norm + 12 code dwords in v[0..3])
};

// ts: the tile's first key (wave-uniform); the buffer resources are rebased at
// its row (64-bit byte offsets)
template <bool VTQ3>
__device__ __forceinline__ void load_tile_q8(const AttnArgs& p, int ts, int nkv, int h, int lane,
                                             int row, int col, TileQ8& t) {
  const uint64_t row0 = (uint64_t)(uint32_t)ts * (uint32_t)nkv;
  const __amdgpu_buffer_rsrc_t rk = cache_rsrc(p.k, row0 * kRowBytes, p.kv_bytes);
  const __amdgpu_buffer_rsrc_t rv = VTQ3 ? cache_rsrc(p.v, row0 * kTq3RowBytes, p.v_bytes)
                                         : cache_rsrc(p.v, row0 * kRowBytes, p.kv_bytes);
#pragma unroll
  for (int g = 0; g < 2; g++) {
    const uint32_t off = (uint32_t)((16 * g + col) * nkv + h) * kRowBytes + 72u * row;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const u4_t c = __builtin_amdgcn_raw_buffer_load_b128(rk, off + 16 * i, 0, 0);
#pragma unroll
      for (int e = 0; e < 4; e++) t.k[g][4 * i + e] = c[e];
    }
    const u2_t c = __builtin_amdgcn_raw_buffer_load_b64(rk, off + 64, 0, 0);
    t.k[g][16] = c[0];
    t.k[g][17] = c[1];
  }
  if constexpr (VTQ3) {
    const uint32_t voff =
        (uint32_t)((lane & 31) * nkv + h) * kTq3RowBytes + 52u * (uint32_t)(lane >> 5);
#pragma unroll
    for (int i = 0; i < 3; i++) t.v[i] = __builtin_amdgcn_raw_buffer_load_b128(rv, voff + 16 * i, 0, 0);
    t.v[3][0] = __builtin_amdgcn_raw_buffer_load_b32(rv, voff + 48, 0, 0);
  } else {
    const uint32_t voff =
        (uint32_t)((lane & 31) * nkv + h) * kRowBytes + 144u * (uint32_t)(lane >> 5);
#pragma unroll
    for (int i = 0; i < 9; i++) t.v[i] = __builtin_amdgcn_raw_buffer_load_b128(rv, voff + 16 * i, 0, 0);
  }
}

__device__ __forceinline__ float scale_of(uint32_t pad_d) { return h2f(pad_d >> 16); }

// half(q * d) for the signed byte B of w (the fp32 product is exact)
template <int B>
__device__ __forceinline__ _Float16 dec(uint32_t w, float d) {
  return (_Float16)((float)(int8_t)(w >> (8 * B)) * d);
}

// A operand of score slice s: block s>>2 of the lane's two, elements 8(s&3)..+7
template <int S>
__device__ __forceinline__ h8_t key_operand(const uint32_t (&k)[18]) {
  constexpr int base = 9 * (S >> 2) + 2 * (S & 3);
  const float d = scale_of(k[9 * (S >> 2) + 8]);
  const uint32_t w0 = k[base], w1 = k[base + 1];
  return h8_t{dec<0>(w0, d), dec<1>(w0, d), dec<2>(w0, d), dec<3>(w0, d),
              dec<0>(w1, d), dec<1>(w1, d), dec<2>(w1, d), dec<3>(w1, d)};
}

__device__ __forceinline__ float xrow_max(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float xrow_sum(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Fused append (q8_attn_kernel APPEND): the wave whose tile holds key
// P = start_pos quantizes the new K and V rows of its kv head with the
// arithmetic of q8_append_kernel (attention.cuh:2587-2609): lane l takes
// elements 4l..4l+3 (block l / 8), the block absmax is an xor reduction over
// its 8 lanes, amax / 127 and 1 / scale are IEEE single roundings, codes are
// rint (half to even) clamped to [-128, 127].  Every lane stores its code
// dword to the cache row (lanes 8b also the fp16 scale, with a 16-bit store
// so that pad keeps what the cache held) and to the wave's row image in LDS
// (9 dwords per block: codes, then pad|d with pad 0).  The key registers of
// key P (lane (row, col = P % 16), blocks 2row and 2row + 1 of group
// (P - ts) / 16), loaded from the not yet written row, are replaced from the
// image, and so are key P's staged values.
constexpr int kNewRowDw = 2 * 72;   // K then V image, 8 blocks x 9 dwords each

__device__ __forceinline__ uint32_t q8_new_dword(uint2 hv, int lane, uint8_t* cache,
                                                 uint64_t row_off, uint32_t* img) {
  const float v[4] = {h2f(hv.x & 0xffffu), h2f(hv.x >> 16), h2f(hv.y & 0xffffu), h2f(hv.y >> 16)};
  float amax = fmaxf(fmaxf(__builtin_fabsf(v[0]), __builtin_fabsf(v[1])),
                     fmaxf(__builtin_fabsf(v[2]), __builtin_fabsf(v[3])));
  amax = fmaxf(amax, __shfl_xor(amax, 1));
  amax = fmaxf(amax, __shfl_xor(amax, 2));
  amax = fmaxf(amax, __shfl_xor(amax, 4));
  const float scale = amax / 127.0f;
  const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
  uint32_t word = 0u;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    int q = (int)__builtin_rintf(v[e] * inv);
    q = q > 127 ? 127 : (q < -128 ? -128 : q);
    word |= ((uint32_t)q & 0xffu) << (8 * e);
  }
  const int b = lane >> 3, i = lane & 7;
  const uint32_t d = f2h(scale);
  *reinterpret_cast<uint32_t*>(cache + row_off + 36 * b + 4 * i) = word;
  img[9 * b + i] = word;
  if (i == 0) {
    *reinterpret_cast<uint16_t*>(cache + row_off + 36 * b + 34) = (uint16_t)d;
    img[9 * b + 8] = d << 16;
  }
  return word;
}

// kn, vn: elements 4 lane .. 4 lane + 3 of the new K and V rows of kv head h
// (loaded at kernel start).
__device__ __forceinline__ void append_new_row(const AttnArgs& p, int kp, int h, int lane, int row,
                                               int col, uint2 kn, uint2 vn, uint32_t* img,
                                               TileQ8& t) {
  const uint64_t row_off = ((uint64_t)(uint32_t)p.start_pos * (uint32_t)p.num_kv + h) * kRowBytes;
  q8_new_dword(kn, lane, p.k_w, row_off, img);
  q8_new_dword(vn, lane, p.v_w, row_off, img + 72);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // keys: selects with constant register indices (the group is wave-uniform,
  // the lane is not), so that the tile registers stay registers
  const bool mine = col == (kp & 15), g0 = (kp >> 4) == 0;
  const uint32_t* src = img + 18 * row;
#pragma unroll
  for (int i = 0; i < 18; i++) {
    const uint32_t nv = src[i];
    t.k[0][i] = (mine && g0) ? nv : t.k[0][i];
    t.k[1][i] = (mine && !g0) ? nv : t.k[1][i];
  }
}

// Values of the new key in the staging area ([8 blk + q][key] code dwords,
// [blk][key] scales), over what the lanes of key kp staged from the cache.
__device__ __forceinline__ void stage_new_values(const uint32_t* img, int kp, int lane, float* st,
                                                 uint32_t* stu) {
  const int b = lane >> 3, i = lane & 7;
  stu[kStCodes + (8 * b + i) * kPitch + kp] = img[72 + 9 * b + i];
  if (i == 0) st[kStScale + b * kPitch + kp] = scale_of(img[72 + 9 * b + 8]);
}

template <int MODE, bool VTQ3 = false, bool APPEND = false>
__global__ __launch_bounds__(kThreads, 2) void q8_attn_kernel(QKV_ATTN_LEAD_PARAMS, AttnArgs pin,
                                                              uint16_t* out) {
  QKV_ATTN_LEAD_APPLY(p, pin);
  static_assert(!VTQ3 || MODE == 0, "mixed formats: fast path only");
  static_assert(!APPEND || (MODE == 0 && !VTQ3), "fused append: Q8 fast path only");
  // APPEND: each wave's new-row image follows the tile staging areas
  constexpr int kLdsNewRow = kLdsTotalTile;
  constexpr int kLdsAppend = kLdsNewRow + kWaves * kNewRowDw * 4;
  __shared__ __attribute__((aligned(16)))
  uint8_t lds[VTQ3 ? kMxLdsTotal : (APPEND && kLdsAppend > kLdsTotal ? kLdsAppend : kLdsTotal)];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row = lane >> 4, col = lane & 15;
  const int gqa = p.num_q / p.num_kv;

  int h, t_idx, split, lo, hi;
  bool has_work = true;
  if (MODE == 1) {
    // work id: (kv head, query, split)
    const int L = blockIdx.x;
    h = L % p.num_kv;
    t_idx = (L / p.num_kv) % p.sub_n;
    split = L / (p.num_kv * p.sub_n);
    const int active_end = p.start_pos + t_idx + 1;
    const int total_tiles = (p.active_end_max + 31) / 32;   // attention.cuh:2660-2663
    const int tps = (total_tiles + p.k_splits - 1) / p.k_splits;
    lo = split * tps * 32;
    hi = min((split + 1) * tps * 32, active_end);
  } else {
    // work id (XCD-aware: the num_kv workgroups of one (query, chunk) share an XCD)
    const int L = blockIdx.x;
    const int xcd = L & 7, r = L >> 3;
    h = r % p.num_kv;
    const int g = (r / p.num_kv) * 8 + xcd;
    has_work = g < p.sub_n * p.n_chunks;
    t_idx = has_work ? g / p.n_chunks : 0;
    split = has_work ? g - t_idx * p.n_chunks : 0;
    const int active_end = p.start_pos + t_idx + 1;
    lo = split * p.chunk_keys;
    hi = has_work ? min(lo + p.chunk_keys, active_end) : lo;
  }


  // query operand, slice s: head `col`, dims (2*row + (s>>2))*32 + 8*(s&3) + i
  h8_t qa[8];
#pragma unroll
  for (int s = 0; s < 8; s++) {
    const int dim = (2 * row + (s >> 2)) * 32 + 8 * (s & 3);
    qa[s] = col < gqa ? *reinterpret_cast<const h8_t*>(
                            p.q + ((long)t_idx * p.num_q + h * gqa + col) * kHD + dim)
                      : h8_t{0, 0, 0, 0, 0, 0, 0, 0};
  }

  const float scale2 = p.scale_log2;
  float m2 = -INFINITY, lsum = 0.0f;
  f4_t acc[16];
#pragma unroll
  for (int t = 0; t < 16; t++) acc[t] = f4_t{0.f, 0.f, 0.f, 0.f};
  if constexpr (VTQ3) {
    // centroid-pair table: wave w writes every lane's copy of entries 16w .. 16w+15
    const uint32_t lane4 = 4u * (uint32_t)lane;
#pragma unroll
    for (int k = 0; k < 16; k++) {
      const uint32_t e = 16u * (uint32_t)wave + k;
      *reinterpret_cast<uint32_t*>(lds + kMxLdsLut + e * 256 + lane4) =
          centroid_scaled_h(e & 7u) | (centroid_scaled_h(e >> 3) << 16);
    }
    __syncthreads();
  }
  constexpr int kCorr = VTQ3 ? kMxStCorr : kStCorr;
  float* st = reinterpret_cast<float*>(lds + (VTQ3 ? kMxLdsStage + wave * kMxStageBytes
                                                   : kLdsStage + wave * kStageBytes));
  uint32_t* stu = reinterpret_cast<uint32_t*>(st);

  // fused append: the new rows' elements of this lane, loaded up front by the
  // wave whose tiles include key start_pos
  uint2 new_k = make_uint2(0u, 0u), new_v = make_uint2(0u, 0u);
  if constexpr (APPEND) {
    if (p.start_pos >= lo + wave * kTile && p.start_pos < hi &&
        ((p.start_pos - lo) / kTile) % kWaves == wave) {
      new_k = *reinterpret_cast<const uint2*>(p.k_new + (long)h * kHD + 4 * lane);
      new_v = *reinterpret_cast<const uint2*>(p.v_new + (long)h * kHD + 4 * lane);
    }
  }
  bool first = true;
  for (int ts = lo + wave * kTile; ts < hi; ts += kWaves * kTile) {
    TileQ8 tr;
    load_tile_q8<VTQ3>(p, ts, p.num_kv, h, lane, row, col, tr);
    if constexpr (APPEND) {
      // the new token (sub_n == 1: key start_pos) lies in at most one tile
      // of the kv head; ts is wave-uniform
      if (p.start_pos >= ts && p.start_pos < ts + kTile)
        append_new_row(p, p.start_pos - ts, h, lane, row, col, new_k, new_v,
                       reinterpret_cast<uint32_t*>(lds + kLdsNewRow) + wave * kNewRowDw, tr);
      // (the new key's value registers stay stale: its staged values are
      // replaced from the image below)
    }

    // ---- scores: D rows = keys 16g + 4*row + r, D col = head `col`
    f4_t sa[2];
#pragma unroll
    for (int g = 0; g < 2; g++) {
      f4_t a = {0.f, 0.f, 0.f, 0.f};
      a = __builtin_amdgcn_mfma_f32_16x16x32_f16(key_operand<0>(tr.k[g]), qa[0], a, 0, 0, 0);
      a = __builtin_amdgcn_mfma_f32_16x16x32_f16(key_operand<1>(tr.k[g]), qa[1], a, 0, 0, 0);
      a = __builtin_amdgcn_mfma_f32_16x16x32_f16(key_operand<2>(tr.k[g]), qa[2], a, 0, 0, 0);
      a = __builtin_amdgcn_mfma_f32_16x16x32_f16(key_operand<3>(tr.k[g]), qa[3], a, 0, 0, 0);
      a = __builtin_amdgcn_mfma_f32_16x16x32_f16(key_operand<4>(tr.k[g]), qa[4], a, 0, 0, 0);
      a = __builtin_amdgcn_mfma_f32_16x16x32_f16(key_operand<5>(tr.k[g]), qa[5], a, 0, 0, 0);
      a = __builtin_amdgcn_mfma_f32_16x16x32_f16(key_operand<6>(tr.k[g]), qa[6], a, 0, 0, 0);
      a = __builtin_amdgcn_mfma_f32_16x16x32_f16(key_operand<7>(tr.k[g]), qa[7], a, 0, 0, 0);
      sa[g] = a;
    }

    // ---- value rows to LDS (keys past the range stage as zeros)
    if constexpr (VTQ3) {
      // lane (key kl, block j): its norm and code groups 0..15 (bytes 3g..3g+2)
      const int kl = lane & 31, j = lane >> 5;
      const bool live = ts + kl < hi;
      uint32_t d[14];
#pragma unroll
      for (int i = 0; i < 3; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) d[4 * i + e] = tr.v[i][e];
      d[12] = tr.v[3][0];
      d[13] = 0u;
      st[kMxStNorm + j * kPitch + kl] = live ? __uint_as_float(d[0]) : 0.f;
#pragma unroll
      for (int g = 0; g < 16; g++) {
        const int w = 1 + ((3 * g) >> 2), sh = (3 * g) & 3;
        stu[kMxStCodes + (16 * j + g) * kPitch + kl] = sh ? __builtin_amdgcn_alignbyte(d[w + 1], d[w], sh) : d[w];
      }
    } else {
      const int kl = lane & 31, hf = lane >> 5;
      const bool live = ts + kl < hi;
#pragma unroll
      for (int b = 0; b < 4; b++) {
        const int blk = 4 * hf + b;
        uint32_t w[9];
#pragma unroll
        for (int i = 0; i < 9; i++) w[i] = live ? tr.v[(9 * b + i) >> 2][(9 * b + i) & 3] : 0u;
#pragma unroll
        for (int q = 0; q < 8; q++) stu[kStCodes + (8 * blk + q) * kPitch + kl] = w[q];
        st[kStScale + blk * kPitch + kl] = scale_of(w[8]);
      }
      if constexpr (APPEND) {
        if (p.start_pos >= ts && p.start_pos < ts + kTile)
          stage_new_values(reinterpret_cast<const uint32_t*>(lds + kLdsNewRow) + wave * kNewRowDw,
                           p.start_pos - ts, lane, st, stu);
      }
    }
    wave_sync();

    float s[2][4];
#pragma unroll
    for (int g = 0; g < 2; g++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int key = ts + 16 * g + 4 * row + r;
        s[g][r] = key < hi ? sa[g][r] * scale2 : -INFINITY;
      }

    // ---- online softmax of head `col`
    float mt = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                     fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
    mt = xrow_max(mt);
    const float mn = fmaxf(m2, mt);
    const float msafe = (mn == -INFINITY) ? 0.0f : mn;
    const float corr = __builtin_amdgcn_exp2f(m2 - msafe);
    float ps = 0.0f;
#pragma unroll
    for (int g = 0; g < 2; g++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        s[g][r] = __builtin_amdgcn_exp2f(s[g][r] - msafe);
        ps += s[g][r];
      }
    lsum = lsum * corr + ps;
    m2 = mn;
    if (!first) {
      if (row == 0) st[kCorr + col] = corr;
      wave_sync();
      const f4_t cr = *reinterpret_cast<const f4_t*>(st + kCorr + 4 * row);
#pragma unroll
      for (int t = 0; t < 16; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) acc[t][r] *= cr[r];
    }
    first = false;

    // ---- values: k index i <-> key 4*row + i (i < 4), 16 + 4*row + (i - 4)
    if constexpr (VTQ3) {
      // tile 8a+e, column col: dim 128a + 8col + e (code group col of block a);
      // A = p * block norm, B = centroids of that dim for the 8 keys
      const uint32_t lane4 = 4u * (uint32_t)lane;
#pragma unroll
      for (int a = 0; a < 2; a++) {
        const f4_t na = *reinterpret_cast<const f4_t*>(st + kMxStNorm + a * kPitch + 4 * row);
        const f4_t nb = *reinterpret_cast<const f4_t*>(st + kMxStNorm + a * kPitch + 16 + 4 * row);
        h8_t pv;
#pragma unroll
        for (int r = 0; r < 4; r++) {
          pv[r] = (_Float16)(s[0][r] * na[r]);
          pv[4 + r] = (_Float16)(s[1][r] * nb[r]);
        }
        const u4_t xa = *reinterpret_cast<const u4_t*>(stu + kMxStCodes + (16 * a + col) * kPitch + 4 * row);
        const u4_t xb =
            *reinterpret_cast<const u4_t*>(stu + kMxStCodes + (16 * a + col) * kPitch + 16 + 4 * row);
        const uint32_t x[8] = {xa[0], xa[1], xa[2], xa[3], xb[0], xb[1], xb[2], xb[3]};
        // keys (2k, 2k + 1) interleaved per dim: field 6d of z[k] holds the two
        // codes of dim 2d, field 6d + 3 of z[4 + k] those of dim 2d + 1, so a
        // table entry is a B dword (key 2k low half, key 2k + 1 high half)
        constexpr uint32_t kEven = 0x1C71C7u;   // dims 0, 2, 4, 6 of a code group
        uint32_t z[8];
#pragma unroll
        for (int k = 0; k < 4; k++) {
          const uint32_t hi = x[2 * k + 1] << 3;
          uint32_t e0, e1;
          asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(e0) : "s"(kEven), "v"(x[2 * k]), "v"(hi));
          asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(e1) : "s"(kEven << 3), "v"(x[2 * k]), "v"(hi));
          z[k] = e0;
          z[4 + k] = e1;
        }
#pragma unroll
        for (int pp = 0; pp < 4; pp++) {   // dims 2pp (e = 0) and 2pp + 1 (e = 1)
#pragma unroll
          for (int e = 0; e < 2; e++) {
            u4_t bv;
#pragma unroll
            for (int k2 = 0; k2 < 4; k2++)
              bv[k2] = *reinterpret_cast<const uint32_t*>(
                  lds + kMxLdsLut + ((((z[4 * e + k2] >> (6 * pp + 3 * e)) & 63u) << 8) | lane4));
            acc[8 * a + 2 * pp + e] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                pv, __builtin_bit_cast(h8_t, bv), acc[8 * a + 2 * pp + e], 0, 0, 0);
          }
        }
      }
    } else {
    h8_t pa;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      pa[r] = (_Float16)s[0][r];
      pa[4 + r] = (_Float16)s[1][r];
    }
#pragma unroll
    for (int a = 0; a < 4; a++) {
      const int dq = 16 * a + col;          // dims 4*dq .. 4*dq+3
      const int blk = dq >> 3;
      const u4_t xa = *reinterpret_cast<const u4_t*>(stu + kStCodes + dq * kPitch + 4 * row);
      const u4_t xb = *reinterpret_cast<const u4_t*>(stu + kStCodes + dq * kPitch + 16 + 4 * row);
      const f4_t da = *reinterpret_cast<const f4_t*>(st + kStScale + blk * kPitch + 4 * row);
      const f4_t db = *reinterpret_cast<const f4_t*>(st + kStScale + blk * kPitch + 16 + 4 * row);
      const uint32_t x[8] = {xa[0], xa[1], xa[2], xa[3], xb[0], xb[1], xb[2], xb[3]};
      const float d[8] = {da[0], da[1], da[2], da[3], db[0], db[1], db[2], db[3]};
#pragma unroll
      for (int e = 0; e < 4; e++) {
        h8_t b;
#pragma unroll
        for (int i = 0; i < 8; i++) b[i] = (_Float16)((float)(int8_t)(x[i] >> (8 * e)) * d[i]);
        acc[4 * a + e] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, b, acc[4 * a + e], 0, 0, 0);
      }
    }
    }
    wave_sync();
  }
  lsum = xrow_sum(lsum);

  // ---- merge the waves in LDS, then write the split's partials
  __syncthreads();
  float* mo = reinterpret_cast<float*>(lds + kLdsMergeO);
  float* ml = reinterpret_cast<float*>(lds + kLdsMergeML);
  if (VTQ3 && 4 * row < gqa) {
    // tile 8a+e, row 4*row+r (head), column col: dim 128a + 8*col + e
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
      for (int r = 0; r < 4; r++)
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
          const int t = 8 * a + 4 * hh;
          f4_t v4 = {acc[t][r], acc[t + 1][r], acc[t + 2][r], acc[t + 3][r]};
          *reinterpret_cast<f4_t*>(&mo[(wave * 8 + 4 * row + r) * kHD + 128 * a + 8 * col + 4 * hh]) = v4;
        }
  } else if (4 * row < gqa) {
    // tile 4a+e, row 4*row+r (head), column col: dim 64a + 4*col + e
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        f4_t v4 = {acc[4 * a][r], acc[4 * a + 1][r], acc[4 * a + 2][r], acc[4 * a + 3][r]};
        *reinterpret_cast<f4_t*>(&mo[(wave * 8 + 4 * row + r) * kHD + 64 * a + 4 * col]) = v4;
      }
  }
  if (row == 0 && col < 8) {
    ml[kMlW0 + wave * 8 + col] = m2;
    ml[kMlLw0 + wave * 8 + col] = lsum;
  }
  __syncthreads();
  const int rows = min(gqa, 8);
  for (int idx = threadIdx.x; idx < rows * 64; idx += kThreads) {
    const int r = idx >> 6, d4 = (idx & 63) * 4;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; w++) M = fmaxf(M, ml[kMlW0 + w * 8 + r]);
    float Ls = 0.f;
    f4_t o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < kWaves; w++) {
      const float mw = ml[kMlW0 + w * 8 + r];
      const float wt = (mw == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
      Ls += wt * ml[kMlLw0 + w * 8 + r];
      o += wt * *reinterpret_cast<const f4_t*>(&mo[(w * 8 + r) * kHD + d4]);
    }
    if (MODE == 1) {
      const int qh = h * gqa + r;
      const long mlx = ((long)qh * p.sub_n_max + t_idx) * p.k_splits + split;
#pragma unroll
      for (int i = 0; i < 4; i++) p.part_o[mlx * kHD + d4 + i] = o[i];
      if (d4 == 0) {
        p.part_m[mlx] = (M == -INFINITY) ? -INFINITY : M * kLn2;
        p.part_l[mlx] = Ls;
      }
    } else {
      // merged row into the wave-0 slot (this thread's own elements), M and L
      // beside it, for the records
      *reinterpret_cast<f4_t*>(&mo[r * kHD + d4]) = o;
      if (d4 == 0) {
        ml[kMlM + r] = M;
        ml[kMlL + r] = Ls;
      }
    }
  }
  if (MODE == 1) return;

  // ---- fast path: tagged records, designated mergers
  __syncthreads();
  const __amdgpu_buffer_rsrc_t rml =
      __builtin_amdgcn_make_buffer_rsrc(p.ws_ml, 0, p.ws_ml_bytes, kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t ro =
      __builtin_amdgcn_make_buffer_rsrc(p.ws_o, 0, p.ws_o_bytes, kBufferRsrcWord3);
  if (has_work)
    store_records<kThreads>(mo, ml + kMlM, ml + kMlL, p, rml, ro, h, t_idx, rows, split);
  merge_phase<kThreads, VTQ3>(reinterpret_cast<float*>(lds + kLdsMergeO),
                               reinterpret_cast<f2_t*>(lds + kLdsMergeML), p, rml, ro, out);
}

}  // namespace

hipError_t launch_q8_attn_split(const AttnArgs& a, hipStream_t stream) {
  const int n_wg = a.num_kv * a.sub_n * a.k_splits;
  hipLaunchKernelGGL((q8_attn_kernel<1>), dim3(n_wg), dim3(kThreads), 0, stream, QKV_ATTN_LEAD_ARGS(a), a, nullptr);
  return hipGetLastError();
}

hipError_t launch_q8_attn_fast(const AttnArgs& a, uint16_t* out, hipStream_t stream) {
  const int groups = a.sub_n * a.n_chunks;
  const int n_wg = ((groups + 7) / 8) * 8 * a.num_kv;
  hipLaunchKernelGGL((q8_attn_kernel<0>), dim3(n_wg), dim3(kThreads), 0, stream, QKV_ATTN_LEAD_ARGS(a), a, out);
  return hipGetLastError();
}

hipError_t launch_q8_attn_fast_append(const AttnArgs& a, uint16_t* out, hipStream_t stream) {
  const int groups = a.sub_n * a.n_chunks;
  const int n_wg = ((groups + 7) / 8) * 8 * a.num_kv;
  hipLaunchKernelGGL((q8_attn_kernel<0, false, true>), dim3(n_wg), dim3(kThreads), 0, stream, QKV_ATTN_LEAD_ARGS(a), a, out);
  return hipGetLastError();
}

hipError_t launch_q8k_tq3v_attn_fast(const AttnArgs& a, uint16_t* out, hipStream_t stream) {
  const int groups = a.sub_n * a.n_chunks;
  const int n_wg = ((groups + 7) / 8) * 8 * a.num_kv;
  hipLaunchKernelGGL((q8_attn_kernel<0, true>), dim3(n_wg), dim3(kThreads), 0, stream, QKV_ATTN_LEAD_ARGS(a), a, out);
  return hipGetLastError();
}

}  // namespace qkv
