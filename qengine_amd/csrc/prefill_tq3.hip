// prefill_tq3.hip -- chunked-prefill and multi-token-verify attention over the
// packed TQ3 cache (gfx950).
//
// Reference semantics (model.cuh:5163-5214, 5256-5330, 5680-5721;
// attention.cuh:1690-1831 and 1837-1891): a chunk of n_tok new tokens at
// positions start_pos .. start_pos + n_tok - 1 attends causally to the cache
// history [0, start_pos), which the reference first dequantizes in bulk to an
// fp16 scratch (tq3_dequantize_kernel, turboquant.cuh:169-200), and to the
// chunk's own keys and values in fp16 as the projections produced them (not
// quantized).  Query token t sees keys 0 .. start_pos + t.  Scores are fp32
// sums of fp16 products, softmax in fp32, the output fp16.  In verify mode the
// block's own rows are read back from the cache, quantized (model.cuh:
// 4566-4571).
//
// The attention reproduces those numerics: every history element is the fp16
// value the reference's dequantization produces (bit for bit), the query and
// the chunk's keys and values are used as given, products are exact fp16 x
// fp16 in fp32, sums fp32.  The only rounding of this build's own is the fp16
// probability in the value MFMA (2^-12 relative per weight).
//
//   prefill_stage_kernel  the history's K and V blocks dequantized with the
//                         reference arithmetic (fp32 centroids, the WHT
//                         butterflies stage by stage, * rs, sign, * norm,
//                         fp16), then the chunk's own fp16 K and V; keys to
//                         kx [kv head][row][256], values to 64-key tiles
//                         vt [kv head][tile][256 dims][64] in the key order
//                         the value MFMA consumes.  The history is padded to a
//                         multiple of 64 rows, the chunk follows; pad rows are
//                         zero.
//   prefill_attn_kernel   one workgroup per (kv head, 64 query tokens, key
//                         split) -- two per kv head for GQA 6, three heads
//                         each -- and one wave per (query head, 32 tokens);
//                         chunks of at most 32 tokens take 32-token
//                         workgroups, two per CU.  Per 32-key tile (keys
//                         [key][dim], values [dim][key] in LDS, shared by the
//                         64 x GQA query rows of the workgroup):
//                           S^T  = K Q^T       v_mfma_f32_32x32x16_f16, M = keys
//                           O^T += V^T P^T     M = dims, N = query tokens
//                         so every lane owns one query row (token lane % 32)
//                         for the softmax and the accumulators.  Workgroups
//                         that stream the same tiles run on one XCD (shared L2).
//   prefill_merge_kernel  merges the key splits (log-sum-exp) and stores fp16
//                         (prefill_merge_wide_kernel when there are many splits).
#include <algorithm>

#include "qkv_device.h"
#include "attn_common.h"
#include "qkv_launch.h"

namespace qkv {
namespace {

typedef float f16x_t __attribute__((ext_vector_type(16)));

constexpr int kHD = 256;
constexpr int kKeys = 64;                 // row granule of the staged K / V (stage tiles)
constexpr int kTK = 32;                   // keys per attention tile
constexpr int kWaveToks = 32;             // query tokens per wave (the MFMA N dimension)

// Token groups of a workgroup: two (64 tokens, 8 waves at GQA 4, one
// workgroup per CU) when the chunk has more than 32 tokens, else one (two
// workgroups per CU).  Every tile a workgroup loads serves all its query rows,
// so 64-token workgroups move half the L2 -> LDS bytes per MFMA of 32-token
// ones (config 5(i): 3.94 against 4.23-4.41 ms per chunk, bit-identical).
__host__ __device__ inline int prefill_token_groups(int n_tok) { return n_tok > kWaveToks ? 2 : 1; }

// LDS of the attention (bytes): two tile buffers, each keys [32][512 B] then
// values [256 dims][64 B]; 64 KB per workgroup, so two one-group workgroups
// share a CU and the matrix core of one overlaps the softmax of the other.  16-byte
// chunks are XOR-swizzled so that the MFMA operand reads (16 lanes per LDS
// cycle, 16 consecutive rows at one logical chunk) hit 16 different 16-byte
// bank groups: key row r holds chunk c at c ^ (r & 15), value row d holds
// chunk c at c ^ ((d >> 2) & 3).  The tiles arrive by direct global-to-LDS
// loads (buffer_load_dwordx4 ... lds: lane l of an instruction writes bytes
// 16l .. 16l+15 of a 1 KB run; each lane fetches the chunk that lands there).
constexpr int kKBytes = kTK * kHD * 2;                // 16 KB
constexpr int kVBytes = kHD * kTK * 2;                // 16 KB
constexpr int kBufBytes = kKBytes + kVBytes;
constexpr int kLdsBytes = 2 * kBufBytes;
static_assert(2 * kLdsBytes <= 160 * 1024, "two one-group prefill workgroups must fit one CU");

typedef __attribute__((address_space(3))) void lds_void_t;

// Value order inside a 32-key half: key 8a + 4h + c sits at position
// 16(a/2) + 8h + 4(a%2) + c, so the 8 keys one lane contributes to a value
// MFMA (its own probabilities, in the score D layout) are contiguous.
__device__ __forceinline__ int value_pos(int key32) {
  const int a = key32 >> 3, h = (key32 >> 2) & 1, c = key32 & 3;
  return 16 * (a >> 1) + 8 * h + 4 * (a & 1) + c;
}

// Placement of the attention workgroups: the qtiles of one pair (kv head,
// head group, key split) stream the same tiles, so they go to consecutive
// slots of `span` XCDs (a power of two, 32 slots -- one per CU -- each);
// workgroup L runs on XCD L % 8.
struct Placement {
  int span, per, pairs_per_round, subs;
};
__host__ __device__ inline Placement placement(int qtiles, int pairs) {
  int want = (qtiles + 31) / 32, span = 1;
  while (span < want && span < 8) span *= 2;
  Placement pl;
  pl.span = span;
  pl.per = (qtiles + span - 1) / span;
  pl.pairs_per_round = 8 / span;
  pl.subs = (pairs + pl.pairs_per_round - 1) / pl.pairs_per_round;
  return pl;
}

}  // namespace

// ---------------------------------------------------------------------------
// staging: one workgroup per (kv head, 64-row tile).  Units (tensor, row,
// 128-block) of 16 lanes; lane `part` of a unit owns elements part*8 ..
// part*8+7.  Keys go straight to their kx row; values are transposed through
// LDS ([dim][value position], 132-byte dim pitch: 2-way banks on the 2-byte
// stores) and leave as whole 16-byte pieces of the two 32-key tiles
// vt [kv head][row / 32][256 dims][32].
// ---------------------------------------------------------------------------
constexpr int kStVPitch = 132;   // bytes per staged value dim row (64 keys fp16 + 4)

__global__ __launch_bounds__(256) void prefill_stage_kernel(PrefillArgs p, const uint16_t* k,
                                                            const uint16_t* v) {
  __shared__ __attribute__((aligned(16))) uint8_t vt_lds[kHD * kStVPitch];
  __shared__ float cent[8];
  const int tid = threadIdx.x, part = tid & 15;
  tq3_centroid_table(cent, tid);
  const Tq3LaneConst lc = tq3_lane_const(part);
  __syncthreads();
  const long rows = (long)p.h_pad + p.n_pad;
  const int tiles = (int)(rows / kKeys);
  const int h = blockIdx.x / tiles, tile = blockIdx.x - h * tiles;
  // 256 units: tensor (K: 0..127, V: 128..255), row r = (u & 127) >> 1, block u & 1
  for (int u = tid >> 4; u < 256; u += 16) {
    const int tv = u >> 7, r = (u & 127) >> 1, blk = u & 1;
    const int row = tile * kKeys + r;
    const int dim0 = blk * 128 + part * 8;
    uint32_t pk[4] = {0u, 0u, 0u, 0u};   // pad rows stay zero
    if (row < p.hist) {
      // history: the reference's dequantization (turboquant.cuh:169-200)
      tq3_group_dequant(tq3_group_load(reinterpret_cast<const uint8_t*>(tv ? p.v_cache : p.k_cache) +
                                           ((uint64_t)(uint32_t)row * (uint32_t)p.num_kv + h) * 104u +
                                           blk * 52u, part),
                        part, cent, lc, pk);
    } else if (row >= p.h_pad && row - p.h_pad < p.n_tok) {
      // the chunk's own keys / values, as given
      const uint16_t* src = (tv ? v : k) + ((long)(row - p.h_pad) * p.num_kv + h) * kHD + dim0;
      const uint4 raw = *reinterpret_cast<const uint4*>(src);
      pk[0] = raw.x;
      pk[1] = raw.y;
      pk[2] = raw.z;
      pk[3] = raw.w;
    }
    if (!tv) {
      *reinterpret_cast<uint4*>(p.kx + ((long)h * rows + row) * kHD + dim0) =
          make_uint4(pk[0], pk[1], pk[2], pk[3]);
    } else {
      const int pos = (r >> 5) * 32 + value_pos(r & 31);
#pragma unroll
      for (int i = 0; i < 8; i++)
        *reinterpret_cast<uint16_t*>(vt_lds + (dim0 + i) * kStVPitch + pos * 2) =
            (uint16_t)((pk[i >> 1] >> (16 * (i & 1))) & 0xffffu);
    }
  }
  __syncthreads();
  // the two 32-key value tiles: 2 x 256 dims x 64 bytes = 2048 16-byte pieces, 8 per thread
  uint4* dst = reinterpret_cast<uint4*>(p.vt + ((long)h * tiles + tile) * kHD * kKeys);
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const int piece = i * 256 + tid, half = piece >> 10, dim = (piece >> 2) & 255, q = piece & 3;
    const uint32_t* src = reinterpret_cast<const uint32_t*>(vt_lds + dim * kStVPitch + half * 64 + q * 16);
    dst[piece] = make_uint4(src[0], src[1], src[2], src[3]);
  }
}

// ---------------------------------------------------------------------------
// attention: 1-D grid (placement above); WAVES query heads of one kv head and
// TG groups of 32 query tokens per workgroup, one wave per (head, group)
// ---------------------------------------------------------------------------
template <int WAVES, int TG, bool FROM_CACHE>
__global__ __launch_bounds__(64 * WAVES * TG, TG == 1 ? 2 : 1) void prefill_attn_kernel(
    PrefillArgs p, const uint16_t* q) {
  constexpr int kToks = kWaveToks * TG;   // query tokens per workgroup
  __shared__ __attribute__((aligned(16))) uint8_t lds[kLdsBytes];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wave = wv % WAVES, tg = wv / WAVES;   // query head, token group
  const int hh = lane >> 5;          // k-group of the MFMA operands / row group of D
  const int tok = lane & 31;         // query token (MFMA N index) of this lane
  const int gqa = p.num_q / p.num_kv;
  const int groups = gqa / WAVES;            // workgroups per kv head
  const int qtiles = (p.n_tok + kToks - 1) / kToks;
  const int pairs = p.num_kv * groups * p.n_split;

  // ---- (pair, qtile) of this workgroup
  int pair, qt;
  {
    const Placement pl = placement(qtiles, pairs);
    const int L = blockIdx.x, xcd = L & 7, r = L >> 3;
    const int sub = r / pl.per, j = r - sub * pl.per;
    pair = sub * pl.pairs_per_round + xcd / pl.span;
    qt = (xcd % pl.span) * pl.per + j;
    if (qt >= qtiles || pair >= pairs || xcd / pl.span >= pl.pairs_per_round) return;
  }
  const int z = pair % p.n_split;
  const int hg_all = pair / p.n_split;                 // kv head * groups + head group
  const int h = hg_all / groups, hg = hg_all - h * groups;
  const int t0 = qt * kToks;
  const int n_q = min(kToks, p.n_tok - t0);
  const int t0w = t0 + kWaveToks * tg;              // this wave's first token
  const int n_qw = min(kWaveToks, p.n_tok - t0w);   // <= 0: a group past the last token
  const int qh = h * gqa + hg * WAVES + wave;

  // 32-key tiles: history rows [0, h_pad) then (unless every key comes from
  // the cache) the chunk's own keys [0, t0 + n_q)
  const int th = p.h_pad / kTK;
  const int tc = FROM_CACHE ? 0 : (t0 + n_q + kTK - 1) / kTK;
  const int total = th + tc;
  const int tps = (total + p.n_split - 1) / p.n_split;
  const int tlo = min(total, z * tps), thi = min(total, tlo + tps);
  const long rows = (long)p.h_pad + p.n_pad;

  // ---- query of (token t0 + tok, head qh): B operands, slice s of block b
  h8_t qb[2][8];
  {
    const uint32_t qbytes = (uint32_t)((long)p.n_tok * p.num_q * kHD * 2);
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(q), 0, qbytes, kBufferRsrcWord3);
    const uint32_t base = tok < n_qw ? (uint32_t)((((long)(t0w + tok) * p.num_q + qh) * kHD) * 2) : qbytes;
#pragma unroll
    for (int b = 0; b < 2; b++)
#pragma unroll
      for (int s = 0; s < 8; s++)
        qb[b][s] = __builtin_bit_cast(
            h8_t, __builtin_amdgcn_raw_buffer_load_b128(rq, base + (b * 128 + 16 * s + 8 * hh) * 2, 0, 0));
  }

  // ---- tile loads: one buffer resource per tensor of this kv head (kx rows
  // and vt tiles share the head stride), the tile offset in the scalar offset;
  // 16 loads of 1 KB per tensor and tile, spread over the waves (with 3 or 6
  // waves the last wave repeats load 15, which writes the same bytes).
  const uint32_t head_bytes = (uint32_t)(rows * kHD * 2);
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(p.kx) + (long)h * rows * kHD, 0, head_bytes, kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(p.vt) + (long)h * rows * kHD, 0, head_bytes, kBufferRsrcWord3);
  constexpr int kLoads = (16 + WAVES * TG - 1) / (WAVES * TG);
  // load j: key rows 2j, 2j+1 (lane l: row 2j + l/32, slot l%32) and value
  // dims 16j .. 16j+15 (lane l: dim 16j + l/4, slot l%4); the value offset
  // within the run does not depend on j
  const int v_off = (lane >> 2) * (kTK * 2) + (((lane & 3) ^ ((lane >> 4) & 3)) * 16);
  // key offset of load j: row 2j + hi, slot l%32 holds chunk (l%32) ^ (row & 15);
  // (2j + hi) & 15 = (2j & 15) ^ hi, so the offset is k_base ^ 16 * (2j & 15).
  // Formed per load (one XOR; kept out of the registers across the tile loop).
  const int k_base = (lane >> 5) * (kHD * 2) + (((lane & 31) ^ (lane >> 5)) * 16);
  auto issue = [&](int ti, int buf) {
    uint8_t* base = lds + buf * kBufBytes;
#pragma unroll
    for (int jj = 0; jj < kLoads; jj++) {
      const int j = min(wv + jj * WAVES * TG, 15);
      int k_off;
      asm volatile("v_xor_b32 %0, %1, %2" : "=v"(k_off) : "s"(16 * ((2 * j) & 15)), "v"(k_base));
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void_t*)(base + j * 1024), 16, k_off,
                                               ti * kKBytes + j * 1024, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_void_t*)(base + kKBytes + j * 1024), 16, v_off,
                                               ti * kVBytes + j * 1024, 0, 0);
    }
  };

  f16x_t acc[8];
#pragma unroll
  for (int d = 0; d < 8; d++) acc[d] = f16x_t{};
  float m2 = -INFINITY, lsum = 0.0f;
  const int t_abs = t0w + tok;       // this lane's token index in the chunk
  const int lim_hist = FROM_CACHE ? min(p.hist, p.start_pos + t_abs + 1) : p.hist;
  // a negative scale is carried by the query (an exact fp16 sign flip), so
  // that the row maximum of the raw scores gives the maximum of the scaled ones
  float sl = p.scale_log2;
  if (sl < 0.0f) {
#pragma unroll
    for (int b = 0; b < 2; b++)
#pragma unroll
      for (int s = 0; s < 8; s++) qb[b][s] = -qb[b][s];
    sl = -sl;
  }
  // The weights are taken against a reference maximum m2 that is raised (and
  // the accumulators rescaled) only when some row's maximum exceeds it by
  // more than kSlack (log2 units): the weights stay below 2^kSlack, inside fp16.
  constexpr float kSlack = 12.0f;
  // operand addresses (bytes within a tile buffer) of this lane
  const int k_row = tok * (kHD * 2);
  const int v_row = tok * (kTK * 2);

  if (tlo < thi) issue(tlo, 0);
  for (int ti = tlo; ti < thi; ti++) {
    const int buf = (ti - tlo) & 1;
    // visible keys of this tile for this lane: tile key index < lim
    const int lim = ti < th ? lim_hist - ti * kTK : t_abs + 1 - (ti - th) * kTK;
    // tile ti has landed (each wave waits for its own loads, then the
    // barrier), and every wave is done with the other buffer's tile
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (ti + 1 < thi) issue(ti + 1, buf ^ 1);
    const uint8_t* kbuf = lds + buf * kBufBytes;
    const uint8_t* vbuf = kbuf + kKBytes;

    // ---- scores S^T = K Q^T: row = key 8(v/4) + 4hh + v%4, column = token.
    // Operand i (block i / 8, slice i % 8) is the logical chunk
    // 16(i/8) + hh + 2(i%8) (dims 128(i/8) + 8hh + 16(i%8)) of key row tok;
    // four reads stay in flight ahead of the MFMAs.
    auto k_operand = [&](int i) {
      const int slot = (i >> 3) * 16 + ((hh + 2 * (i & 7)) ^ (tok & 15));
      return *reinterpret_cast<const h8_t*>(kbuf + k_row + slot * 16);
    };
    f16x_t sd = f16x_t{};
    h8_t ka[4];
#pragma unroll
    for (int i = 0; i < 4; i++) ka[i] = k_operand(i);
#pragma unroll
    for (int i = 0; i < 16; i++) {
      sd = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[i & 3], qb[i >> 3][i & 7], sd, 0, 0, 0);
      if (i + 4 < 16) ka[i & 3] = k_operand(i + 4);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);     // four reads ahead
#pragma unroll
    for (int i = 0; i < 12; i++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA i
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // read i + 4
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    // Row maximum (scaled).  Tiles every row sees whole keep the raw scores
    // (scaled inside the exponent); the others are scaled and masked here.
    float mt = -INFINITY, sl_w;
    if (__builtin_amdgcn_ballot_w64(lim < kTK) == 0) {
#pragma unroll
      for (int v = 0; v < 16; v++) mt = fmaxf(mt, sd[v]);
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt), false, false);
      mt = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * sl;
      sl_w = sl;
    } else {
      const int lim_h = lim - 4 * hh;
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const float sv = 8 * (v >> 2) + (v & 3) < lim_h ? sd[v] * sl : -INFINITY;
        sd[v] = sv;
        mt = fmaxf(mt, sv);
      }
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt), false, false);
      mt = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
      sl_w = 1.0f;
    }
    if (__builtin_amdgcn_ballot_w64(mt > m2 + kSlack) != 0) {
      const float mn = fmaxf(m2, mt);
      const float corr = (mn == -INFINITY) ? 1.0f : __builtin_amdgcn_exp2f(m2 - mn);
      lsum *= corr;
#pragma unroll
      for (int d = 0; d < 8; d++) acc[d] *= corr;
      m2 = mn;
    }
    const float msafe = (m2 == -INFINITY) ? 0.0f : m2;
    // ---- values O^T += V^T P^T.  B operand sg: the weights v = 8sg .. 8sg+7
    // (keys 16sg + 8hh .. in value order), fp16; the row sum takes them as used.
#pragma unroll
    for (int sg = 0; sg < 2; sg++) {
      h8_t pb;
#pragma unroll
      for (int i = 0; i < 8; i++) pb[i] = (_Float16)__builtin_amdgcn_exp2f(__builtin_fmaf(sd[8 * sg + i], sl_w, -msafe));
#pragma unroll
      for (int i = 0; i < 8; i++) lsum += (float)pb[i];
      const int slot = (2 * sg + hh) ^ ((tok >> 2) & 3);
#pragma unroll
      for (int d = 0; d < 8; d++) {
        const h8_t a = *reinterpret_cast<const h8_t*>(vbuf + d * 32 * (kTK * 2) + v_row + slot * 16);
        acc[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb, acc[d], 0, 0, 0);
      }
    }
  }

  // ---------------- partials of this split: m (log2 units), l, o
  {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(lsum), __float_as_uint(lsum), false, false);
    lsum = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
  if (tok < n_qw) {
    const long row = ((long)z * p.n_tok + t0w + tok) * p.num_q + qh;
    float* po = p.part_o + row * kHD;
#pragma unroll
    for (int d = 0; d < 8; d++)
#pragma unroll
      for (int a = 0; a < 4; a++)
        *reinterpret_cast<f4_t*>(po + d * 32 + 8 * a + 4 * hh) =
            f4_t{acc[d][4 * a], acc[d][4 * a + 1], acc[d][4 * a + 2], acc[d][4 * a + 3]};
    if (hh == 0) *reinterpret_cast<f2_t*>(p.part_ml + 2 * row) = f2_t{m2, lsum};
  }
}

// ---------------------------------------------------------------------------
// merge of the key splits and fp16 store: 32 threads per row, 8 dims each
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillArgs p, uint16_t* out) {
  const long row = (long)blockIdx.x * 8 + (threadIdx.x >> 5);   // t * num_q + qh
  if (row >= (long)p.n_tok * p.num_q) return;
  const int d0 = (threadIdx.x & 31) * 8;
  const long nrows = (long)p.n_tok * p.num_q;
  float M = -INFINITY;
  for (int z = 0; z < p.n_split; z++) {
    const f2_t ml = *reinterpret_cast<const f2_t*>(p.part_ml + 2 * (z * nrows + row));
    if (ml[1] > 0.f) M = fmaxf(M, ml[0]);
  }
  float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float L = 0.f;
  for (int z = 0; z < p.n_split; z++) {
    const f2_t ml = *reinterpret_cast<const f2_t*>(p.part_ml + 2 * (z * nrows + row));
    if (!(ml[1] > 0.f)) continue;
    const float w = __builtin_amdgcn_exp2f(ml[0] - M);
    L += w * ml[1];
    const float* po = p.part_o + (z * nrows + row) * kHD + d0;
    const f4_t a = *reinterpret_cast<const f4_t*>(po);
    const f4_t b = *reinterpret_cast<const f4_t*>(po + 4);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      x[i] += w * a[i];
      x[4 + i] += w * b[i];
    }
  }
  const float inv = L > 0.f ? 1.0f / L : 0.f;
  uint32_t pk[4];
#pragma unroll
  for (int i = 0; i < 4; i++) pk[i] = f2h(x[2 * i] * inv) | (f2h(x[2 * i + 1] * inv) << 16);
  *reinterpret_cast<uint4*>(out + row * kHD + d0) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
// Many key splits (verify mode: up to 512): one workgroup per (token, q head)
// row.  The split maxima and weights are reduced across the workgroup first;
// then 8 groups of 32 threads take every 8th split (8 dims per thread, the
// loads of a group's splits independent of each other), and the groups' sums
// meet in LDS.
constexpr int kMergeMaxSplits = 512;
__global__ __launch_bounds__(256) void prefill_merge_wide_kernel(PrefillArgs p, uint16_t* out) {
  __shared__ float w_s[kMergeMaxSplits];
  __shared__ float red[8][kHD];
  __shared__ float stat[2][4];
  const long row = blockIdx.x;   // t * num_q + qh
  const long nrows = (long)p.n_tok * p.num_q;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float m = -INFINITY;
  for (int z = tid; z < p.n_split; z += 256) {
    const f2_t ml = *reinterpret_cast<const f2_t*>(p.part_ml + 2 * (z * nrows + row));
    if (ml[1] > 0.f) m = fmaxf(m, ml[0]);
  }
  m = wave_max(m);
  if (lane == 0) stat[0][wave] = m;
  __syncthreads();
  const float M = fmaxf(fmaxf(stat[0][0], stat[0][1]), fmaxf(stat[0][2], stat[0][3]));
  float l = 0.f;
  for (int z = tid; z < p.n_split; z += 256) {
    const f2_t ml = *reinterpret_cast<const f2_t*>(p.part_ml + 2 * (z * nrows + row));
    const float w = ml[1] > 0.f ? __builtin_amdgcn_exp2f(ml[0] - M) : 0.f;
    w_s[z] = w;
    l += w * ml[1];
  }
  l = wave_sum(l);
  if (lane == 0) stat[1][wave] = l;
  __syncthreads();
  const float L = (stat[1][0] + stat[1][1]) + (stat[1][2] + stat[1][3]);
  const int sg = tid >> 5, d0 = (tid & 31) * 8;
  float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int z = sg; z < p.n_split; z += 8) {
    const float w = w_s[z];
    const float* po = p.part_o + (z * nrows + row) * kHD + d0;
    const f4_t a = *reinterpret_cast<const f4_t*>(po);
    const f4_t b = *reinterpret_cast<const f4_t*>(po + 4);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      x[i] += w * a[i];
      x[4 + i] += w * b[i];
    }
  }
#pragma unroll
  for (int i = 0; i < 8; i++) red[sg][d0 + i] = x[i];
  __syncthreads();
  if (tid < 32) {
    const float inv = L > 0.f ? 1.0f / L : 0.f;
    float y[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      float v = 0.f;
#pragma unroll
      for (int g = 0; g < 8; g++) v += red[g][d0 + i];
      y[i] = v * inv;
    }
    uint32_t pk[4];
#pragma unroll
    for (int i = 0; i < 4; i++) pk[i] = f2h(y[2 * i]) | (f2h(y[2 * i + 1]) << 16);
    *reinterpret_cast<uint4*>(out + row * kHD + d0) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
  }
}

PrefillGeom prefill_geom(int num_q, int num_kv, int n_tok, int start_pos) {
  PrefillGeom g{};
  g.n_pad = (n_tok + kKeys - 1) / kKeys * kKeys;
  // history rows: start_pos (prefill) or start_pos + n_tok (verify), padded to
  // whole tiles; the workspace covers the larger of the two
  g.h_pad = (start_pos + n_tok + kKeys - 1) / kKeys * kKeys;
  const int tg = prefill_token_groups(n_tok);
  const int qtiles = (n_tok + kWaveToks * tg - 1) / (kWaveToks * tg);
  const int wgs = num_kv * (num_q / num_kv == 6 ? 2 : 1) * qtiles;
  const int tiles = g.h_pad / kKeys + g.n_pad / kKeys;
  const int slots = tg == 2 ? 256 : 512;          // workgroups of one round: 256 CUs
  int ns = (slots + wgs - 1) / wgs;
  ns = std::min(ns, std::max(1, tiles / 8));      // at least ~8 tiles per split
  g.n_split = std::max(1, ns);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off = (off + bytes + 255) & ~(size_t)255;
    return at;
  };
  const size_t rows = (size_t)g.h_pad + g.n_pad;
  g.kx_off = take((size_t)num_kv * rows * kHD * 2);
  g.vt_off = take((size_t)num_kv * rows * kHD * 2);
  g.ml_off = take((size_t)g.n_split * n_tok * num_q * 2 * 4);
  g.o_off = take((size_t)g.n_split * n_tok * num_q * kHD * 4);
  g.total = off;
  return g;
}

hipError_t launch_prefill_tq3(const PrefillArgs& a, int gqa, const uint16_t* q, const uint16_t* k,
                              const uint16_t* v, uint16_t* out, hipStream_t stream) {
  {
    const long tiles = ((long)a.h_pad + a.n_pad) / kKeys;
    hipLaunchKernelGGL(prefill_stage_kernel, dim3((unsigned)(a.num_kv * tiles)), dim3(256), 0,
                       stream, a, k, v);
  }
  const int tg = prefill_token_groups(a.n_tok);
  const int qtiles = (a.n_tok + kWaveToks * tg - 1) / (kWaveToks * tg);
  const int groups = gqa == 6 ? 2 : 1;
  const Placement pl = placement(qtiles, a.num_kv * groups * a.n_split);
  const dim3 grid((unsigned)(8 * pl.subs * pl.per));
  if (gqa != 4 && gqa != 6) return hipErrorInvalidValue;
  // GQA 6: two workgroups of three heads per kv head
  const int heads = gqa == 6 ? 3 : 4;
  const dim3 block((unsigned)(64 * heads * tg));
  if (tg == 2) {
    if (gqa == 4 && !a.from_cache)
      hipLaunchKernelGGL((prefill_attn_kernel<4, 2, false>), grid, block, 0, stream, a, q);
    else if (gqa == 4)
      hipLaunchKernelGGL((prefill_attn_kernel<4, 2, true>), grid, block, 0, stream, a, q);
    else if (!a.from_cache)
      hipLaunchKernelGGL((prefill_attn_kernel<3, 2, false>), grid, block, 0, stream, a, q);
    else
      hipLaunchKernelGGL((prefill_attn_kernel<3, 2, true>), grid, block, 0, stream, a, q);
  } else {
    if (gqa == 4 && !a.from_cache)
      hipLaunchKernelGGL((prefill_attn_kernel<4, 1, false>), grid, block, 0, stream, a, q);
    else if (gqa == 4)
      hipLaunchKernelGGL((prefill_attn_kernel<4, 1, true>), grid, block, 0, stream, a, q);
    else if (!a.from_cache)
      hipLaunchKernelGGL((prefill_attn_kernel<3, 1, false>), grid, block, 0, stream, a, q);
    else
      hipLaunchKernelGGL((prefill_attn_kernel<3, 1, true>), grid, block, 0, stream, a, q);
  }
  const long rows = (long)a.n_tok * a.num_q;
  if (a.n_split > kMergeMaxSplits) return hipErrorInvalidValue;
  if (a.n_split >= 16)   // one workgroup per row, the splits spread over its threads
    hipLaunchKernelGGL(prefill_merge_wide_kernel, dim3((unsigned)rows), dim3(256), 0, stream, a, out);
  else
    hipLaunchKernelGGL(prefill_merge_kernel, dim3((unsigned)((rows + 7) / 8)), dim3(256), 0, stream, a,
                       out);
  return hipGetLastError();
}

}  // namespace qkv
