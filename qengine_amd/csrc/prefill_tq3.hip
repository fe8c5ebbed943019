// prefill_tq3.hip -- chunked-prefill attention over the packed TQ3 cache (gfx950).
//
// Reference semantics (model.cuh:5163-5214, 5256-5330, 5680-5721;
// attention.cuh:1690-1831 and 1837-1891): a chunk of n_tok new tokens at
// positions start_pos .. start_pos + n_tok - 1 attends causally to the cache
// history [0, start_pos), which the reference first dequantizes in bulk to an
// fp16 scratch (tq3_dequantize_kernel), and to the chunk's own keys and values
// in fp16 as produced by the projections (not quantized).  Query token t sees
// keys 0 .. start_pos + t.  Scores are fp32 dot products, softmax in fp32, the
// output fp16.
//
// Design (not the reference's): everything runs in the rotated domain of the
// codec, R = rs * H * D (orthogonal).  A history key decodes to
// norm * R^T c[idx], so q.k = norm * (R q).c[idx]; the chunk's own keys and
// values are rotated once (k~ = R k, v~ = R v, fp16) and the query likewise.
// Values accumulate in rotated coordinates and each output row is rotated back
// once at the end.  No key or value is ever inverse-transformed.
//
//   prefill_rotate_kernel   R q, R k, R v of the chunk into the workspace; the
//                           values go to 64-key tiles stored [dim][key] in the
//                           key order the value MFMA consumes.
//   prefill_attn_kernel     one workgroup per (kv head, 32 query tokens, key
//                           split) -- two per kv head for GQA 6, three heads
//                           each -- and one wave per query head.  Per
//                           64-key tile the history codes are decoded ONCE into
//                           LDS (fp16 centroids through the per-lane pair
//                           table, keys [key][dim], values [dim][key]) and
//                           shared by the 32 x GQA query rows:
//                             S^T  = K~ Q~^T      v_mfma_f32_32x32x16_f16, M = keys
//                             O^T += V~^T P^T     M = dims, N = query tokens
//                           so every lane owns one query row (token lane % 32)
//                           for the softmax and the accumulators.  Block norms
//                           scale the two 128-dim halves of a score and fold
//                           into P for the values.
//   prefill_merge_kernel    merges the key splits (log-sum-exp), rotates back
//                           (o = D H rs o~) and stores fp16.
#include <algorithm>

#include "qkv_device.h"
#include "attn_common.h"
#include "qkv_launch.h"

namespace qkv {
namespace {

typedef float f16x_t __attribute__((ext_vector_type(16)));

constexpr int kHD = 256;
constexpr int kKeys = 64;                 // keys per tile
constexpr int kToks = 32;                 // query tokens per workgroup

// LDS layout (bytes)
constexpr int kLut = 0;                   // centroid-pair table, one copy per lane (64 KiB)
constexpr int kKPitch = 528;              // key row: 256 fp16 + 16 B (conflict-free 16-B reads)
constexpr int kKTile = 65536;             // [64 keys][kKPitch]
constexpr int kVPitch = 144;              // dim row: 2 x 32 keys fp16 (value order) + 16 B
constexpr int kVTile = kKTile + kKeys * kKPitch;      // [256 dims][kVPitch]
constexpr int kRawK = kVTile + kHD * kVPitch;         // [64][104 B] raw key rows of the kv head
constexpr int kRawV = kRawK + kKeys * 104;
constexpr int kNk = kRawV + kKeys * 104;              // key norms [2 blocks][64] f32
constexpr int kNv = kNk + 2 * kKeys * 4;              // value norms [2][64]
constexpr int kLdsBytes = kNv + 2 * kKeys * 4;
static_assert(kLdsBytes <= 160 * 1024, "prefill LDS must fit one CU");

// Value order inside a 32-key half: key 8a + 4h + c sits at position
// 16(a/2) + 8h + 4(a%2) + c, so the 8 keys one lane contributes to a value
// MFMA (its own probabilities, in the score D layout) are contiguous.
__device__ __forceinline__ int value_pos(int key32) {
  const int a = key32 >> 3, h = (key32 >> 2) & 1, c = key32 & 3;
  return 16 * (a >> 1) + 8 * h + 4 * (a & 1) + c;
}

__device__ __forceinline__ uint32_t lut_at(const uint8_t* lds, uint32_t addr) {
  return *reinterpret_cast<const uint32_t*>(lds + kLut + addr);
}

// Table address of the 6-bit field at bit BIT of a 6-dword code stream.
template <int BIT>
__device__ __forceinline__ uint32_t pair_addr6(uint32_t& chain, const uint32_t (&q)[6]) {
  constexpr int w = BIT >> 5, sh = BIT & 31;
  if constexpr (sh + 6 <= 32)
    chain = sdwa_index<sh>(chain, q[w]);
  else
    chain = sdwa_index<0>(chain, __builtin_amdgcn_alignbit(q[w + 1], q[w], sh));
  return chain;
}

// Decode the 64 codes of a 192-bit stream into 32 fp16 pairs (dims 2m, 2m+1).
template <int M>
__device__ __forceinline__ void decode64(const uint8_t* lds, uint32_t (&ac)[4],
                                         const uint32_t (&q)[6], uint32_t (&out)[32]) {
  if constexpr (M < 32) {
    out[M] = lut_at(lds, pair_addr6<6 * M>(ac[M & 3], q));
    decode64<M + 1>(lds, ac, q, out);
  }
}

// Raw rows of one history tile: 64 keys x 104 B of kv head h, for K and V,
// as 8-byte pieces (13 per row); thread tid owns pieces tid + NT*j.
constexpr int kRawPieces = kKeys * 13 * 2;
template <int NT>
struct RawTile {
  static constexpr int kPer = (kRawPieces + NT - 1) / NT;
  u2_t d[kPer];
};

// Loads of history tile ti (rows past start_pos read as zero; a tile index
// past the history loads nothing useful and is never stored).
// k0: the tile's first key (workgroup-uniform); the buffer resources are
// rebased at its row (64-bit byte offsets).
template <int NT>
__device__ __forceinline__ void load_raw(RawTile<NT>& r, const PrefillArgs& p, int k0, int num_kv,
                                         int h, int tid) {
  const uint64_t off0 = (uint64_t)(uint32_t)k0 * (uint32_t)num_kv * 104u;
  const __amdgpu_buffer_rsrc_t rk = cache_rsrc(p.k_cache, off0, p.kv_bytes);
  const __amdgpu_buffer_rsrc_t rv = cache_rsrc(p.v_cache, off0, p.kv_bytes);
#pragma unroll
  for (int j = 0; j < RawTile<NT>::kPer; j++) {
    const int i = tid + NT * j;
    const int tv = i >= kKeys * 13;
    const int jj = i - tv * kKeys * 13;
    const int key = jj / 13, piece = jj - key * 13;
    const uint32_t off = (uint32_t)((key * num_kv + h) * 104 + piece * 8);
    r.d[j] = (i < kRawPieces) ? __builtin_amdgcn_raw_buffer_load_b64(tv ? rv : rk, off, 0, 0)
                              : u2_t{0u, 0u};
  }
}

template <int NT>
__device__ __forceinline__ void store_raw(const RawTile<NT>& r, uint8_t* lds, int tid) {
#pragma unroll
  for (int j = 0; j < RawTile<NT>::kPer; j++) {
    const int i = tid + NT * j;
    if (i < kRawPieces) {
      const int tv = i >= kKeys * 13;
      const int jj = i - tv * kKeys * 13;
      const int key = jj / 13, piece = jj - key * 13;
      *reinterpret_cast<u2_t*>(lds + (tv ? kRawV : kRawK) + key * 104 + piece * 8) = r.d[j];
    }
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// rotation of the chunk's queries, keys and values (16 lanes per 128-block)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void prefill_rotate_kernel(PrefillArgs p, const uint16_t* q,
                                                             const uint16_t* k,
                                                             const uint16_t* v) {
  const int lane = threadIdx.x & 63;
  const int part = threadIdx.x & 15;
  const long bid = (long)blockIdx.x * 16 + (threadIdx.x >> 4);
  const long nq_blk = (long)p.n_tok * p.num_q * 2;
  const long nk_blk = (long)p.n_pad * p.num_kv * 2;
  if (bid >= nq_blk + 2 * nk_blk) return;   // 16-lane groups leave together
  int which, row, blk;
  long rest;
  if (bid < nq_blk) {
    which = 0;
    rest = bid;
  } else if (bid < nq_blk + nk_blk) {
    which = 1;
    rest = bid - nq_blk;
  } else {
    which = 2;
    rest = bid - nq_blk - nk_blk;
  }
  blk = (int)(rest & 1);
  row = (int)(rest >> 1);   // q: t * num_q + qh;  k/v: u * num_kv + h
  float x[8];
  {
    uint4 raw = make_uint4(0u, 0u, 0u, 0u);
    if (which == 0) {
      raw = *reinterpret_cast<const uint4*>(q + (long)row * kHD + blk * 128 + part * 8);
    } else {
      const int u = row / p.num_kv;
      if (u < p.n_tok) {
        const uint16_t* src = which == 1 ? k : v;
        raw = *reinterpret_cast<const uint4*>(src + (long)row * kHD + blk * 128 + part * 8);
      }
    }
    const uint32_t wv[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      x[2 * i] = h2f(wv[i] & 0xffffu);
      x[2 * i + 1] = h2f(wv[i] >> 16);
    }
  }
  const uint32_t sbits = sign_word_sel(part >> 2) >> (8 * (part & 3));   // elements part*8..+7
#pragma unroll
  for (int i = 0; i < 8; i++) x[i] = ((sbits >> i) & 1u) ? x[i] : -x[i];
  wht8_inreg(x);
  wht_xor_lanes16(x, lane);
  const float rs = wht_scale();
  uint32_t pk[4];
#pragma unroll
  for (int i = 0; i < 4; i++) pk[i] = f2h(x[2 * i] * rs) | (f2h(x[2 * i + 1] * rs) << 16);
  const int dim0 = blk * 128 + part * 8;
  if (which == 0) {
    *reinterpret_cast<uint4*>(p.qr + (long)row * kHD + dim0) =
        make_uint4(pk[0], pk[1], pk[2], pk[3]);
    return;
  }
  const int u = row / p.num_kv, h = row - u * p.num_kv;
  if (which == 1) {
    *reinterpret_cast<uint4*>(p.kr + ((long)h * p.n_pad + u) * kHD + dim0) =
        make_uint4(pk[0], pk[1], pk[2], pk[3]);
    return;
  }
  // values: tile (h, u / 64), [dim][value position of u % 64]
  uint16_t* tile = p.vt + ((long)h * (p.n_pad / kKeys) + u / kKeys) * kHD * kKeys;
  const int key64 = u % kKeys;
  const int pos = (key64 >> 5) * 32 + value_pos(key64 & 31);
#pragma unroll
  for (int i = 0; i < 8; i++)
    tile[(dim0 + i) * kKeys + pos] = (uint16_t)((pk[i >> 1] >> (16 * (i & 1))) & 0xffffu);
}

// ---------------------------------------------------------------------------
// attention: grid (num_kv * gqa / WAVES, ceil(n_tok / 32), n_split); WAVES
// query heads of one kv head per workgroup, one wave per head
// ---------------------------------------------------------------------------
template <int WAVES, bool FROM_CACHE>
__global__ __launch_bounds__(64 * WAVES, 1) void prefill_attn_kernel(PrefillArgs p) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kLdsBytes];
  constexpr int NT = 64 * WAVES;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hh = lane >> 5;          // k-group of the MFMA operands / row group of D
  const int tok = lane & 31;         // query token (MFMA N index) of this lane
  const int gqa = p.num_q / p.num_kv;
  const int groups = gqa / WAVES;            // workgroups per kv head
  const int h = blockIdx.x / groups, hg = blockIdx.x - h * groups;
  const int qt = blockIdx.y, z = blockIdx.z;
  const int t0 = qt * kToks;
  const int n_q = min(kToks, p.n_tok - t0);
  const int qh = h * gqa + hg * WAVES + wave;

  // tiles: cache rows [0, hist) then (unless every key comes from the cache)
  // the chunk's own keys [0, t0 + n_q)
  const int hist = FROM_CACHE ? p.start_pos + t0 + n_q : p.start_pos;
  const int th = (hist + kKeys - 1) / kKeys;
  const int tc = FROM_CACHE ? 0 : (t0 + n_q + kKeys - 1) / kKeys;
  const int total = th + tc;
  const int tps = (total + p.n_split - 1) / p.n_split;
  const int tlo = min(total, z * tps), thi = min(total, tlo + tps);

  // ---- centroid-pair table: entry E of lane L at byte E*256 + 4L holds the
  // fp16 pair (centroid[E & 7], centroid[(E >> 3) & 7])
  const uint32_t lane4 = 4u * (uint32_t)lane;
  for (int e = wave; e < 256; e += WAVES) {
    const uint32_t pr = f2h(centroid_imm((uint32_t)e & 7u)) | (f2h(centroid_imm(((uint32_t)e >> 3) & 7u)) << 16);
    *reinterpret_cast<uint32_t*>(lds + kLut + e * 256 + lane4) = pr;
  }

  // ---- rotated query of (token t0 + tok, head qh): B operands, slice s of block b
  h8_t qb[2][8];
  {
    const uint32_t qbytes = (uint32_t)((long)p.n_tok * p.num_q * kHD * 2);
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
        p.qr, 0, qbytes, kBufferRsrcWord3);
    const uint32_t base = tok < n_q ? (uint32_t)((((long)(t0 + tok) * p.num_q + qh) * kHD) * 2) : qbytes;
#pragma unroll
    for (int b = 0; b < 2; b++)
#pragma unroll
      for (int s = 0; s < 8; s++)
        qb[b][s] = __builtin_bit_cast(
            h8_t, __builtin_amdgcn_raw_buffer_load_b128(rq, base + (b * 128 + 16 * s + 8 * hh) * 2, 0, 0));
  }


  f16x_t acc[8];
#pragma unroll
  for (int d = 0; d < 8; d++) acc[d] = f16x_t{};
  float m2 = -INFINITY, lsum = 0.0f;
  const float* nk = reinterpret_cast<const float*>(lds + kNk);
  const float* nv = reinterpret_cast<const float*>(lds + kNv);
  const int t_abs = t0 + tok;        // this lane's token index in the chunk

  // the first tile's raw rows (history tiles only; a chunk tile loads nothing)
  RawTile<NT> raw;
  if (tlo < min(thi, th)) load_raw(raw, p, tlo * kKeys, p.num_kv, h, tid);

  for (int ti = tlo; ti < thi; ti++) {
    const bool cached = ti < th;
    const int k0 = cached ? ti * kKeys : (ti - th) * kKeys;
    const int nkeys = cached ? min(kKeys, hist - k0) : kKeys;
    __syncthreads();   // the previous tile's MFMAs are done with the tile buffers
    if (cached) {
      // raw rows of kv head h (104 B per key: 2 blocks of 52 B), loaded during
      // the previous tile; rows past start_pos read as zero (buffer range)
      store_raw(raw, lds, tid);
      // the next history tile's rows go out now and arrive during this tile
      if (ti + 1 < min(thi, th)) load_raw(raw, p, (ti + 1) * kKeys, p.num_kv, h, tid);
      __syncthreads();
      uint32_t ac[4] = {lane4, lane4, lane4, lane4};
      // keys: item (key, quarter): block quarter >> 1, codes 64*(quarter & 1) ..
      for (int it = tid; it < kKeys * 4; it += NT) {
        const int key = it & 63, qtr = it >> 6;
        const int b = qtr >> 1, half = qtr & 1;
        const uint8_t* src = lds + kRawK + key * 104 + b * 52 + 4 + 24 * half;
        uint32_t cq[6];
#pragma unroll
        for (int w = 0; w < 6; w++) cq[w] = reinterpret_cast<const uint32_t*>(src)[w];
        uint32_t pr[32];
        decode64<0>(lds, ac, cq, pr);
        uint8_t* dst = lds + kKTile + key * kKPitch + (b * 128 + 64 * half) * 2;
#pragma unroll
        for (int w = 0; w < 8; w++)
          *reinterpret_cast<uint4*>(dst + 16 * w) =
              make_uint4(pr[4 * w], pr[4 * w + 1], pr[4 * w + 2], pr[4 * w + 3]);
      }
      __builtin_amdgcn_sched_barrier(0);   // keep the key and value decode apart (registers)
      // values: item (block, code group g, half kt, pair A, row group r): keys
      // kt*32 + 16A + 8(i>>2) + 4r + (i&3), i = 0..7, at value positions
      // kt*32 + 16A + 8r + i; dims b*128 + 8g .. +7
      for (int it = tid; it < 256; it += NT) {
        const int b = it >> 7, g = (it >> 3) & 15, kt = (it >> 2) & 1, A = (it >> 1) & 1, r = it & 1;
        uint32_t cp[8][4];
#pragma unroll
        for (int i = 0; i < 8; i++) {
          const int key = kt * 32 + 16 * A + 8 * (i >> 2) + 4 * r + (i & 3);
          const int off = kRawV + key * 104 + b * 52 + 4 + 3 * g;
          const uint32_t* wp = reinterpret_cast<const uint32_t*>(lds + (off & ~3));
          const uint32_t w = __builtin_amdgcn_alignbyte(wp[1], wp[0], off & 3);
          cp[i][0] = lut_at(lds, ac[0] = sdwa_index<0>(ac[0], w));
          cp[i][1] = lut_at(lds, ac[1] = sdwa_index<6>(ac[1], w));
          cp[i][2] = lut_at(lds, ac[2] = sdwa_index<12>(ac[2], w));
          cp[i][3] = lut_at(lds, ac[3] = sdwa_index<18>(ac[3], w));
        }
        uint8_t* dst = lds + kVTile + (b * 128 + 8 * g) * kVPitch + (kt * 32 + 16 * A + 8 * r) * 2;
#pragma unroll
        for (int m = 0; m < 4; m++)
#pragma unroll
          for (int e = 0; e < 2; e++) {
            const uint32_t sel = e ? 0x07060302u : 0x05040100u;
            *reinterpret_cast<uint4*>(dst + (2 * m + e) * kVPitch) =
                make_uint4(__builtin_amdgcn_perm(cp[1][m], cp[0][m], sel),
                           __builtin_amdgcn_perm(cp[3][m], cp[2][m], sel),
                           __builtin_amdgcn_perm(cp[5][m], cp[4][m], sel),
                           __builtin_amdgcn_perm(cp[7][m], cp[6][m], sel));
          }
      }
      __builtin_amdgcn_sched_barrier(0);
      for (int it = tid; it < 4 * kKeys; it += NT) {
        const int key = it & 63, b = (it >> 6) & 1, tv = it >> 7;
        const float nrm = *reinterpret_cast<const float*>(lds + (tv ? kRawV : kRawK) + key * 104 + b * 52);
        *reinterpret_cast<float*>(lds + (tv ? kNv : kNk) + (b * kKeys + key) * 4) = nrm;
      }
    } else {
      // the chunk's own rotated keys and value tile (fp16, norm 1)
      const uint4* ksrc = reinterpret_cast<const uint4*>(p.kr + ((long)h * p.n_pad + k0) * kHD);
      for (int i = tid; i < kKeys * 32; i += NT) {
        const int key = i >> 5, piece = i & 31;
        *reinterpret_cast<uint4*>(lds + kKTile + key * kKPitch + piece * 16) = ksrc[i];
      }
      const uint4* vsrc = reinterpret_cast<const uint4*>(
          p.vt + ((long)h * (p.n_pad / kKeys) + k0 / kKeys) * kHD * kKeys);
      for (int i = tid; i < kHD * 8; i += NT) {
        const int dim = i >> 3, piece = i & 7;
        *reinterpret_cast<uint4*>(lds + kVTile + dim * kVPitch + piece * 16) = vsrc[i];
      }
      for (int it = tid; it < 4 * kKeys; it += NT)
        *reinterpret_cast<float*>(lds + kNk + it * 4) = 1.0f;   // kNk and kNv are adjacent
    }
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);

    // The two 32-key halves kt of the tile run one after the other: scores,
    // an online-softmax step, values.
    // every key of the tile visible to every token of the workgroup
    const bool dense = cached && nkeys == kKeys && (!FROM_CACHE || k0 + kKeys - 1 <= p.start_pos + t0);
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
      __builtin_amdgcn_sched_barrier(0);
      // ---- scores S^T = K~ Q~^T: D[b], row = key kt*32 + 8(v/4) + 4hh + v%4, col = token
      f16x_t sd[2];
#pragma unroll
      for (int b = 0; b < 2; b++) {
        sd[b] = f16x_t{};
        const uint8_t* arow = lds + kKTile + (kt * 32 + tok) * kKPitch + (b * 128 + 8 * hh) * 2;
#pragma unroll
        for (int s = 0; s < 8; s++) {
          const h8_t a = *reinterpret_cast<const h8_t*>(arow + 32 * s);
          sd[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qb[b][s], sd[b], 0, 0, 0);
        }
      }
      float sc[16];
#pragma unroll
      for (int a = 0; a < 4; a++) {
        const int kb = kt * 32 + 8 * a + 4 * hh;
        const f4_t n0 = *reinterpret_cast<const f4_t*>(nk + kb);
        const f4_t n1 = *reinterpret_cast<const f4_t*>(nk + kKeys + kb);
#pragma unroll
        for (int c = 0; c < 4; c++) {
          float sv = (n0[c] * sd[0][4 * a + c] + n1[c] * sd[1][4 * a + c]) * p.scale_log2;
          if (!dense) {
            const int key = kb + c;
            // history keys (k0 + key < start_pos) are visible to every token
            const bool vis = cached ? (key < nkeys) & (!FROM_CACHE || k0 + key <= p.start_pos + t_abs)
                                    : (k0 + key <= t_abs);
            sv = vis ? sv : -INFINITY;
          }
          sc[4 * a + c] = sv;
        }
      }
      // ---- online softmax of this lane's row (partner lane: lane ^ 32)
      float mt = sc[0];
#pragma unroll
      for (int v = 1; v < 16; v++) mt = fmaxf(mt, sc[v]);
      {
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt), false, false);
        mt = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
      }
      // The accumulators are rescaled only on steps where some row's maximum
      // grows (a wave-uniform branch, rare after the first tiles).
      if (__builtin_amdgcn_ballot_w64(mt > m2) != 0) {
        const float mn = fmaxf(m2, mt);
        const float corr = (mn == -INFINITY) ? 1.0f : __builtin_amdgcn_exp2f(m2 - mn);
        lsum *= corr;
#pragma unroll
        for (int d = 0; d < 8; d++) acc[d] *= corr;
        m2 = mn;
      }
      const float msafe = (m2 == -INFINITY) ? 0.0f : m2;
#pragma unroll
      for (int v = 0; v < 16; v++) {
        sc[v] = __builtin_amdgcn_exp2f(sc[v] - msafe);
        lsum += sc[v];
      }
      // ---- values O^T += V~^T (P * value norm)^T.  B operand (b, sg): the
      // probabilities v = 8sg .. 8sg+7, each times its key's value norm in block b.
#pragma unroll
      for (int sg = 0; sg < 2; sg++) {
        h8_t pb[2];
#pragma unroll
        for (int b = 0; b < 2; b++) {
#pragma unroll
          for (int a2 = 0; a2 < 2; a2++) {
            const int a = 2 * sg + a2;
            const f4_t nn = *reinterpret_cast<const f4_t*>(nv + b * kKeys + kt * 32 + 8 * a + 4 * hh);
#pragma unroll
            for (int c = 0; c < 4; c++) pb[b][4 * a2 + c] = (_Float16)(sc[4 * a + c] * nn[c]);
          }
        }
#pragma unroll
        for (int d = 0; d < 8; d++) {
          const h8_t a = *reinterpret_cast<const h8_t*>(
              lds + kVTile + (d * 32 + tok) * kVPitch + (kt * 32 + 16 * sg + 8 * hh) * 2);
          acc[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb[d >> 2], acc[d], 0, 0, 0);
        }
      }
    }
  }

  // ---------------- partials of this split: m (log2 units), l, o~ (rotated)
  {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(lsum), __float_as_uint(lsum), false, false);
    lsum = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
  if (tok < n_q) {
    const long row = ((long)z * p.n_tok + t0 + tok) * p.num_q + qh;
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
// merge of the key splits, rotation back, fp16 store: 32 threads per row
// (16 per 128-block, 8 dims each)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillArgs p, uint16_t* out) {
  const int lane = threadIdx.x & 63;
  const long row = (long)blockIdx.x * 8 + (threadIdx.x >> 5);   // t * num_q + qh
  if (row >= (long)p.n_tok * p.num_q) return;                    // 32-thread groups leave together
  const int blk = (threadIdx.x >> 4) & 1, part = threadIdx.x & 15;
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
    const float* po = p.part_o + (z * nrows + row) * kHD + blk * 128 + part * 8;
    const f4_t a = *reinterpret_cast<const f4_t*>(po);
    const f4_t b = *reinterpret_cast<const f4_t*>(po + 4);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      x[i] += w * a[i];
      x[4 + i] += w * b[i];
    }
  }
  const float inv = L > 0.f ? 1.0f / L : 0.f;
#pragma unroll
  for (int i = 0; i < 8; i++) x[i] *= inv;
  wht8_inreg(x);
  wht_xor_lanes16(x, lane);
  const float rs = wht_scale();
  const uint32_t sbits = sign_word_sel(part >> 2) >> (8 * (part & 3));
  uint32_t pk[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    float y0 = x[2 * i] * rs, y1 = x[2 * i + 1] * rs;
    y0 = ((sbits >> (2 * i)) & 1u) ? y0 : -y0;
    y1 = ((sbits >> (2 * i + 1)) & 1u) ? y1 : -y1;
    pk[i] = f2h(y0) | (f2h(y1) << 16);
  }
  *reinterpret_cast<uint4*>(out + row * kHD + blk * 128 + part * 8) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
PrefillGeom prefill_geom(int num_q, int num_kv, int n_tok, int start_pos) {
  PrefillGeom g{};
  g.n_pad = (n_tok + kKeys - 1) / kKeys * kKeys;
  const int qtiles = (n_tok + kToks - 1) / kToks;
  const int wgs = num_kv * (num_q / num_kv == 6 ? 2 : 1) * qtiles;
  const int tiles = (start_pos + kKeys - 1) / kKeys + (n_tok + kKeys - 1) / kKeys;
  int ns = (256 + wgs - 1) / wgs;                 // fill 256 CUs
  ns = std::min(ns, std::max(1, tiles / 8));      // at least ~8 tiles per split
  g.n_split = std::max(1, ns);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off = (off + bytes + 255) & ~(size_t)255;
    return at;
  };
  g.qr_off = take((size_t)n_tok * num_q * kHD * 2);
  g.kr_off = take((size_t)num_kv * g.n_pad * kHD * 2);
  g.vt_off = take((size_t)num_kv * g.n_pad * kHD * 2);
  g.ml_off = take((size_t)g.n_split * n_tok * num_q * 2 * 4);
  g.o_off = take((size_t)g.n_split * n_tok * num_q * kHD * 4);
  g.total = off;
  return g;
}

hipError_t launch_prefill_tq3(const PrefillArgs& a, int gqa, const uint16_t* q, const uint16_t* k,
                              const uint16_t* v, uint16_t* out, hipStream_t stream) {
  {
    const long blocks = (long)a.n_tok * a.num_q * 2 + 2L * a.n_pad * a.num_kv * 2;
    hipLaunchKernelGGL(prefill_rotate_kernel, dim3((unsigned)((blocks + 15) / 16)), dim3(256), 0,
                       stream, a, q, k, v);
  }
  const int qtiles = (a.n_tok + kToks - 1) / kToks;
  const dim3 g4(a.num_kv, qtiles, a.n_split), g6(a.num_kv * 2, qtiles, a.n_split);
  if (gqa == 4 && !a.from_cache)
    hipLaunchKernelGGL((prefill_attn_kernel<4, false>), g4, dim3(256), 0, stream, a);
  else if (gqa == 4)
    hipLaunchKernelGGL((prefill_attn_kernel<4, true>), g4, dim3(256), 0, stream, a);
  else if (gqa == 6 && !a.from_cache)   // two workgroups of three heads per kv head
    hipLaunchKernelGGL((prefill_attn_kernel<3, false>), g6, dim3(192), 0, stream, a);
  else if (gqa == 6)
    hipLaunchKernelGGL((prefill_attn_kernel<3, true>), g6, dim3(192), 0, stream, a);
  else
    return hipErrorInvalidValue;
  const long rows = (long)a.n_tok * a.num_q;
  hipLaunchKernelGGL(prefill_merge_kernel, dim3((unsigned)((rows + 7) / 8)), dim3(256), 0, stream, a,
                     out);
  return hipGetLastError();
}

}  // namespace qkv
