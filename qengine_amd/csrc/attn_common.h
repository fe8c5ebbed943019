// attn_common.h -- argument block and wave-level helpers shared by the
// attention kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qkv_device.h"

namespace qkv {

constexpr float kLn2 = 0.69314718055994531f;
constexpr float kLog2e = 1.44269504088896341f;

// Fast-path workspace: kWsHeaderBytes at its start, then the record scalars
// {m, l, tag of 128-block unit 0, tag of unit 1} (kRecMlBytes each) and the
// record rows.  A tag is kTagValid while its record is waiting for that unit's
// merger and 0 otherwise (the state of a zero-filled workspace).  Header word
// kWsErrorWord is 0 while the workspace is consistent; a merger whose bounded
// wait ran out sets it to kWsErrorTimeout, and from then on every merge of a
// launch on that workspace writes NaN rows until the workspace is zero-filled
// again (records it could not account for may still carry set tags).
constexpr int kWsHeaderBytes = 256;
constexpr int kRecMlBytes = 16;
constexpr uint32_t kTagValid = 1u;
constexpr int kWsErrorWord = 0;
constexpr int kWsErrorTimeout = 1;
// Poll limit of a merger waiting for the records of one launch (each poll
// sleeps ~64 cycles after two memory round trips; the default limit is
// seconds, far beyond any legitimate wait).
constexpr int kMergeSpinLimit = 1 << 22;

struct AttnArgs {
  const uint16_t* q;        // [sub_n][num_q][256] fp16
  const uint32_t* k;        // slot-base key cache (blocks viewed as dwords)
  const uint32_t* v;        // slot-base value cache
  uint64_t kv_bytes;        // readable bytes of each cache from its base
  uint64_t v_bytes;         // value cache extent when its format differs from the keys' (else unused)
  int num_q, num_kv;
  int start_pos, sub_n, sub_n_max;
  int qpw;                  // queries per workgroup (MFMA columns = qpw * gqa <= 16)
  int active_end_max;       // reference split sizing (split API)
  int k_splits;             // reference split count (split API)
  int n_chunks;             // workgroups per (kv head, query group): k_splits or key chunks
  int chunk_keys;           // keys per fast-path chunk (multiple of 256)
  int n_slots;              // fast-path records per (q head, query): n_chunks
  float scale_log2;         // softmax scale * log2(e)
  int sink_tok, window_tok;
  const uint32_t* tree_mask;
  // paged caches (fast path): when block_tables is set, key index k of query
  // (slot) t lives in cache row block_tables[t * bt_stride + k / block_tokens]
  // * block_tokens + k % block_tokens, and ctx_lens[t] (clamped to
  // [0, ctx_max]) replaces start_pos + t + 1 as the query's key count
  const int32_t* block_tables;
  int bt_stride, block_tokens;
  const int32_t* ctx_lens;
  int ctx_max;
  // block-sparse split (tq3_attn_kernel<2>): query t of kv head h attends the
  // 64-key blocks block_index[(h * sub_n_max + t) * top_k + i] (ascending,
  // -1 after the last); split z takes entries z * ceil(top_k / k_splits) ..
  const int32_t* block_index;
  int top_k;
  // split API partials (reference layout)
  float* part_m;
  float* part_l;
  float* part_o;
  // fast-path workspace
  float* ws_ml;             // [num_q][sub_n][n_slots] x {m (log2 units), l, tag0, tag1}
  float* ws_o;              // [num_q][sub_n][n_slots][256] rotated coordinates
  int* ws_header;           // kWsHeaderBytes; word kWsErrorWord: sticky merge error
  uint32_t ws_ml_bytes, ws_o_bytes;
  int spin_limit;           // merger poll limit (kMergeSpinLimit unless a test lowers it)
  // fused Q8 append (q8_attn_kernel APPEND, sub_n == 1): the new token's fp16
  // K and V rows [num_kv][256], quantized in the kernel, used for key
  // start_pos and written to that row of the caches (k_w, v_w = k, v)
  const uint16_t* k_new;
  const uint16_t* v_new;
  uint8_t* k_w;
  uint8_t* v_w;
};

// ---- leading (preloaded) kernel arguments -------------------------------
// The library is compiled with -mllvm -amdgpu-kernarg-preload-count=16: on
// gfx950 the command processor writes the leading kernel arguments straight
// into SGPRs at wave launch (14 SGPRs, after the kernarg segment pointer).
// The attention kernels therefore take the fields their first loads depend on
// as leading scalar arguments ahead of the AttnArgs block (whose remaining
// fields are read through the kernarg segment as before), so that the query
// and tile loads issue without waiting for a kernel-argument round trip.
// (Firmware without preload support runs the compiler's compatibility
// prologue, which loads the same SGPRs.)
//   lead_heads: num_q | num_kv << 16;  lead_flags: qpw | paged << 8 | ragged << 9
#define QKV_ATTN_LEAD_PARAMS                                                                    \
  const uint16_t *lead_q, const uint32_t *lead_k, const uint32_t *lead_v, uint64_t lead_kv_bytes, \
      uint32_t lead_heads, uint32_t lead_flags, int lead_start_pos, int lead_sub_n,              \
      int lead_n_chunks, int lead_chunk_keys
#define QKV_ATTN_LEAD_ARGS(a)                                                                    \
  (a).q, (a).k, (a).v, (a).kv_bytes, ::qkv::attn_lead_heads(a), ::qkv::attn_lead_flags(a),      \
      (a).start_pos, (a).sub_n, (a).n_chunks, (a).chunk_keys
// Local AttnArgs `p`: the block `pin` with the leading arguments written over
// it (the compiler then takes those fields from the preloaded SGPRs).
#define QKV_ATTN_LEAD_APPLY(p, pin)                                                   \
  AttnArgs p = (pin);                                                                 \
  p.q = lead_q;                                                                       \
  p.k = lead_k;                                                                       \
  p.v = lead_v;                                                                       \
  p.kv_bytes = lead_kv_bytes;                                                         \
  p.num_q = (int)(lead_heads & 0xffffu);                                              \
  p.num_kv = (int)(lead_heads >> 16);                                                 \
  p.qpw = (int)(lead_flags & 0xffu);                                                  \
  p.start_pos = lead_start_pos;                                                       \
  p.sub_n = lead_sub_n;                                                               \
  p.n_chunks = lead_n_chunks;                                                         \
  p.chunk_keys = lead_chunk_keys
inline uint32_t attn_lead_heads(const AttnArgs& a) {
  return (uint32_t)a.num_q | ((uint32_t)a.num_kv << 16);
}
inline uint32_t attn_lead_flags(const AttnArgs& a) {
  return (uint32_t)a.qpw | (a.block_tables ? 1u << 8 : 0u) | (a.ctx_lens ? 1u << 9 : 0u);
}
// Head counts that fit the 16-bit fields of lead_heads.
constexpr int kLeadMaxHeads = 0xffff;

// Buffer resource over bytes [off, extent) of a cache, rebased at the 64-bit
// byte offset `off` (wave-uniform) so that the in-tile offsets of a load stay
// small: caches past 4 GiB are addressed exactly.  Bytes at or past `extent`
// read as zero (the buffer range check), also for a tile that starts there.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t cache_rsrc(const void* base, uint64_t off,
                                                             uint64_t extent) {
  const bool in = off < extent;
  const uint64_t rem = in ? extent - off : 0;
  char* b = const_cast<char*>(static_cast<const char*>(base)) + (in ? off : 0);
  return __builtin_amdgcn_make_buffer_rsrc(b, 0, (uint32_t)(rem < 0xffffffffull ? rem : 0xffffffffull),
                                           0x00020000);
}

// ---- DPP wave reductions (result broadcast through lane 63) -------------
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v),
                                                               __builtin_bit_cast(int, v), CTRL,
                                                               ROW_MASK, 0xf, false));
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));         // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_f<0x4E>(v));         // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_f<0x124>(v));        // row_ror:4
  v = fmaxf(v, dpp_f<0x128>(v));        // row_ror:8
  v = fmaxf(v, dpp_f<0x142, 0xa>(v));   // row_bcast:15
  v = fmaxf(v, dpp_f<0x143, 0xc>(v));   // row_bcast:31
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x124>(v);
  v += dpp_f<0x128>(v);
  v += dpp_f<0x142, 0xa>(v);
  v += dpp_f<0x143, 0xc>(v);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Table address: byte 1 of `addr` := bits SHIFT..SHIFT+7 of w, bytes 0, 2, 3
// (4 * lane, 0, 0) kept -- one v_lshrrev_b32 with SDWA dst_sel:BYTE_1 and
// dst_unused:UNUSED_PRESERVE.  Each address register is reused by the next
// lookup of its chain, so no copy of 4 * lane is needed per lookup.
template <int SHIFT>
__device__ __forceinline__ uint32_t sdwa_index(uint32_t addr, uint32_t w) {
  asm("v_lshrrev_b32_sdwa %0, %2, %1 dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:DWORD "
      "src1_sel:DWORD"
      : "+v"(addr)
      : "v"(w), "i"(SHIFT));
  return addr;
}
// Lloyd-Max centroid i (turboquant.cuh:27-30) selected from immediates.
__device__ __forceinline__ float centroid_imm(uint32_t i) {
  // i >= 4: +m[i-4]; i < 4: -m[3-i]  (symmetric table)
  const float mpos = (i & 2) ? ((i & 1) ? 0.190303f : 0.118828f) : ((i & 1) ? 0.066847f : 0.021664f);
  const uint32_t j = 3u - (i & 3u);
  const float mneg = (j & 2) ? ((j & 1) ? 0.190303f : 0.118828f) : ((j & 1) ? 0.066847f : 0.021664f);
  return (i & 4) ? mpos : -mneg;
}

// Scaled centroid table of the rotated-domain consumers.  The fp16 LUT holds
// the Lloyd-Max levels (turboquant.cuh:27-30) times kCenScale, a factor chosen
// so that all four magnitudes land within 2.6e-5 (relative) of an fp16 value
// (unscaled, the fp16 levels are up to 2.0e-4 off, enough to move attention
// rows by ~1e-3); scores and value sums are divided by kCenScale again in
// fp32 (key norms carry kCenScaleInv, outputs are multiplied by it).
constexpr float kCenScale = 1.14951002597808838f;
constexpr float kCenScaleInv = 1.0f / kCenScale;
// fp16 bits of kCenScale * |centroid| for magnitude index 0..3 (round to nearest)
constexpr uint16_t kCenScaledH[4] = {0x2660, 0x2ceb, 0x305f, 0x3300};
__device__ __forceinline__ uint32_t centroid_scaled_h(uint32_t i) {
  // i >= 4: +m[i-4]; i < 4: -m[3-i] (symmetric table)
  const uint32_t m = (i & 4u) ? (i & 3u) : (3u - (i & 3u));
  const uint32_t mag = (m & 2u) ? ((m & 1u) ? kCenScaledH[3] : kCenScaledH[2])
                                : ((m & 1u) ? kCenScaledH[1] : kCenScaledH[0]);
  return (i & 4u) ? mag : (mag | 0x8000u);
}

// ---- 128-point Walsh-Hadamard pieces (butterflies (a,b) -> (a+b, a-b)) ----
// Element e = part*8 + i of a 128-block lives in register i of lane `part`
// (16 consecutive lanes per block).
__device__ __forceinline__ void wht8_inreg(float (&x)[8]) {
#pragma unroll
  for (int step = 1; step < 8; step <<= 1)
#pragma unroll
    for (int i = 0; i < 8; i += 2 * step)
#pragma unroll
      for (int j = i; j < i + step; j++) {
        const float a = x[j], b = x[j + step];
        x[j] = a + b;
        x[j + step] = a - b;
      }
}

// Value of lane (lane ^ M) inside each 16-lane row, through DPP (no LDS):
// quad_perm for M = 1, 2; row_ror:8 for M = 8; for M = 4 lanes with bit 2 set
// take row_ror:4 (lane - 4), the others row_ror:12 (lane + 4).
template <int M>
__device__ __forceinline__ float xor16_partner(float v, int lane) {
  if constexpr (M == 1) return dpp_f<0xB1>(v);
  else if constexpr (M == 2) return dpp_f<0x4E>(v);
  else if constexpr (M == 8) return dpp_f<0x128>(v);
  else {
    // both moves run on every lane (a DPP move reading a lane that is
    // inactive at that point returns the lane's own value)
    const float from_lower = dpp_f<0x124>(v), from_upper = dpp_f<0x12C>(v);
    return (lane & 4) ? from_lower : from_upper;
  }
}

template <int M>
__device__ __forceinline__ void wht_xor_stage(float (&x)[8], int lane) {
  const bool upper = (lane & M) != 0;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const float o = xor16_partner<M>(x[i], lane);
    x[i] = upper ? (o - x[i]) : (x[i] + o);
  }
}

// Butterfly stages 8..64 of a 128-point WHT spread over 16 lanes x 8 elements
// (lane = element octet): stage 8*M pairs lane with lane ^ M.
__device__ __forceinline__ void wht_xor_lanes16(float (&x)[8], int lane) {
  wht_xor_stage<1>(x, lane);
  wht_xor_stage<2>(x, lane);
  wht_xor_stage<4>(x, lane);
  wht_xor_stage<8>(x, lane);
}

// fp32 Lloyd-Max level i (turboquant.cuh:27-30), selected without a memory
// lookup: i >= 4: +m[i-4], i < 4: -m[3-i].
__device__ __forceinline__ float centroid_f32(uint32_t i) {
  const uint32_t m = (i & 4u) ? (i & 3u) : (3u - (i & 3u));
  const float mag = (m & 2u) ? ((m & 1u) ? 0.190303f : 0.118828f) : ((m & 1u) ? 0.066847f : 0.021664f);
  return (i & 4u) ? mag : -mag;
}

// The reference's TQ3 dequantization of one 52-byte block (turboquant.cuh:
// 169-200), bit for bit, spread over 16 consecutive lanes: lane `part` of the
// group gets elements part*8 .. part*8+7 as four fp16 pairs.  fp32 centroids,
// the seven butterfly stages in the reference's pairing (three in registers,
// four across the lanes), * rs, sign, * norm kept an fp32 product, fp16.
// The three dwords a lane needs (norm and the two code words holding its
// group), loaded apart from the arithmetic so that a caller can issue the
// loads of several blocks before the first is used.
struct Tq3Group {
  float norm;
  uint32_t lo, hi;
};
__device__ __forceinline__ Tq3Group tq3_group_load(const uint8_t* blk, int part) {
  // code group `part`: bytes 3*part .. 3*part+2 of the 48 code bytes
  const int w0 = (3 * part) >> 2;
  const uint32_t* cw = reinterpret_cast<const uint32_t*>(blk + 4);
  return Tq3Group{*reinterpret_cast<const float*>(blk), cw[w0], cw[min(w0 + 1, 11)]};
}

// What a lane of the group dequantization keeps for the whole kernel: the
// factors rs * sign of its elements (negating the fp32 product x * rs is
// exact, so the sign folds into the factor) and the sign-bit flips of its
// four cross-lane butterfly stages (set where the lane is the upper one of a
// pair).
struct Tq3LaneConst {
  float rsi[8];
  uint32_t flip[4];
};
__device__ __forceinline__ Tq3LaneConst tq3_lane_const(int part) {
  Tq3LaneConst c;
  const float rs = wht_scale();
  const uint32_t sbits = sign_word_sel(part >> 2) >> (8 * (part & 3));   // elements part*8..+7
#pragma unroll
  for (int i = 0; i < 8; i++) c.rsi[i] = ((sbits >> i) & 1u) ? rs : -rs;
#pragma unroll
  for (int k = 0; k < 4; k++) c.flip[k] = ((part >> k) & 1) ? 0x80000000u : 0u;
  return c;
}
// The eight fp32 levels in LDS (threads 0..7 write them; a barrier follows
// before the first tq3_group_dequant): a lane's level is one LDS read, where
// a select chain would cost several four-cycle selects per element.
__device__ __forceinline__ void tq3_centroid_table(float* cent, int tid) {
  if (tid < 8) cent[tid] = centroid_f32((uint32_t)tid);
}

// One cross-lane butterfly stage (partner lane ^ M inside the 16-lane group):
// the lower lane of a pair takes own + partner, the upper partner - own,
// formed as partner + (own with its sign bit flipped) -- IEEE a - b is
// a + (-b), so the values are those of the two-operation form -- in one
// DPP-sourced add.
template <int CTRL>
__device__ __forceinline__ float dpp_mov_bc(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
}
template <int M>
__device__ __forceinline__ void tq3_xor_stage(float (&x)[8], uint32_t flip) {
#pragma unroll
  for (int i = 0; i < 8; i++) {
    float o;
    if constexpr (M == 1) o = dpp_mov_bc<0xB1>(x[i]);                       // quad_perm [1,0,3,2]
    else if constexpr (M == 2) o = dpp_mov_bc<0x4E>(x[i]);                  // quad_perm [2,3,0,1]
    else if constexpr (M == 4) o = dpp_mov_bc<0x1B>(dpp_mov_bc<0x141>(x[i]));   // i ^ 7, then ^ 3
    else o = dpp_mov_bc<0x128>(x[i]);                                       // row_ror:8
    x[i] = o + __uint_as_float(__float_as_uint(x[i]) ^ flip);
  }
}

// Every lane of the 16-lane group must be active (the stages read the other
// lanes of the group).
__device__ __forceinline__ void tq3_group_dequant(const Tq3Group& gr, int part, const float* cent,
                                                  const Tq3LaneConst& lc, uint32_t (&pk)[4]) {
  const uint32_t g = __builtin_amdgcn_alignbyte(gr.hi, gr.lo, (3 * part) & 3);
  float x[8];
#pragma unroll
  for (int i = 0; i < 8; i++) x[i] = cent[(g >> (3 * i)) & 7u];
  wht8_inreg(x);
  tq3_xor_stage<1>(x, lc.flip[0]);
  tq3_xor_stage<2>(x, lc.flip[1]);
  tq3_xor_stage<4>(x, lc.flip[2]);
  tq3_xor_stage<8>(x, lc.flip[3]);
#pragma unroll
  for (int i = 0; i < 4; i++) {
    // the reference rounds v*norm to fp32, then to fp16: the empty asm keeps
    // the fp32 product (no fused fp16-rounding mixed FMA)
    float pa = (x[2 * i] * lc.rsi[2 * i]) * gr.norm, pb = (x[2 * i + 1] * lc.rsi[2 * i + 1]) * gr.norm;
    asm volatile("" : "+v"(pa), "+v"(pb));
    pk[i] = f2h(pa) | (f2h(pb) << 16);
  }
}

hipError_t launch_tq3_attn(const AttnArgs& a, int mode, uint16_t* out, hipStream_t stream);
// Scratch of the allocation-free TQ3 decode (attn_tq3.hip): this device's copy
// of a file-scope device array of kNoAllocScratchBytes.  The first call for a
// device (that device current) looks its address up; with `clear`, or on that
// first call, the scratch is zero-filled on `stream` (a fill kernel).
constexpr size_t kNoAllocScratchBytes = 8u << 20;
hipError_t noalloc_scratch(int device, bool clear, hipStream_t stream, void** ptr);
hipError_t launch_q8_attn_split(const AttnArgs& a, hipStream_t stream);
hipError_t launch_q8_attn_fast(const AttnArgs& a, uint16_t* out, hipStream_t stream);
hipError_t launch_q8k_tq3v_attn_fast(const AttnArgs& a, uint16_t* out, hipStream_t stream);
hipError_t launch_q8_attn_fast_append(const AttnArgs& a, uint16_t* out, hipStream_t stream);
hipError_t launch_split_merge(const float* m, const float* l, const float* o, uint16_t* out,
                              int num_q, int sub_n, int sub_n_max, int k_splits,
                              hipStream_t stream);
size_t tq3_attn_lds_bytes();

}  // namespace qkv
