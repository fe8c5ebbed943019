// attn_tq3.hip -- split-K flash decode over the packed TQ3 cache (gfx950).
//
// Reference semantics: flash_attn_chunk_fused_split_tq3 (attention.cuh:1905-2177)
// and flash_attn_split_merge (attention.cuh:1837-1891).
//
// Design (not the reference's): attention runs in the rotated domain.  With
// R = rs*H*D (orthogonal, D = signs, H = Sylvester Hadamard), a stored block
// decodes to k = norm * R^T c[idx], so q.k = norm * (R q).c[idx]: the query is
// rotated once per workgroup and keys are never inverse-transformed.  Values
// accumulate sum_t p_t norm_t c[idx_t] in rotated coordinates and each output
// row is rotated back once.
//
// Workgroup: 8 waves (two per SIMD) on one kv head and one key chunk; each
// wave takes 64-key tiles.  The first wave of each SIMD issues its first
// tile's loads before the second, so that its tile arrives first and is
// computed while the second one streams.  Per tile:
//   scores  v_mfma_f32_16x16x32_f16, A = key codes of 16 keys x 32 dims, B =
//           rotated query (columns = heads, held in 32 VGPRs for the whole
//           kernel; the fp16 rounding and the remainder of the query either
//           share the 16 columns, or, for calls with more than 8 / GQA
//           queries, fill them with 16 / GQA queries each, the remainders
//           read from LDS into a second product chained onto the first):
//           lane (key, octet o) reads the 12 aligned bytes holding
//           code groups 4o..4o+3 of each 128-block and decodes centroid pairs
//           through a per-lane LDS table.  One accumulator per 128-block, each
//           scaled by its block norm (which carries the softmax scale).
//   softmax online, per head, base 2.
//   values  v_mfma_f32_16x16x32_f16, A = p*norm (fp16, the lane's own
//           probabilities), B = codes of 32 keys x 16 dims.  The wave's value
//           rows are loaded with aligned 16-byte loads (lane = key) and staged
//           in LDS; lane (n, o) gathers dim group n of both blocks for 8 keys
//           and interleaves the codes of key pairs (bit select), so that each
//           table entry read is a B dword (two keys, one dim); the table
//           reads run two steps ahead.
// Merging: the 8 waves merge in LDS and each merged piece goes straight to
// its record {m, l, tags} + o[256] (rotated); the tags are set once the
// workgroup's data stores are complete.  The last workgroups of the grid are
// designated mergers, one per (q head, query, 128-block) unit: each polls its
// unit's tags (bounded), clears them, reads the rows in one round of 16-byte
// loads, merges, rotates back and stores fp16 (attn_fastmerge.h).  Only
// mergers wait, so progress does not depend on workgroup co-residency.  Paged
// (ragged) launches split each kv head's record shares over the slots in
// proportion to their key counts.  Split API: one workgroup per reference
// split, written in the reference partial layout.
#include <mutex>
#include <type_traits>

#include "qkv_device.h"
#include "attn_common.h"
#include "attn_fastmerge.h"
#include "qkv_launch.h"
#include "tq3_encode.h"

namespace qkv {

typedef uint32_t u32_a1 __attribute__((aligned(1)));

constexpr int kTile = 64;
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kHD = 256;

// Phase stamps of the fast path (a diagnostic build, compiled with
// -DQKV_PHASE_TRACE; the product build has none of this).  Every wave keeps
// s_memrealtime values (100 MHz, one clock for the whole GPU) at the phase
// boundaries below in registers and stores them once, at the end of the
// kernel, to qkv_phase_stamps[workgroup][wave][16]; slot 15 holds the XCD
// the workgroup ran on.  Workgroups past kTraceMaxWgs are not recorded.
enum TracePhase {
  kPhEntry = 0,      // kernel entry
  kPhQuery = 1,      // the query has arrived
  kPhSetup = 2,      // table and rotated query ready (setup barrier passed)
  kPhScores = 3,     // the wave's first tile: scores done
  kPhSoftmax = 4,    // the wave's first tile: staging and softmax done
  kPhTiles = 5,      // every tile of the wave done
  kPhMerged = 6,     // in-workgroup merge done (records stored)
  kPhPublished = 7,  // tags stored
  kPhPolled = 8,     // mergers: every record of the unit seen
  kPhEnd = 9,        // the workgroup is done (mergers: output stored)
  kPhMergeBar = 10,  // in-workgroup merge: every wave's rows are in LDS (barrier passed)
  kPhRowsIn = 11,    // mergers: the unit's record rows have arrived
  kPhFolded = 12,    // mergers: the waves' partials are folded (before normalise/rotate/store)
  kPhSetupWork = 13, // the wave's setup work done (before the setup barrier)
  kPhTileBar = 14,   // every wave's tiles done (the barrier before the in-workgroup merge)
  kPhXcd = 15
};
#ifdef QKV_PHASE_TRACE
constexpr int kTraceMaxWgs = 4096;
__device__ uint64_t qkv_phase_stamps[kTraceMaxWgs * kWaves * 16];
#define QKV_STAMP(k) (trace_st[k] = __builtin_amdgcn_s_memrealtime())
#else
#define QKV_STAMP(k) ((void)0)
#endif

// Per-wave staging of one 64-key tile, in dwords; every row holds 64 keys
// (key = position in the tile) at a pitch of 68, so 16 lanes reading 16-byte
// pieces of 16 different rows hit 16 disjoint bank quads.
constexpr int kKeyPitch = 68;
constexpr int kStCodes = 0;                  // [block j][group g] rows: value code group g (3 bytes, dword-expanded)
constexpr int kStVn = 32 * kKeyPitch;        // [block j] rows: value block norms
constexpr int kStKn = 34 * kKeyPitch;        // [block j] rows: key block norms
constexpr int kStCorr = 36 * kKeyPitch;      // 16 floats: per-head rescale of the accumulators
constexpr int kStageBytes = (36 * kKeyPitch + 16) * 4;   // 9856

// LDS layout (bytes).  The merge area aliases the staging areas (used after the loop).
// Centroid-pair table, one copy per lane: entry E of lane L at byte
// E * 256 + 4 * L, so every lane reads its own bank and a wave's 64 lookups
// never conflict.  An address is 4 * L in byte 0 and an 8-bit index in byte 1,
// written by one SDWA shift (sdwa_index): the low 6 bits of the index are two
// 3-bit codes, the top 2 bits are whatever follows them in the code stream,
// so entry E holds the pair of E & 63.  The table sits at LDS offset 0 so
// that no base has to be added (256 x 64 x 4 B = 64 KiB).
constexpr int kLdsLut = 0;
constexpr int kLdsLutBytes = 256 * 64 * 4;
constexpr int kLdsStage = kLdsLut + kLdsLutBytes;            // per wave, kStageBytes
constexpr int kLdsQ = kLdsStage + kWaves * kStageBytes;      // rotated query, 512 x 16 B (q_unit)
constexpr int kLdsTileEnd = kLdsQ + 16 * 256 * 2;
// After the tile loop the table and the staging areas are free: the merge
// area starts at 0.
constexpr int kLdsMergeO = 0;                                // [waves][16 rows][256] f32
constexpr int kLdsMergeML = kLdsMergeO + kWaves * 16 * kHD * 4;
constexpr int kLdsMergeEnd = kLdsMergeML + 512 * 4;
// one-query step with its token appended in the launch: the new key's
// encoded K and V blocks (4 x 13 dwords)
constexpr int kLdsNewRow = kLdsTileEnd;
constexpr int kLdsTotal = kLdsNewRow + 256;
static_assert(kLdsMergeEnd <= kLdsQ, "merge area must not reach the query scratch");
static_assert(kTracePolledByte >= kWaves * 128 * 4 && kTracePolledByte + 24 <= kLdsMergeML - kLdsMergeO,
              "the merger's trace slot lies in the merge area, past the reduction area");

// merge-area float offsets (ML): m[w][16], l[w][16], M[16], L[16]
constexpr int kMlW0 = 0, kMlLw0 = 16 * kWaves, kMlM = 32 * kWaves, kMlL = 32 * kWaves + 16;
static_assert(kMlL + 16 <= 512, "merge scalars must fit the ML area");

// 16-byte unit of the rotated-query scratch holding elements 8(4o+u)..+7 of
// 128-block j of column c, s = 4j + u.  The column is swizzled with (u, o) so
// that the 16 lanes of one WHT writing (fixed c, j) and the 16 lanes of one
// MFMA row reading (fixed s, o) each touch 16 distinct 16-byte bank groups.
__device__ __forceinline__ int q_unit(int c, int s, int o) {
  return (s * 4 + o) * 16 + (c ^ (4 * (s & 3) + o));
}

__device__ __forceinline__ uint32_t lut_read(const uint8_t* lds, uint32_t addr) {
  return *reinterpret_cast<const uint32_t*>(lds + kLdsLut + addr);
}

// Table address of the 6-bit field at bit BIT of a 3-dword code stream
// (a field that crosses a dword boundary is first funnel-shifted to bit 0).
template <int BIT>
__device__ __forceinline__ uint32_t pair_addr3(uint32_t& chain, const uint32_t (&q)[3]) {
  constexpr int w = BIT >> 5, sh = BIT & 31;
  if constexpr (sh + 6 <= 32)
    chain = sdwa_index<sh>(chain, q[w]);
  else
    chain = sdwa_index<0>(chain, __builtin_amdgcn_alignbit(q[w + 1], q[w], sh));
  return chain;
}

// B operand for code group U (8 codes, bits 24U..24U+23) of a 3-dword stream.
template <int U>
__device__ __forceinline__ h8_t group_operand(const uint8_t* lds, uint32_t (&ac)[4],
                                              const uint32_t (&q)[3]) {
  u4_t v;
  v[0] = lut_read(lds, pair_addr3<24 * U + 0>(ac[0], q));
  v[1] = lut_read(lds, pair_addr3<24 * U + 6>(ac[1], q));
  v[2] = lut_read(lds, pair_addr3<24 * U + 12>(ac[2], q));
  v[3] = lut_read(lds, pair_addr3<24 * U + 18>(ac[3], q));
  return __builtin_bit_cast(h8_t, v);
}

// Score MFMAs for one 16-key group: 4 slices per block, one accumulator per
// block.  Slice U+1's table reads are issued before slice U's MFMAs.
// CHAIN: the query remainders (lo) have MFMA columns of their own in a second
// product chained onto the same accumulator; slice s of this lane's lo
// operand is at LDS byte qlo + 1024 s.
template <int U, bool CHAIN>
__device__ __forceinline__ void score_group(const uint8_t* lds, uint32_t (&ac)[4], const uint32_t (&k0)[3],
                                            const uint32_t (&k1)[3], const h8_t (&qa)[8],
                                            uint32_t qlo,
                                            const h8_t& b0, const h8_t& b1, f4_t& a0, f4_t& a1) {
  if constexpr (U < 4) {
    h8_t n0, n1, l0, l1;
    if constexpr (CHAIN) {
      l0 = *reinterpret_cast<const h8_t*>(lds + qlo + 1024 * U);
      l1 = *reinterpret_cast<const h8_t*>(lds + qlo + 1024 * (4 + U));
    }
    if constexpr (U < 3) {
      n0 = group_operand<U + 1>(lds, ac, k0);
      n1 = group_operand<U + 1>(lds, ac, k1);
    }
    a0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(b0, qa[U], a0, 0, 0, 0);
    a1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(b1, qa[4 + U], a1, 0, 0, 0);
    if constexpr (CHAIN) {
      a0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(b0, l0, a0, 0, 0, 0);
      a1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(b1, l1, a1, 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (U < 3) score_group<U + 1, CHAIN>(lds, ac, k0, k1, qa, qlo, n0, n1, a0, a1);
  }
}

// One value pass: a (32-key chunk c2, 128-block j) pair.  MFMA k index i of
// the pass is key 32*c2 + 4*row + i (i < 4) or 32*c2 + 16 + 4*row + i - 4.
// x: the code group `col` (8 dims, 24 bits) of key i as loaded; from the
// pass's first table reads on (interleave_pairs), the codes of keys 2k and
// 2k + 1 interleaved per dim, so that one 6-bit field is a table index whose
// entry is already the B dword (key 2k in the low half, key 2k + 1 in the
// high half): x[k] holds dims 0, 2, 4, 6 (field 6d: codes of dim 2d),
// x[4 + k] dims 1, 3, 5, 7 (field 6d + 3: codes of dim 2d + 1).
// a: A operand (p * value norm of those keys, head `col`).
struct ValuePass {
  uint32_t x[8];
  h8_t a;
};

// Dims 0, 2, 4, 6 of a 24-bit code group (bits 6d .. 6d + 2).
constexpr uint32_t kEvenDims = 0x1C71C7u;

// (a & m) | (b & ~m) in one v_bfi_b32 (the compiler splits some constant
// masks into an and plus an and-or)
__device__ __forceinline__ uint32_t bit_select(uint32_t m, uint32_t a, uint32_t b) {
  uint32_t d;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(d) : "s"(m), "v"(a), "v"(b));
  return d;
}

// Codes and A operand of pass c = 2*c2 + j from the tile's staging area.
__device__ __forceinline__ void value_pass_load(const float* st, const uint32_t* stu, int c, int row,
                                                int col, const float (&s)[4][4], ValuePass& vp) {
  const int c2 = c >> 1, j = c & 1;
  const f4_t va = *reinterpret_cast<const f4_t*>(st + kStVn + j * kKeyPitch + 32 * c2 + 4 * row);
  const f4_t vb = *reinterpret_cast<const f4_t*>(st + kStVn + j * kKeyPitch + 32 * c2 + 16 + 4 * row);
  const u4_t xa = *reinterpret_cast<const u4_t*>(stu + kStCodes + (16 * j + col) * kKeyPitch + 32 * c2 + 4 * row);
  const u4_t xb =
      *reinterpret_cast<const u4_t*>(stu + kStCodes + (16 * j + col) * kKeyPitch + 32 * c2 + 16 + 4 * row);
#pragma unroll
  for (int r = 0; r < 4; r++) {
    vp.a[r] = (_Float16)(s[2 * c2][r] * va[r]);
    vp.a[4 + r] = (_Float16)(s[2 * c2 + 1][r] * vb[r]);
    vp.x[r] = xa[r];
    vp.x[4 + r] = xb[r];
  }
}

// Key pairs (i, i + 1) = (2k, 2k + 1) of a pass's codes as loaded (x[i]: key
// i's code group): the second key's codes moved up by one code, merged with
// the first key's by bit select.  Done in place at the pass's first table
// reads, two steps after its staging loads were issued.
__device__ __forceinline__ void interleave_pairs(uint32_t (&x)[8]) {
  uint32_t z[8];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const uint32_t hi = x[2 * k + 1] << 3;
    z[k] = bit_select(kEvenDims, x[2 * k], hi);
    z[4 + k] = bit_select(kEvenDims << 3, x[2 * k], hi);
  }
#pragma unroll
  for (int i = 0; i < 8; i++) x[i] = z[i];
}

// Table reads of dims 2PP (cp[0..3]) and 2PP+1 (cp[4..7]) of the 4 key pairs:
// each entry is a B dword (two keys, one dim).
template <int PP>
__device__ __forceinline__ void value_pairs(const uint8_t* lds, uint32_t (&ac)[4], uint32_t (&x)[8],
                                            uint32_t (&cp)[8]) {
  if constexpr (PP == 0) interleave_pairs(x);
#pragma unroll
  for (int k = 0; k < 4; k++) {
    ac[k] = sdwa_index<6 * PP>(ac[k], x[k]);
    cp[k] = lut_read(lds, ac[k]);
  }
#pragma unroll
  for (int k = 0; k < 4; k++) {
    ac[k] = sdwa_index<6 * PP + 3>(ac[k], x[4 + k]);
    cp[4 + k] = lut_read(lds, ac[k]);
  }
}

// Step K of the value phase (pass c = K / 4, centroid pair PP = K % 4): tiles
// 8j + 2PP (low dim) and 8j + 2PP + 1 (high dim).  Software-pipelined two
// steps deep: the table reads of step K+2 are issued before the perms and
// MFMAs of step K (cp: step K's pairs, cq: step K+1's), and the codes and A
// operand of pass c+1 are read during the first step of pass c.
// FIRST: the workgroup's first tile, whose passes 0 and 1 write every
// accumulator tile for the first time (zero C operand).
template <int K, bool FIRST>
__device__ __forceinline__ void value_steps(const uint8_t* lds, uint32_t (&ac)[4], ValuePass (&vp)[2],
                                            const uint32_t (&cp)[8], const uint32_t (&cq)[8],
                                            f4_t (&acc)[16], const float* st, const uint32_t* stu, int row,
                                            int col, const float (&s)[4][4]) {
  if constexpr (K < 16) {
    constexpr int c = K >> 2, PP = K & 3;
    if constexpr (PP == 0 && c < 3) value_pass_load(st, stu, c + 1, row, col, s, vp[(c + 1) & 1]);
    uint32_t cn[8];
    if constexpr (K + 2 < 16) value_pairs<(K + 2) & 3>(lds, ac, vp[((K + 2) >> 2) & 1].x, cn);
#pragma unroll
    for (int e = 0; e < 2; e++) {
      u4_t bv;
#pragma unroll
      for (int k2 = 0; k2 < 4; k2++) bv[k2] = cp[4 * e + k2];
      constexpr int t0 = 8 * (c & 1) + 2 * PP;
      const f4_t cin = (FIRST && c < 2) ? f4_t{0.f, 0.f, 0.f, 0.f} : acc[t0 + e];
      acc[t0 + e] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vp[c & 1].a, __builtin_bit_cast(h8_t, bv),
                                                           cin, 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (K < 15) value_steps<K + 1, FIRST>(lds, ac, vp, cq, cn, acc, st, stu, row, col, s);
  }
}

// Registers of one 64-key tile.  Buffer loads: offsets are 32-bit and reads
// past the cache extent (num_records) return zero, so partial tiles need no
// branches; keys in [hi, extent) are read and masked out of the softmax.
struct TileRegs {
  u4_t vr[6];            // value row of key ts+lane (dwords 0..23)
  u2_t vr6;              // dwords 24..25
  uint32_t kq[4][2][3];  // key code groups 4*row..4*row+3, group g, block j
  float kn[4][2];        // key block norms, group g, block j
};

// prow: cache row of the tile's first key (64 consecutive rows, wave-uniform);
// the buffer resources are rebased at that row (64-bit byte offset)
__device__ __forceinline__ void load_tile(const AttnArgs& p, int prow, int nkv, int h, int lane,
                                          int row, int col, TileRegs& tr) {
  const uint64_t off0 = (uint64_t)(uint32_t)prow * (uint32_t)nkv * 104u;
  const __amdgpu_buffer_rsrc_t rk = cache_rsrc(p.k, off0, p.kv_bytes);
  const __amdgpu_buffer_rsrc_t rv = cache_rsrc(p.v, off0, p.kv_bytes);
  // keys first (group by group): the score MFMAs of group g only wait for
  // group g, and values arrive while the scores are computed
#pragma unroll
  for (int g = 0; g < 4; g++) {
    const uint32_t krow = (uint32_t)((16 * g + col) * nkv + h) * 104u;
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const u3_t c = __builtin_amdgcn_raw_buffer_load_b96(rk, krow + 52 * j + 4 + 12 * row, 0, 0);
      tr.kq[g][j][0] = c[0];
      tr.kq[g][j][1] = c[1];
      tr.kq[g][j][2] = c[2];
      tr.kn[g][j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rk, krow + 52 * j, 0, 0));
    }
  }
  const uint32_t vrow = (uint32_t)(lane * nkv + h) * 104u;
#pragma unroll
  for (int i = 0; i < 6; i++) tr.vr[i] = __builtin_amdgcn_raw_buffer_load_b128(rv, vrow + 16 * i, 0, 0);
  tr.vr6 = __builtin_amdgcn_raw_buffer_load_b64(rv, vrow + 96, 0, 0);
}

// The encoded new key (4 x 13 dwords at nr) written over the registers of
// the tile that holds it, r = its index in the tile: lanes (row, col = r & 15)
// of its 16-key group take its key code pieces and norms, lane r its value row
// (constant register indices).
__device__ __forceinline__ void patch_new_key(TileRegs& tr, const uint32_t* nr, int r, int lane, int row,
                                              int col) {
  const int g = r >> 4;
  if (col == (r & 15)) {
#pragma unroll
    for (int G = 0; G < 4; G++) {
#pragma unroll
      for (int j = 0; j < 2; j++) {
        tr.kq[G][j][0] = g == G ? nr[13 * j + 1 + 3 * row] : tr.kq[G][j][0];
        tr.kq[G][j][1] = g == G ? nr[13 * j + 2 + 3 * row] : tr.kq[G][j][1];
        tr.kq[G][j][2] = g == G ? nr[13 * j + 3 + 3 * row] : tr.kq[G][j][2];
        tr.kn[G][j] = g == G ? __uint_as_float(nr[13 * j]) : tr.kn[G][j];
      }
    }
  }
  if (lane == r) {
#pragma unroll
    for (int i = 0; i < 6; i++) tr.vr[i] = u4_t{nr[26 + 4 * i], nr[27 + 4 * i], nr[28 + 4 * i], nr[29 + 4 * i]};
    tr.vr6 = u2_t{nr[50], nr[51]};
  }
}

// Key visibility of one query (attention.cuh:1923-1929, 2101-2105): the
// sink/window rule on 32-key tiles, then the tree bits for keys of the block.
// Branch-free: every key of a tile is tested with the same instructions.
struct KeyRule {
  int start_pos, sink, window;
  bool sw, has_tree;
  uint32_t tree_bits;   // bit j: key start_pos + j is visible
  __device__ KeyRule(int start_pos_, int t_idx, int sink_, int window_, const uint32_t* tree)
      : start_pos(start_pos_), sink(sink_), window(window_), sw(sink_ > 0 || window_ > 0),
        has_tree(tree != nullptr), tree_bits(tree ? tree[t_idx] : 0u) {}
  // every key of [a, b) is visible (no rule applies there)
  __device__ __forceinline__ bool all_visible(int b) const {
    return !sw && (!has_tree || b <= start_pos);
  }
  __device__ __forceinline__ bool visible(int key, int active_end) const {
    const int ts = key & ~31;
    const int te = min(ts + 32, active_end);
    const bool sw_ok = !sw | (ts < sink) | (te > active_end - window);
    const bool tree_ok = !has_tree | (key < start_pos) |
                         (((tree_bits >> ((key - start_pos) & 31)) & 1u) != 0u);
    return sw_ok & tree_ok;
  }
};

// max / sum inside each 16-lane row (all lanes of the row receive the result)
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x124>(v));
  v = fmaxf(v, dpp_f<0x128>(v));
  return v;
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x124>(v);
  v += dpp_f<0x128>(v);
  return v;
}

// Max / sum over the 4 rows of the wave (lanes l, l^16, l^32, l^48); every
// lane receives the result.  Each gfx950 row swap leaves a lane holding its
// own value and its partner row's value in the two registers.
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

// Rotate the merged rows back (o = rs*D*H*o_rot per 128-block).  final: divide
// by L and store fp16 rows [t][q_head][256]; otherwise store the unnormalised
// f32 partial of reference split `split` (m in natural-log units).
__device__ void finish_rows(const uint8_t* lds, const AttnArgs& p, int h, int t, int rows,
                            bool final, int split, uint16_t* out) {
  const float* mo = reinterpret_cast<const float*>(lds + kLdsMergeO);
  const float* ml = reinterpret_cast<const float*>(lds + kLdsMergeML);
  const int gqa = p.num_q / p.num_kv;
  const int lane = threadIdx.x & 63;
  for (int w0 = 0; w0 < rows * 2; w0 += kThreads / 16) {
    const int wht = w0 + (threadIdx.x >> 4);
    const int part = threadIdx.x & 15;
    const int r = wht >> 1, blk = wht & 1;
    const bool live = wht < rows * 2;
    const float L = live ? ml[kMlL + r] : 0.f;
    // the centroid table is scaled by kCenScale: undo it here (fp32)
    const float scale = (final ? (L > 0.f ? 1.0f / L : 0.f) : 1.0f) * kCenScaleInv;
    float x[8];
#pragma unroll
    for (int i = 0; i < 8; i++) x[i] = live ? mo[r * kHD + blk * 128 + part * 8 + i] * scale : 0.f;
    wht8_inreg(x);
    wht_xor_lanes16(x, lane);
    if (!live) continue;
    const float rs = wht_scale();
    const int qh = h * gqa + r % gqa, tq = t + r / gqa;
    float y[8];
    const uint32_t sbits = sign_word_sel(part >> 2) >> (8 * (part & 3));  // elements part*8..+7
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const bool pos = (sbits >> i) & 1u;
      const float v = x[i] * rs;
      y[i] = pos ? v : -v;
    }
    if (final) {
      uint32_t pk[4];
#pragma unroll
      for (int i = 0; i < 4; i++) pk[i] = f2h(y[2 * i]) | (f2h(y[2 * i + 1]) << 16);
      *reinterpret_cast<uint4*>(out + ((long)tq * p.num_q + qh) * kHD + blk * 128 + part * 8) =
          make_uint4(pk[0], pk[1], pk[2], pk[3]);
    } else {
      const long mlx = ((long)qh * p.sub_n_max + tq) * p.k_splits + split;
#pragma unroll
      for (int i = 0; i < 8; i++) p.part_o[mlx * kHD + blk * 128 + part * 8 + i] = y[i];
      if (blk == 0 && part == 0) {
        const float M = ml[kMlM + r];
        p.part_m[mlx] = (M == -INFINITY) ? -INFINITY : M * kLn2;
        p.part_l[mlx] = ml[kMlL + r];
      }
    }
  }
}

// MODE 0: fast path (final fp16 rows).  MODE 1: reference split partials.
// MODE 2: block-sparse split partials (attention.cuh:2193-2433): one query
// per workgroup (qpw = 1), split z over the query's selected 64-key blocks.
// CHAIN (fast path, several queries): 16 / GQA queries per workgroup, every
// MFMA column a real (query, head); the remainders ride in a chained second
// score product (see score_group).
// APPEND (MODE 0, one query): the step's new token is encoded in the launch
// (qkv_decode_attn_tq3_append), a separate instance so that the plain decode
// compiles without it.
template <int MODE, bool CHAIN = false, bool APPEND = false>
__global__ __launch_bounds__(kThreads, 1) void tq3_attn_kernel(QKV_ATTN_LEAD_PARAMS, AttnArgs pin,
                                                                uint16_t* out) {
  QKV_ATTN_LEAD_APPLY(p, pin);
  const bool paged = (lead_flags & (1u << 8)) != 0, ragged = (lead_flags & (1u << 9)) != 0;
  // static LDS: table and tile offsets fold into the instructions' offset field
  __shared__ __attribute__((aligned(16))) uint8_t lds[kLdsTotal];
#ifdef QKV_PHASE_TRACE
  uint64_t trace_st[15] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
#endif
  QKV_STAMP(kPhEntry);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int gqa = __builtin_amdgcn_readfirstlane(p.num_q / p.num_kv);   // scalar register

  // ---- work id (XCD-aware: the num_kv workgroups of one (query group, chunk)
  // share an XCD).  A workgroup serves queries t0 .. t0+nq-1 (nq <= qpw) of
  // one kv head: MFMA column c = qi * gqa + hh is q head h*gqa + hh of query
  // t0 + qi (columns past nq * gqa carry nothing).
  int h, t0, chunk;
  int rec_t0, rec_chunk;      // record coordinates of this workgroup's rows
  int chunk_keys = p.chunk_keys;
  bool has_work;
  {
    const int L = blockIdx.x;
    const int xcd = L & 7, r = L >> 3;
    h = r % p.num_kv;
    const int g = (r / p.num_kv) * 8 + xcd;
    const int groups = (p.sub_n + p.qpw - 1) / p.qpw;
    has_work = g < groups * p.n_chunks;
    if (MODE == 0 && ragged) {
      // ragged slots (one query each): share g of the length-proportional split
      int first, count;
      const int s = has_work ? share_slot(p, g, first, count) : -1;
      has_work = s >= 0;
      t0 = has_work ? s : 0;
      chunk = has_work ? g - first : 0;
      if (has_work) {   // the slot's keys in count chunks of whole 512-key steps
        const int per = (slot_keys(p, s) + count - 1) / count;
        chunk_keys = max(1, (per + kWaves * kTile - 1) / (kWaves * kTile)) * (kWaves * kTile);
      }
      rec_t0 = 0;
      rec_chunk = g;
    } else {
      const int tq = has_work ? g / p.n_chunks : 0;
      chunk = has_work ? g - tq * p.n_chunks : 0;
      t0 = tq * p.qpw;
      rec_t0 = t0;
      rec_chunk = chunk;
    }
  }
  if (MODE >= 1 && !has_work) return;
  const int nq = min(p.qpw, p.sub_n - t0);
  // accumulator rows (columns) that hold heads (uniform: kept in a scalar register)
  const int rows_used = __builtin_amdgcn_readfirstlane(nq * gqa);
  const int row = lane >> 4;        // 16-lane row of the MFMA D layout
  const int col = lane & 15;
  const int t_col = t0 + min(col / gqa, nq - 1);   // this lane's query (clamped for dead columns)
  // ---- the query load goes out first: its address depends only on the
  // preloaded arguments
  // 32 WHTs of 128 (16 columns x 2 blocks), 16 lanes each
  const int q_wht = threadIdx.x >> 4;
  const int q_part = threadIdx.x & 15;
  const int q_col = q_wht >> 1, q_blk = q_wht & 1;   // column, 128-block
  u4_t q_raw;
  {
    // unconditional (rows past the buffer's extent read as zero): a load
    // under a branch makes the compiler wait for every load at the join
    const uint32_t q_extent = (uint32_t)(p.sub_n * p.num_q * kHD * 2);
    const __amdgpu_buffer_rsrc_t rq =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p.q), 0, q_extent, kBufferRsrcWord3);
    const uint32_t qoff =
        q_col < rows_used ? (uint32_t)((((t0 + q_col / gqa) * p.num_q + h * gqa + q_col % gqa) * kHD +
                                        q_blk * 128 + q_part * 8) * 2)
                          : q_extent;
    q_raw = __builtin_amdgcn_raw_buffer_load_b128(rq, qoff, 0, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
  // key counts: the lane's own query, and the first / last query of the group
  // (a paged group has one query)
  const int active_end = ragged ? min(max(p.ctx_lens[t_col], 0), p.ctx_max)
                                    : p.start_pos + t_col + 1;
  const int active_first = ragged ? active_end : p.start_pos + t0 + 1;
  const int active_last = ragged ? active_end : p.start_pos + t0 + nq;
  int lo = 0, hi = 0, hi_col = 0, hi_first = 0;
  if (MODE == 0) {
    if (has_work) {
      lo = chunk * chunk_keys;
      // the last chunk of a contiguous launch runs to the end of the keys: the
      // host may have joined a remainder of at most one tile to it
      const int c_end = (!ragged && chunk == p.n_chunks - 1) ? active_last : lo + chunk_keys;
      hi = min(c_end, active_last);
      hi_col = min(c_end, active_end);
      hi_first = min(c_end, active_first);
    }
  } else if (MODE == 2) {
    // the selected blocks bound the keys; the query's causal end masks them
    lo = 0;
    hi = active_end;
    hi_col = active_end;
    hi_first = active_end;
  } else {
    // reference split range (attention.cuh:1944-1951)
    const int total_tiles = (p.active_end_max + 31) / 32;
    const int tps = (total_tiles + p.k_splits - 1) / p.k_splits;
    lo = chunk * tps * 32;
    hi = min((chunk + 1) * tps * 32, active_last);
    hi_col = min((chunk + 1) * tps * 32, active_end);
    hi_first = min((chunk + 1) * tps * 32, active_first);
  }
  lo = __builtin_amdgcn_readfirstlane(lo);
  hi = __builtin_amdgcn_readfirstlane(hi);
  hi_first = __builtin_amdgcn_readfirstlane(hi_first);
  // appended token (one-query launches of qkv_decode_attn_tq3_append): the
  // wave whose tiles hold key start_pos (tile k of wave w starts at lo + 64w
  // + k * 512), and its input, lane l: 16-byte piece l & 15 of block l >> 4
  // (K block 0, K block 1, V block 0, V block 1 of kv head h)
  int fa_wave = -1;
  uint4 fa_raw = make_uint4(0u, 0u, 0u, 0u);
  if constexpr (APPEND) {
    if (p.k_new != nullptr && has_work && lo <= p.start_pos && p.start_pos < hi)
      fa_wave = ((p.start_pos - lo) >> 6) & (kWaves - 1);
    fa_wave = __builtin_amdgcn_readfirstlane(fa_wave);
    if (fa_wave == wave) {
      const int blk = lane >> 4;
      fa_raw = *reinterpret_cast<const uint4*>((blk < 2 ? p.k_new : p.v_new) + h * kHD + (blk & 1) * 128 +
                                               8 * (lane & 15));
    }
  }
  // A dead column has a zero query: its scores are 0 and its accumulator rows
  // are never stored, so it needs no mask of its own.

  // ---- setup: centroid-pair table, rotated query --------------------------
  // The query is loaded and rotated before any tile load is issued: a query
  // load issued after the tile loads of the whole chip would wait behind
  // them in the memory queues.
  // paged caches: the block-table entries of this wave's first 64 tiles (lane
  // k: tile k, key lo + wave*64 + k*kStep), loaded now so that no tile load
  // waits for a table read (rows past the table's extent read as 0)
  constexpr int kStep = kWaves * kTile;
  // block-sparse: lane k holds entry k of this split's block list; the list
  // ends at its first -1 (n_sel entries); wave w takes entries w, w + 8, ...
  int sel = -1, n_sel = 0;
  if constexpr (MODE == 2) {
    const int per = (p.top_k + p.k_splits - 1) / p.k_splits;
    const int tk_lo = chunk * per, tk_n = max(0, min(per, p.top_k - tk_lo));
    const __amdgpu_buffer_rsrc_t rbi = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int32_t*>(p.block_index), 0, (uint32_t)(p.num_kv * p.sub_n_max * p.top_k * 4),
        kBufferRsrcWord3);
    // unconditional load (an out-of-range offset reads 0), masked after
    const uint32_t off = lane < tk_n
        ? (uint32_t)((((h * p.sub_n_max + t0) * p.top_k) + tk_lo + lane) * 4) : 0xffffffffu;
    const int ld = (int)__builtin_amdgcn_raw_buffer_load_b32(rbi, off, 0, 0);
    const int e = lane < tk_n ? ld : -1;
    const uint64_t ends = __builtin_amdgcn_ballot_w64(e < 0);
    n_sel = ends ? (int)__builtin_ctzll(ends) : 64;
    sel = e;
  }
  const int ts0 = MODE == 2 ? (wave < n_sel ? __builtin_amdgcn_readlane(sel, wave) * kTile : 0)
                            : lo + wave * kTile;
  const __amdgpu_buffer_rsrc_t rbt = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int32_t*>(p.block_tables), 0,
      p.block_tables ? (uint32_t)(p.sub_n * p.bt_stride * 4) : 0u, kBufferRsrcWord3);
  auto bt_batch = [&](int k0) -> int {   // entries of tiles k0 .. k0+63 (one per lane)
    const int ts = ts0 + (k0 + lane) * kStep;
    int bt = __builtin_amdgcn_readfirstlane(max(p.block_tokens, 1));
    asm volatile("" : "+s"(bt));   // (divisor re-read per batch, not held through the loop)
    const uint32_t off = ts < hi ? (uint32_t)((t0 * p.bt_stride + ts / bt) * 4) : 0xffffffffu;
    return (int)__builtin_amdgcn_raw_buffer_load_b32(rbt, off, 0, 0);
  };
  int bt_entry = paged ? bt_batch(0) : 0, bt_k0 = 0;
  // cache row of this wave's tile starting at key ts: ts itself for a
  // contiguous cache; through the query's block table for a paged one (block
  // sizes are multiples of 64, so a 64-key tile never straddles two blocks);
  // rows outside the cache extent read as zero (buffer range checks)
  auto wave_tile_row = [&](int ts) -> int {
    if (!paged) return ts;
    if (ts >= hi) return 0;
    const int k = (ts - ts0) / kStep;
    if (k - bt_k0 >= 64) {
      bt_k0 = k & ~63;
      bt_entry = bt_batch(bt_k0);
    }
    const int e = __builtin_amdgcn_readlane(bt_entry, k - bt_k0);
    // (the divisor re-read per tile instead of held through the loop)
    int bt = __builtin_amdgcn_readfirstlane(p.block_tokens);
    asm volatile("" : "+s"(bt));
    const int b = ts / bt;
    return e * bt + (ts - b * bt);
  };
  // waves 0..3 issue their first tile's loads as soon as the query has
  // arrived (so it does not queue behind them), ahead of the table build
  // and the rotation; waves 4..7 issue theirs after the setup barrier.
  __builtin_amdgcn_s_waitcnt(0);
  QKV_STAMP(kPhQuery);
  TileRegs tr;
  if (wave < 4) load_tile(p, wave_tile_row(ts0), p.num_kv, h, lane, row, col, tr);
  // centroid-pair table: entry e = (centroid[e & 7], centroid[(e >> 3) & 7])
  // as fp16, from immediates (wave-uniform values); wave w writes every lane's
  // copy of entries 32w .. 32w+31
  static_assert(kWaves == 8, "8 waves x 32 entries");
  const uint32_t lane4 = 4u * (uint32_t)lane;
  {
    const uint32_t w = (uint32_t)wave;
#pragma unroll
    for (int hk = 0; hk < 4; hk++) {
      const uint32_t hi = centroid_scaled_h((4u * w + hk) & 7u) << 16;
#pragma unroll
      for (int k = 0; k < 8; k++)
        *reinterpret_cast<uint32_t*>(lds + kLdsLut + (w * 32 + hk * 8 + k) * 256 + lane4) =
            centroid_scaled_h(k) | hi;
    }
  }
  uint32_t ac[4] = {lane4, lane4, lane4, lane4};   // table address chains
  uint32_t q_lo[4] = {0u, 0u, 0u, 0u};              // CHAIN: this thread's query remainders
  {
    // rotated query: fp16 in LDS scratch (q_unit), so that each lane's A
    // operand slice is one 16-byte read
    // Column c < 8 holds the fp16 rounding of the rotated query (hi) and
    // column c + 8 the fp16 rounding of its remainder (lo): the score MFMA
    // computes both against the same decoded keys and the two halves are added
    // in fp32, so the rotated query is carried to ~2^-22 (real columns <= 8).
    uint16_t* qs = reinterpret_cast<uint16_t*>(lds + kLdsQ);
    const int o = q_part >> 2, u = q_part & 3;   // elements part*8..+7 = code group 4*o + u
    if (CHAIN) {
      // every column is a (query, head) of its own; the remainders stay in
      // registers until the rounded query has been read (then they replace it)
      uint32_t pk[4] = {0u, 0u, 0u, 0u};
      if (q_col < rows_used) {
        float x[8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          x[2 * i] = h2f(q_raw[i] & 0xffffu);
          x[2 * i + 1] = h2f(q_raw[i] >> 16);
        }
        const uint32_t sbits = sign_word_sel(q_part >> 2) >> (8 * (q_part & 3));
#pragma unroll
        for (int i = 0; i < 8; i++) {
          const bool pos = (sbits >> i) & 1u;
          x[i] = pos ? x[i] : -x[i];
        }
        wht8_inreg(x);
        wht_xor_lanes16(x, lane);
        const float rs = wht_scale();
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const float a = x[2 * i] * rs, b = x[2 * i + 1] * rs;
          const uint32_t ha = f2h(a), hb = f2h(b);
          pk[i] = ha | (hb << 16);
          q_lo[i] = f2h(a - h2f(ha)) | (f2h(b - h2f(hb)) << 16);
        }
      }
      *reinterpret_cast<uint4*>(qs + q_unit(q_col, 4 * q_blk + u, o) * 8) =
          make_uint4(pk[0], pk[1], pk[2], pk[3]);
    } else if (q_col >= 8) {
      // columns 8..15 are written by the waves of columns 0..7
    } else if (2 * wave >= rows_used) {
      // a wave whose two columns are both dead writes zeros (hi and lo)
      *reinterpret_cast<uint4*>(qs + q_unit(q_col, 4 * q_blk + u, o) * 8) = make_uint4(0, 0, 0, 0);
      *reinterpret_cast<uint4*>(qs + q_unit(q_col + 8, 4 * q_blk + u, o) * 8) = make_uint4(0, 0, 0, 0);
    } else {
      float x[8];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        x[2 * i] = h2f(q_raw[i] & 0xffffu);
        x[2 * i + 1] = h2f(q_raw[i] >> 16);
      }
      const uint32_t sbits = sign_word_sel(q_part >> 2) >> (8 * (q_part & 3));   // elements part*8..+7
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const bool pos = (sbits >> i) & 1u;
        x[i] = pos ? x[i] : -x[i];
      }
      wht8_inreg(x);
      wht_xor_lanes16(x, lane);
      const float rs = wht_scale();
      uint32_t pk[4], pl[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float a = x[2 * i] * rs, b = x[2 * i + 1] * rs;
        const uint32_t ha = f2h(a), hb = f2h(b);
        pk[i] = ha | (hb << 16);
        pl[i] = f2h(a - h2f(ha)) | (f2h(b - h2f(hb)) << 16);
      }
      *reinterpret_cast<uint4*>(qs + q_unit(q_col, 4 * q_blk + u, o) * 8) =
          make_uint4(pk[0], pk[1], pk[2], pk[3]);
      *reinterpret_cast<uint4*>(qs + q_unit(q_col + 8, 4 * q_blk + u, o) * 8) =
          make_uint4(pl[0], pl[1], pl[2], pl[3]);
    }
  }
  if constexpr (APPEND) {
    // the step's new token appended in this launch (qkv_decode_attn_tq3_append
    // with one query): the wave whose tile holds key start_pos encodes its
    // K and V blocks (one 16-lane row each, tq3_encode_row16), stores them
    // to the caches and keeps them in LDS for its tile registers
    if (fa_wave == wave) {
      const uint32_t word = tq3_encode_row16(fa_raw, lane);
      const int blk = lane >> 4, t = lane & 15;
      if (t <= 12) {
        const int w = t == 12 ? 0 : 1 + t;
        reinterpret_cast<uint32_t*>(lds + kLdsNewRow)[blk * 13 + w] = word;
        uint32_t* dst = reinterpret_cast<uint32_t*>(blk < 2 ? p.k_w : p.v_w) +
                        ((long)p.start_pos * p.num_kv + h) * 26 + (blk & 1) * 13 + w;
        *dst = word;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }
  QKV_STAMP(kPhSetupWork);
  __syncthreads();
  QKV_STAMP(kPhSetup);
  // (built after the setup: its tree word is a load the first loads must not wait for)
  const KeyRule rule(p.start_pos, t_col, p.sink_tok, p.window_tok, p.tree_mask);
  // ---- first tile: the first wave of each SIMD (waves 0..3) issues its loads
  // before the second (waves 4..7), so that across the chip the first waves'
  // tiles arrive in the first half of the stream and are computed while the
  // second waves' tiles are still in flight.
  if (wave >= 4) load_tile(p, wave_tile_row(ts0), p.num_kv, h, lane, row, col, tr);
  // qa[s], slice s = 4j+u: column `col`, element i = dim 128j + 8(4*row+u) + i
  h8_t qa[8];
  {
    const uint16_t* qs = reinterpret_cast<const uint16_t*>(lds + kLdsQ);
#pragma unroll
    for (int s = 0; s < 8; s++)   // dead columns were written as zeros
      qa[s] = *reinterpret_cast<const h8_t*>(qs + q_unit(col, s, row) * 8);
  }
  // CHAIN: the remainders replace the rounded query in the scratch, unswizzled
  // (written once): 16-byte unit (s * 4 + o) * 16 + c holds elements
  // 8(4o+u)..+7 of 128-block j of column c, s = 4j + u
  const uint32_t qlo = (uint32_t)(kLdsQ + row * 256 + col * 16);
  if constexpr (CHAIN) {
    __syncthreads();
    {
      const int o = q_part >> 2, u = q_part & 3;
      *reinterpret_cast<uint4*>(lds + kLdsQ + (((4 * q_blk + u) * 4 + o) * 16 + q_col) * 16) =
          make_uint4(q_lo[0], q_lo[1], q_lo[2], q_lo[3]);
    }
    __syncthreads();
  }

  const float scale2 = p.scale_log2 * kCenScaleInv;
  float m2 = -INFINITY;   // running max of head `col` (base-2 units)
  float lsum = 0.0f;      // this lane's part of the running sum of head `col`
  f4_t acc[16];

  float* st = reinterpret_cast<float*>(lds + kLdsStage + wave * kStageBytes);
  uint32_t* stu = reinterpret_cast<uint32_t*>(st);

  // One 64-key tile.  The wave's first tile is a separate instance: its loads
  // were issued with the setup, and its accumulators start at zero.
  auto tile_body = [&](auto first_tag, int ts) {
    constexpr bool first = decltype(first_tag)::value;
    auto& kq = tr.kq;
    auto& kn = tr.kn;

    // ---------------- scores: D rows = keys 16g + 4*row + r, D col = head `col` ----------------
    f4_t sa[4][2];
#pragma unroll
    for (int g = 0; g < 4; g++) {
      sa[g][0] = f4_t{0.f, 0.f, 0.f, 0.f};
      sa[g][1] = f4_t{0.f, 0.f, 0.f, 0.f};
      score_group<0, CHAIN>(lds, ac, kq[g][0], kq[g][1], qa, qlo, group_operand<0>(lds, ac, kq[g][0]),
                            group_operand<0>(lds, ac, kq[g][1]), sa[g][0], sa[g][1]);
    }

    if constexpr (first) QKV_STAMP(kPhScores);
    // ---------------- staging: key norms, value rows (lane = key ts + lane) ----------------
    if (row == 0) {
#pragma unroll
      for (int g = 0; g < 4; g++) {
        // key norms carry the softmax scale and undo the table scale
        st[kStKn + 16 * g + col] = kn[g][0] * scale2;
        st[kStKn + kKeyPitch + 16 * g + col] = kn[g][1] * scale2;
      }
    }
    {
      uint32_t d[27];
#pragma unroll
      for (int i = 0; i < 6; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) d[4 * i + e] = tr.vr[i][e];
      d[24] = tr.vr6[0];
      d[25] = tr.vr6[1];
      d[26] = 0u;
#pragma unroll
      for (int j = 0; j < 2; j++) {
        stu[kStVn + j * kKeyPitch + lane] = d[13 * j];
#pragma unroll
        for (int g = 0; g < 16; g++) {
          // code group g of block j: bytes 3g..3g+2 of the codes (dword 13j+1 on)
          const int w = 13 * j + 1 + ((3 * g) >> 2), sh = (3 * g) & 3;
          stu[kStCodes + (16 * j + g) * kKeyPitch + lane] =
              sh ? __builtin_amdgcn_alignbyte(d[w + 1], d[w], sh) : d[w];
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // dense is wave-uniform: the common full tile (every key visible to every
    // query of the group) skips the per-key rule
    const bool dense = ts + kTile <= hi_first && rule.all_visible(ts + kTile);
    float s[4][4];
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const f4_t k0 = *reinterpret_cast<const f4_t*>(st + kStKn + 16 * g + 4 * row);
      const f4_t k1 = *reinterpret_cast<const f4_t*>(st + kStKn + kKeyPitch + 16 * g + 4 * row);
#pragma unroll
      for (int r = 0; r < 4; r++) {
        s[g][r] = k0[r] * sa[g][0][r] + k1[r] * sa[g][1][r];
        if constexpr (!CHAIN)
          s[g][r] += dpp_f<0x128>(s[g][r]);   // + the lo half of the query (column + 8, row_ror:8)
      }
    }
    if (!dense) {
#pragma unroll
      for (int g = 0; g < 4; g++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int key = ts + 16 * g + 4 * row + r;
          const bool vis = (key < hi_col) & rule.visible(key, active_end);   // padded keys too
          s[g][r] = vis ? s[g][r] : -INFINITY;
        }
    }

    // ---------------- online softmax of head `col` (its 64 keys sit in 4 rows) ----------------
    float mt = s[0][0];
#pragma unroll
    for (int g = 0; g < 4; g++)
#pragma unroll
      for (int r = 0; r < 4; r++) mt = fmaxf(mt, s[g][r]);
    mt = xrow_max(mt);
    const float mn = fmaxf(m2, mt);
    const float msafe = (mn == -INFINITY) ? 0.0f : mn;   // all keys so far masked: p = 0
    const float corr = __builtin_amdgcn_exp2f(m2 - msafe);
    float ps = 0.0f;
#pragma unroll
    for (int g = 0; g < 4; g++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        s[g][r] = __builtin_amdgcn_exp2f(s[g][r] - msafe);
        ps += s[g][r];
      }
    lsum = lsum * corr + ps;
    m2 = mn;
    if constexpr (!first) {   // accumulators are still zero on the first tile
      // accumulator rows are heads 4*row + r: their factors come from lanes 4*row + r
      if (row == 0) st[kStCorr + col] = corr;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const f4_t cr = *reinterpret_cast<const f4_t*>(st + kStCorr + 4 * row);
#pragma unroll
      for (int t = 0; t < 16; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) acc[t][r] *= cr[r];
    }

    if constexpr (first) QKV_STAMP(kPhSoftmax);
    // ---------------- values ----------------
    // 32-key chunk c2: MFMA k index i <-> key 32*c2 + 4*row + i (i < 4) and
    // 32*c2 + 16 + 4*row + (i - 4) (i >= 4), in both operands.  A = p * value
    // norm (head `col`, this lane's own probabilities), B = codes of 8 keys
    // in dim group `col`.
    {
      ValuePass vp[2];
      uint32_t cp[8], cq[8];
      value_pass_load(st, stu, 0, row, col, s, vp[0]);
      value_pairs<0>(lds, ac, vp[0].x, cp);
      value_pairs<1>(lds, ac, vp[0].x, cq);
      value_steps<0, first>(lds, ac, vp, cp, cq, acc, st, stu, row, col, s);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  // lo and hi are wave-uniform (a paged workgroup serves one query): the tile
  // loop is a scalar loop
  if constexpr (MODE == 2) {
    if (wave < n_sel) {
      tile_body(std::true_type{}, ts0);
      for (int k = wave + kWaves; k < n_sel; k += kWaves) {
        const int ts = __builtin_amdgcn_readlane(sel, k) * kTile;
        load_tile(p, ts, p.num_kv, h, lane, row, col, tr);
        tile_body(std::false_type{}, ts);
      }
    } else {
#pragma unroll
      for (int t = 0; t < 16; t++) acc[t] = f4_t{0.f, 0.f, 0.f, 0.f};
    }
  } else if (ts0 < hi) {
    if (APPEND && fa_wave == wave && ts0 <= p.start_pos && p.start_pos < ts0 + kTile)
      patch_new_key(tr, reinterpret_cast<const uint32_t*>(lds + kLdsNewRow), p.start_pos - ts0, lane, row, col);
    tile_body(std::true_type{}, ts0);
    for (int ts = ts0 + kStep; ts < hi; ts += kStep) {
      load_tile(p, wave_tile_row(ts), p.num_kv, h, lane, row, col, tr);
      if (APPEND && fa_wave == wave && ts <= p.start_pos && p.start_pos < ts + kTile)
        patch_new_key(tr, reinterpret_cast<const uint32_t*>(lds + kLdsNewRow), p.start_pos - ts, lane, row, col);
      tile_body(std::false_type{}, ts);
    }
  } else {
#pragma unroll
    for (int t = 0; t < 16; t++) acc[t] = f4_t{0.f, 0.f, 0.f, 0.f};
  }
  lsum = xrow_sum(lsum);
  QKV_STAMP(kPhTiles);

  // ---------------- merge the 4 waves in LDS ----------------
  __syncthreads();
  QKV_STAMP(kPhTileBar);
  float* mo = reinterpret_cast<float*>(lds + kLdsMergeO);    // [wave][8][256]
  float* ml = reinterpret_cast<float*>(lds + kLdsMergeML);
  // (row offset recomputed from the thread index rather than held through the loop)
  int row4 = ((int)threadIdx.x & 63) >> 4 << 2;
  asm volatile("" : "+v"(row4));
  if (row4 < rows_used) {   // accumulator rows 4*row + r; rows >= rows_used are unused
    // acc tile t: rows 4*row+r, dim 128*(t>>3) + 8*col + (t&7): 16-byte stores
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
      for (int q4 = 0; q4 < 4; q4++) {
        const int t = 4 * q4;   // tiles t..t+3: dims 128*(q4>>1) + 8*col + 4*(q4&1) + 0..3
        *reinterpret_cast<f4_t*>(mo + (wave * 16 + row4 + r) * kHD + 128 * (q4 >> 1) + 8 * col +
                                 4 * (q4 & 1)) = f4_t{acc[t][r], acc[t + 1][r], acc[t + 2][r], acc[t + 3][r]};
      }
  }
  if (row == 0) {
    ml[kMlW0 + wave * 16 + col] = m2;
    ml[kMlLw0 + wave * 16 + col] = lsum;
  }
  __syncthreads();
  QKV_STAMP(kPhMergeBar);
  const int rows = rows_used;
  // fast path: every merged piece goes straight to its record
  const __amdgpu_buffer_rsrc_t rml =
      __builtin_amdgcn_make_buffer_rsrc(p.ws_ml, 0, MODE == 0 ? p.ws_ml_bytes : 0u, kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t ro =
      __builtin_amdgcn_make_buffer_rsrc(p.ws_o, 0, MODE == 0 ? p.ws_o_bytes : 0u, kBufferRsrcWord3);
  // (an opaque copy of gqa: its division reciprocal is formed here, not held
  // in a register through the tile loop)
  int gqa_m = gqa;
  asm volatile("" : "+s"(gqa_m));
  for (int idx = threadIdx.x; idx < rows * 64; idx += kThreads) {
    const int r = idx >> 6, d4 = (idx & 63) * 4;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; w++) M = fmaxf(M, ml[kMlW0 + w * 16 + r]);
    float L = 0.f;
    f4_t o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < kWaves; w++) {
      const float mw = ml[kMlW0 + w * 16 + r];
      const float wt = (mw == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
      L += wt * ml[kMlLw0 + w * 16 + r];
      o += wt * *reinterpret_cast<const f4_t*>(mo + (w * 16 + r) * kHD + d4);
    }
    if constexpr (MODE >= 1) {
      *reinterpret_cast<f4_t*>(mo + r * kHD + d4) = o;   // wave-0 slot, own elements only
      if (d4 == 0) {
        ml[kMlM + r] = M;
        ml[kMlL + r] = L;
      }
    } else if (has_work) {
      store_record_piece(p, rml, ro, h * gqa_m + r % gqa_m, rec_t0 + r / gqa_m, rec_chunk, d4, o, M, L);
    }
  }

  if constexpr (MODE >= 1) {
    __syncthreads();
    finish_rows(lds, p, h, t0, rows, false, chunk, nullptr);
    return;
  }

  // ---------------- fast path: tagged records, designated mergers ----------------
  QKV_STAMP(kPhMerged);
  if (has_work) publish_records(p, rml, h, gqa_m, rec_t0, rows, rec_chunk);
  QKV_STAMP(kPhPublished);
#ifdef QKV_PHASE_TRACE
  if (threadIdx.x < 3) *reinterpret_cast<uint64_t*>(lds + kLdsMergeO + kTracePolledByte + 8 * threadIdx.x) = 0;
#endif
  using ML = MergeLayout<kThreads>;
  static_assert(kLdsMergeO + ML::kRedFloats * 4 <= kLdsMergeML, "merge reduction must fit");
  merge_phase<kThreads, true>(reinterpret_cast<float*>(lds + kLdsMergeO),
                              reinterpret_cast<f2_t*>(lds + kLdsMergeML), p, rml, ro, out);
#ifdef QKV_PHASE_TRACE
  __syncthreads();
  trace_st[kPhPolled] = *reinterpret_cast<const uint64_t*>(lds + kLdsMergeO + kTracePolledByte);
  trace_st[kPhRowsIn] = *reinterpret_cast<const uint64_t*>(lds + kLdsMergeO + kTracePolledByte + 8);
  trace_st[kPhFolded] = *reinterpret_cast<const uint64_t*>(lds + kLdsMergeO + kTracePolledByte + 16);
  QKV_STAMP(kPhEnd);
  if (lane < 15 && blockIdx.x < kTraceMaxWgs) {
    uint64_t v = 0;
#pragma unroll
    for (int i = 0; i < 15; i++) v = lane == i ? trace_st[i] : v;
    qkv_phase_stamps[(blockIdx.x * kWaves + wave) * 16 + lane] = v;
  }
  if (lane == 0 && blockIdx.x < kTraceMaxWgs)
    qkv_phase_stamps[(blockIdx.x * kWaves + wave) * 16 + kPhXcd] =
        __builtin_amdgcn_s_getreg((3 << 11) | 20) & 15u;   // HW_REG_XCC_ID bits 3:0
#endif
}

// ---- shared-decode multi-query fast path ----------------------------------
// Calls with more than 16 (query, head) columns (a verify block, a tree
// verify): tq3_attn_kernel<0, true> decodes every tile once per 16 columns,
// and that decode (table-index shifts, code interleaves, table reads) is what
// bounds it.  Here every 64-key tile is decoded ONCE per workgroup, by all 8
// waves, into LDS as fp16 scaled centroids -- keys as rows [key][dim], values
// as rows [dim][key] in the value MFMA's key order -- and four groups of two
// waves run the MFMAs of up to 64 columns from there: wave w serves columns
// 16 (w & 3) .. +15 over keys 32 (w >> 2) .. +31 of the tile.
//   scores  v_mfma_f32_16x16x32_f16, A = 16 decoded keys x 32 dims (one
//           16-byte LDS read per lane), B = the rotated query of the wave's
//           16 columns as an fp16 rounding and its fp16 remainder (64 VGPRs),
//           two products chained onto one accumulator per 128-block, each
//           scaled by its key block norm.
//   softmax online, per column, base 2 (the wave's 32 keys sit in 4 rows).
//   values  v_mfma_f32_16x16x32_f16, A = p * value norm (the lane's own
//           probabilities), B = 32 keys x 16 dims of decoded values.
// The two waves of a column group merge in LDS and the merged rows become
// records, merged across workgroups as in tq3_attn_kernel (attn_fastmerge.h).
namespace mq {
// Decoded tiles, XOR-swizzled in 16-byte chunks so that the MFMA operand reads
// (16 lanes per LDS cycle: 16 rows at one logical chunk) and the decode's
// stores hit 16 different bank groups (padded rows do not on this LDS):
// key r's chunk c at c ^ (r & 15), dim d's chunk c at c ^ (d & 7).
constexpr int kKRow = 512;      // decoded key row: 256 fp16
constexpr int kVRow = 128;      // decoded value row (one dim): 64 fp16
constexpr int kLdsK = kLdsLut + kLdsLutBytes;          // [64 keys][kKRow]
constexpr int kLdsV = kLdsK + 64 * kKRow;              // [256 dims][kVRow]
constexpr int kLdsNorm = kLdsV + 256 * kVRow;          // kn[2][64] (x softmax scale), vn[2][64] f32
constexpr int kLdsCorr = kLdsNorm + 4 * 64 * 4;        // per wave: 16 rescale factors
// the tile as loaded: key rows at 112 r, value rows at 112 r + 16 ((r >> 2) & 15)
// (value rows 4 apart start in different bank groups: the value decode reads
// rows 4kq + i for 16 kq at once)
constexpr int kRawPitch = 112;
constexpr int kLdsRawK = kLdsCorr + kWaves * 16 * 4;
constexpr int kLdsRawV = kLdsRawK + 64 * kRawPitch;
constexpr int kLdsEnd = kLdsRawV + 64 * kRawPitch + 16 * 16;
// fused append: the encoded 13-dword blocks of this workgroup's new keys
// (at most 64 keys x K, V x 2 blocks)
constexpr int kLdsEnc = kLdsEnd;
constexpr int kLdsEncEnd = kLdsEnc + 64 * 4 * 13 * 4;
// setup: the rotated query's fp16 rounding and remainder, [64 columns][kKRow]
// each (swizzled as the keys), over the decoded tile areas (read into
// registers before tile 0)
constexpr int kLdsQhi = kLdsK;
constexpr int kLdsQlo = kLdsK + 64 * kKRow;
// after the tile loop: [8 waves][16 rows][kMoPitch floats], then m, l [8][16]
constexpr int kMoPitch = 260;
constexpr int kLdsMo = 0;
constexpr int kLdsMl = kWaves * 16 * kMoPitch * 4;
static_assert(kLdsQlo + 64 * kKRow <= kLdsNorm, "query scratch must fit the decoded tile areas");
static_assert(kLdsMl + 2 * kWaves * 16 * 4 <= kLdsEnd && kLdsMl + 256 * 8 <= kLdsEnd, "merge area must fit");
static_assert(kLdsMl >= kWaves * 128 * 4, "merger reduction area must not reach the merger scalars");
static_assert(kLdsEncEnd <= 160 * 1024, "LDS");
__device__ __forceinline__ int raw_v_row(int r) { return kLdsRawV + r * kRawPitch + 16 * ((r >> 2) & 15); }
}  // namespace mq

// One tile's rows as loaded: thread (row r = tid / 8, piece pc = tid % 8)
// holds bytes 16 pc .. 16 pc + 15 of key row r and of value row r (piece 6:
// bytes 96..103 used; piece 7 repeats piece 6 and is not stored).  Two wide
// loads per thread and tile.
struct MqRaw {
  u4_t k, v;
};

__device__ __forceinline__ void mq_load(const AttnArgs& p, int ts, int nkv, int h, int tid, MqRaw& r) {
  const uint64_t off0 = (uint64_t)(uint32_t)ts * (uint32_t)nkv * 104u;
  const __amdgpu_buffer_rsrc_t rk = cache_rsrc(p.k, off0, p.kv_bytes);
  const __amdgpu_buffer_rsrc_t rv = cache_rsrc(p.v, off0, p.kv_bytes);
  const int row = tid >> 3, pc = min(tid & 7, 6);
  const uint32_t off = (uint32_t)(row * nkv + h) * 104u + 16u * (uint32_t)pc;
  r.k = __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0);
  r.v = __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0);
}

__device__ __forceinline__ void mq_store_raw(uint8_t* lds, const MqRaw& r, int tid) {
  const int row = tid >> 3, pc = tid & 7;
  uint8_t* dk = lds + mq::kLdsRawK + row * mq::kRawPitch + 16 * pc;
  uint8_t* dv = lds + mq::raw_v_row(row) + 16 * pc;
  if (pc < 6) {
    *reinterpret_cast<u4_t*>(dk) = r.k;
    *reinterpret_cast<u4_t*>(dv) = r.v;
  } else if (pc == 6) {
    *reinterpret_cast<u2_t*>(dk) = u2_t{r.k[0], r.k[1]};
    *reinterpret_cast<u2_t*>(dv) = u2_t{r.v[0], r.v[1]};
  }
}

// Decode the staged tile into the LDS tile areas (every thread of the
// workgroup; the caller orders it against the MFMA phase with barriers).
// Key role: lane = key, wave = (block j = wave & 1, octet o = wave >> 1): code
// groups 4o..4o+3 of block j.  Value role: keys 4kq..4kq+3 (kq = lane & 15),
// code group g = 4 (wave >> 1) + (lane >> 4) of block j.
__device__ __forceinline__ void mq_decode(uint8_t* lds, uint32_t lane4, int lane, int j, int o, int kq,
                                          int g, float scale2) {
  uint32_t ac[4] = {lane4, lane4, lane4, lane4};
  // keys: row `lane`, dims 128j + 32o + 8U + 0..7 from code group 4o + U
  {
    const uint32_t* rk = reinterpret_cast<const uint32_t*>(lds + mq::kLdsRawK + lane * mq::kRawPitch + 52 * j);
    const uint32_t q[3] = {rk[1 + 3 * o], rk[2 + 3 * o], rk[3 + 3 * o]};
    const int kd = mq::kLdsK + lane * mq::kKRow + 256 * j + 16 * ((4 * o) ^ (lane & 15));   // chunk 4o + U at (4o + U) ^ (lane & 15)
    const h8_t k0 = group_operand<0>(lds, ac, q);
    const h8_t k1 = group_operand<1>(lds, ac, q);
    const h8_t k2 = group_operand<2>(lds, ac, q);
    const h8_t k3 = group_operand<3>(lds, ac, q);
    *reinterpret_cast<h8_t*>(lds + (kd ^ 0)) = k0;
    *reinterpret_cast<h8_t*>(lds + (kd ^ 16)) = k1;
    *reinterpret_cast<h8_t*>(lds + (kd ^ 32)) = k2;
    *reinterpret_cast<h8_t*>(lds + (kd ^ 48)) = k3;
    if (o == 0) {   // waves 0 and 1: the block norms of key `lane`
      const float* rv = reinterpret_cast<const float*>(lds + mq::raw_v_row(lane) + 52 * j);
      float* nm = reinterpret_cast<float*>(lds + mq::kLdsNorm);
      nm[64 * j + lane] = __uint_as_float(rk[0]) * scale2;
      nm[128 + 64 * j + lane] = rv[0];
    }
  }
  // values: keys 4kq..4kq+3 in dims 128j + 8g + 0..7; the codes of key pairs
  // (4kq, 4kq+1) and (4kq+2, 4kq+3) interleaved per dim, so that each table
  // entry is two keys at one dim
  {
    const int gb = 52 * j + 4 * ((4 + 3 * g) >> 2);   // dword holding the group's first byte
    const uint32_t sh = (uint32_t)((4 + 3 * g) & 3);
    uint32_t x[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t* rv = reinterpret_cast<const uint32_t*>(lds + mq::raw_v_row(4 * kq + i) + gb);
      x[i] = __builtin_amdgcn_alignbyte(rv[1], rv[0], sh);
    }
    const uint32_t h0 = x[1] << 3, h1 = x[3] << 3;
    const uint32_t ze0 = bit_select(kEvenDims, x[0], h0), zo0 = bit_select(kEvenDims << 3, x[0], h0);
    const uint32_t ze1 = bit_select(kEvenDims, x[2], h1), zo1 = bit_select(kEvenDims << 3, x[2], h1);
    // row (dim) e: keys of half H = kq >> 3 at bytes 64H + 16kb (+8 for the
    // half's keys 16.. of unit kb), the order of the value MFMA's k index
    const int kq7 = kq & 7;
  // (dim 128j + 8g + e: chunk c at c ^ e)
  const int vd = mq::kLdsV + (128 * j + 8 * g) * mq::kVRow + 16 * (4 * (kq >> 3) + (kq7 & 3)) + 8 * (kq7 >> 2);
    uint32_t w[16];
    w[0] = lut_read(lds, ac[0] = sdwa_index<0>(ac[0], ze0));
    w[1] = lut_read(lds, ac[1] = sdwa_index<0>(ac[1], ze1));
    w[2] = lut_read(lds, ac[2] = sdwa_index<3>(ac[2], zo0));
    w[3] = lut_read(lds, ac[3] = sdwa_index<3>(ac[3], zo1));
    w[4] = lut_read(lds, ac[0] = sdwa_index<6>(ac[0], ze0));
    w[5] = lut_read(lds, ac[1] = sdwa_index<6>(ac[1], ze1));
    w[6] = lut_read(lds, ac[2] = sdwa_index<9>(ac[2], zo0));
    w[7] = lut_read(lds, ac[3] = sdwa_index<9>(ac[3], zo1));
    w[8] = lut_read(lds, ac[0] = sdwa_index<12>(ac[0], ze0));
    w[9] = lut_read(lds, ac[1] = sdwa_index<12>(ac[1], ze1));
    w[10] = lut_read(lds, ac[2] = sdwa_index<15>(ac[2], zo0));
    w[11] = lut_read(lds, ac[3] = sdwa_index<15>(ac[3], zo1));
    w[12] = lut_read(lds, ac[0] = sdwa_index<18>(ac[0], ze0));
    w[13] = lut_read(lds, ac[1] = sdwa_index<18>(ac[1], ze1));
    w[14] = lut_read(lds, ac[2] = sdwa_index<21>(ac[2], zo0));
    w[15] = lut_read(lds, ac[3] = sdwa_index<21>(ac[3], zo1));
#pragma unroll
    for (int e = 0; e < 8; e++)
      *reinterpret_cast<u2_t*>(lds + (vd ^ (16 * e)) + mq::kVRow * e) = u2_t{w[2 * e], w[2 * e + 1]};
  }
}

__global__ __launch_bounds__(kThreads, 1) void tq3_mq_kernel(QKV_ATTN_LEAD_PARAMS, AttnArgs pin,
                                                              uint16_t* out) {
  QKV_ATTN_LEAD_APPLY(p, pin);
  __shared__ __attribute__((aligned(16))) uint8_t lds[mq::kLdsEncEnd];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gqa = __builtin_amdgcn_readfirstlane(p.num_q / p.num_kv);
  // work id, XCD-aware as in tq3_attn_kernel: the num_kv workgroups of one
  // (query block, chunk) share an XCD
  int h, t0, chunk;
  bool has_work;
  {
    const int L = blockIdx.x;
    const int xcd = L & 7, r = L >> 3;
    h = r % p.num_kv;
    const int g = (r / p.num_kv) * 8 + xcd;
    const int groups = (p.sub_n + p.qpw - 1) / p.qpw;
    has_work = g < groups * p.n_chunks;
    const int tq = has_work ? g / p.n_chunks : 0;
    chunk = has_work ? g - tq * p.n_chunks : 0;
    t0 = tq * p.qpw;
  }
  const int nq = min(p.qpw, p.sub_n - t0);
  const int cols = __builtin_amdgcn_readfirstlane(nq * gqa);   // <= 64
  // ---- query loads first: 128 WHTs of 128 (64 columns x 2 blocks), 16 lanes
  // each, four per thread
  const int q_part = tid & 15;
  u4_t q_raw[4];
  {
    const uint32_t q_extent = (uint32_t)(p.sub_n * p.num_q * kHD * 2);
    const __amdgpu_buffer_rsrc_t rq =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p.q), 0, q_extent, kBufferRsrcWord3);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int wi = (tid >> 4) + 32 * i, c = wi >> 1, jb = wi & 1;
      const uint32_t qoff = c < cols ? (uint32_t)((((t0 + c / gqa) * p.num_q + h * gqa + c % gqa) * kHD +
                                                   jb * 128 + q_part * 8) * 2)
                                     : q_extent;
      q_raw[i] = __builtin_amdgcn_raw_buffer_load_b128(rq, qoff, 0, 0);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // ---- key range of the workgroup and of this lane's column
  const int grp = wave & 3, half = wave >> 2;   // MFMA role: columns 16 grp.., keys 32 half.. of a tile
  const int n = lane & 15, kb = lane >> 4;
  const int col = 16 * grp + n;
  const int t_col = t0 + min(col / gqa, nq - 1);
  const int active_end = p.start_pos + t_col + 1;
  const int active_first = p.start_pos + t0 + 1;
  const int active_last = p.start_pos + t0 + nq;
  int lo = 0, hi = 0, hi_col = 0, hi_first = 0;
  if (has_work) {
    lo = chunk * p.chunk_keys;
    // the last chunk runs to the end of the keys (the host may have joined a
    // remainder of at most one tile to it)
    const int c_end = chunk == p.n_chunks - 1 ? active_last : lo + p.chunk_keys;
    hi = min(c_end, active_last);
    hi_col = min(c_end, active_end);
    hi_first = min(c_end, active_first);
  }
  lo = __builtin_amdgcn_readfirstlane(lo);
  hi = __builtin_amdgcn_readfirstlane(hi);
  hi_first = __builtin_amdgcn_readfirstlane(hi_first);
  // ---- fused append (qkv_decode_attn_tq3_append): the new keys start_pos ..
  // start_pos + sub_n - 1 that this workgroup reads, [new_lo, new_lo + n_new),
  // are encoded here (tq3_encode_row16, the small append's arithmetic), 32
  // blocks per round; the last query group's workgroups also store them to
  // the caches.  Their cache rows are read (stale) like every other row and
  // the encoded rows are written over them in the LDS staging before decode.
  int new_lo = 0, n_new = 0;
  if (p.k_new != nullptr && has_work && hi > max(lo, p.start_pos)) {
    new_lo = max(lo, p.start_pos);
    n_new = hi - new_lo;   // <= sub_n <= 64 (the host takes this path only then)
  }
  new_lo = __builtin_amdgcn_readfirstlane(new_lo);
  n_new = __builtin_amdgcn_readfirstlane(n_new);
  auto enc_input = [&](int round) {
    const int j = 32 * round + (tid >> 4), t = tid & 15;
    uint4 raw = make_uint4(0u, 0u, 0u, 0u);
    if (j < 4 * n_new) {
      const int tv = (j >> 1) & 1, blk = j & 1;
      const uint16_t* src = (tv ? p.v_new : p.k_new) +
                            ((long)(new_lo + (j >> 2) - p.start_pos) * p.num_kv + h) * kHD + blk * 128 + 8 * t;
      raw = *reinterpret_cast<const uint4*>(src);
    }
    return raw;
  };
  // the inputs of the first two rounds (16 new keys) are requested now
  uint4 enc_raw0 = make_uint4(0u, 0u, 0u, 0u), enc_raw1 = make_uint4(0u, 0u, 0u, 0u);
  if (n_new > 0) enc_raw0 = enc_input(0);
  if (n_new > 8) enc_raw1 = enc_input(1);
  // decode roles
  const int dj = wave & 1, dof = wave >> 1;              // keys: block, octet
  const int kq = lane & 15, vg = 4 * (wave >> 1) + (lane >> 4);   // values: key quad, code group
  // tiles of the chunk; rows loaded two tiles ahead of their decode
  const int n_tiles = hi > lo ? (hi - lo + kTile - 1) / kTile : 0;
  MqRaw ra, rb;
  if (n_tiles > 0) mq_load(p, lo, p.num_kv, h, tid, ra);
  if (n_tiles > 1) mq_load(p, lo + kTile, p.num_kv, h, tid, rb);
  // ---- setup: centroid-pair table (as tq3_attn_kernel), rotated query
  const uint32_t lane4 = 4u * (uint32_t)lane;
  {
    const uint32_t w = (uint32_t)wave;
#pragma unroll
    for (int hk = 0; hk < 4; hk++) {
      const uint32_t hv = centroid_scaled_h((4u * w + hk) & 7u) << 16;
#pragma unroll
      for (int k = 0; k < 8; k++)
        *reinterpret_cast<uint32_t*>(lds + kLdsLut + (w * 32 + hk * 8 + k) * 256 + lane4) =
            centroid_scaled_h(k) | hv;
    }
  }
  {
    const uint32_t sbits = sign_word_sel(q_part >> 2) >> (8 * (q_part & 3));   // elements part*8..+7
    const float rs = wht_scale();
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int wi = (tid >> 4) + 32 * i, c = wi >> 1, jb = wi & 1;
      float x[8];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        x[2 * e] = h2f(q_raw[i][e] & 0xffffu);
        x[2 * e + 1] = h2f(q_raw[i][e] >> 16);
      }
#pragma unroll
      for (int e = 0; e < 8; e++) x[e] = ((sbits >> e) & 1u) ? x[e] : -x[e];
      wht8_inreg(x);
      wht_xor_lanes16(x, lane);
      uint32_t pk[4], pl[4];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const float a = x[2 * e] * rs, b = x[2 * e + 1] * rs;
        const uint32_t ha = f2h(a), hb = f2h(b);
        pk[e] = ha | (hb << 16);
        pl[e] = f2h(a - h2f(ha)) | (f2h(b - h2f(hb)) << 16);
      }
      const int qb = c * mq::kKRow + 256 * jb + 16 * (q_part ^ (c & 15));
      *reinterpret_cast<uint4*>(lds + mq::kLdsQhi + qb) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
      *reinterpret_cast<uint4*>(lds + mq::kLdsQlo + qb) = make_uint4(pl[0], pl[1], pl[2], pl[3]);
    }
  }
  if (n_new > 0) {
    const bool put = t0 + nq == p.sub_n;   // the last query group stores the rows
    uint32_t* enc = reinterpret_cast<uint32_t*>(lds + mq::kLdsEnc);
    for (int round = 0; 32 * round < 4 * n_new; round++) {
      const uint4 raw = round == 0 ? enc_raw0 : round == 1 ? enc_raw1 : enc_input(round);
      const uint32_t word = tq3_encode_row16(raw, lane);
      const int j = 32 * round + (tid >> 4), t = tid & 15;
      if (j < 4 * n_new && t <= 12) {
        const int w = t == 12 ? 0 : 1 + t;
        enc[j * 13 + w] = word;
        if (put) {
          const int tv = (j >> 1) & 1, blk = j & 1;
          uint32_t* dst = reinterpret_cast<uint32_t*>(tv ? p.v_w : p.k_w) +
                          ((long)(new_lo + (j >> 2)) * p.num_kv + h) * 26 + blk * 13 + w;
          *dst = word;
        }
      }
    }
  }
  if (n_tiles > 0) {   // tile 0 staged; its registers take tile 2
    mq_store_raw(lds, ra, tid);
    if (n_tiles > 2) mq_load(p, lo + 2 * kTile, p.num_kv, h, tid, ra);
  }
  __syncthreads();
  // qa[s] / ql[s]: column `col`, dims 32s + 8kb .. +7 (B operand of slice s)
  h8_t qa[8], ql[8];
#pragma unroll
  for (int s = 0; s < 8; s++) {
    qa[s] = *reinterpret_cast<const h8_t*>(lds + ((mq::kLdsQhi + col * mq::kKRow + 16 * (kb ^ n)) ^ (64 * s)));
    ql[s] = *reinterpret_cast<const h8_t*>(lds + ((mq::kLdsQlo + col * mq::kKRow + 16 * (kb ^ n)) ^ (64 * s)));
  }
  const KeyRule rule(p.start_pos, t_col, p.sink_tok, p.window_tok, p.tree_mask);
  const bool live = 16 * grp < cols;   // wave-uniform: the group holds columns
  const float scale2 = p.scale_log2 * kCenScaleInv;
  float m2 = -INFINITY, lsum = 0.0f;
  f4_t acc[16];
#pragma unroll
  for (int t = 0; t < 16; t++) acc[t] = f4_t{0.f, 0.f, 0.f, 0.f};
  const float* nm = reinterpret_cast<const float*>(lds + mq::kLdsNorm);
  float* corr_w = reinterpret_cast<float*>(lds + mq::kLdsCorr) + 16 * wave;
  __syncthreads();   // the query scratch is read: the tile areas are free

  // Tile t: decode the staged rows; then stage tile t + 1 (its registers take
  // tile t + 3) while the MFMAs of tile t run.  The loop is unrolled by two so
  // that the two register sets stay fixed registers.
  auto tile_step = [&](int t, MqRaw& nxt) {
    const int ts = lo + t * kTile;
    if (n_new > 0) {
      // the encoded new keys of this tile over their staged (stale) rows
      const int a0 = max(ts, new_lo), a1 = min(ts + kTile, new_lo + n_new);
      if (a0 < a1) {
        const uint32_t* enc = reinterpret_cast<const uint32_t*>(lds + mq::kLdsEnc);
        for (int idx = tid; idx < (a1 - a0) * 52; idx += kThreads) {
          const int kk = idx / 52, rem = idx - kk * 52, tv = rem / 26, w = rem - tv * 26;
          const int key = a0 + kk, r = key - ts;
          const uint32_t val = enc[((key - new_lo) * 4 + tv * 2 + w / 13) * 13 + w % 13];
          *reinterpret_cast<uint32_t*>(lds + (tv ? mq::raw_v_row(r) : mq::kLdsRawK + r * mq::kRawPitch) +
                                       4 * w) = val;
        }
        __syncthreads();
      }
    }
    mq_decode(lds, lane4, lane, dj, dof, kq, vg, scale2);
    __syncthreads();
    if (t + 1 < n_tiles) {
      mq_store_raw(lds, nxt, tid);
      if (t + 3 < n_tiles) mq_load(p, ts + 3 * kTile, p.num_kv, h, tid, nxt);
    }
    if (live) {
      // ---- scores: D rows = keys 32 half + 16 mb + 4 kb + r, column `col`
      f4_t sa[2][2];
#pragma unroll
      for (int mb = 0; mb < 2; mb++) sa[mb][0] = sa[mb][1] = f4_t{0.f, 0.f, 0.f, 0.f};
      const int kbase = mq::kLdsK + (32 * half + n) * mq::kKRow + 16 * (kb ^ n);   // key 32 half + 16 mb + n, chunk (4s + kb) ^ n
      // operand reads two slices ahead of their MFMAs (three rotating buffers)
      h8_t ka[3][2];
#pragma unroll
      for (int s = 0; s < 2; s++)
#pragma unroll
        for (int mb = 0; mb < 2; mb++)
          ka[s][mb] = *reinterpret_cast<const h8_t*>(lds + (kbase ^ (64 * s)) + 16 * mb * mq::kKRow);
#pragma unroll
      for (int s = 0; s < 8; s++) {
        if (s + 2 < 8) {
#pragma unroll
          for (int mb = 0; mb < 2; mb++)
            ka[(s + 2) % 3][mb] = *reinterpret_cast<const h8_t*>(lds + (kbase ^ (64 * (s + 2))) + 16 * mb * mq::kKRow);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int mb = 0; mb < 2; mb++) {
          sa[mb][s >> 2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[s % 3][mb], qa[s], sa[mb][s >> 2], 0, 0, 0);
          sa[mb][s >> 2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[s % 3][mb], ql[s], sa[mb][s >> 2], 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      const bool dense = ts + kTile <= hi_first && rule.all_visible(ts + kTile);
      float sc[2][4];
#pragma unroll
      for (int mb = 0; mb < 2; mb++) {
        const int k0 = 32 * half + 16 * mb + 4 * kb;
        const f4_t n0 = *reinterpret_cast<const f4_t*>(nm + k0);
        const f4_t n1 = *reinterpret_cast<const f4_t*>(nm + 64 + k0);
#pragma unroll
        for (int r = 0; r < 4; r++) sc[mb][r] = n0[r] * sa[mb][0][r] + n1[r] * sa[mb][1][r];
      }
      if (!dense) {
#pragma unroll
        for (int mb = 0; mb < 2; mb++)
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const int key = ts + 32 * half + 16 * mb + 4 * kb + r;
            const bool vis = (key < hi_col) & rule.visible(key, active_end);
            sc[mb][r] = vis ? sc[mb][r] : -INFINITY;
          }
      }
      // ---- online softmax of column `col` (its 32 keys sit in the 4 rows)
      float mt = sc[0][0];
#pragma unroll
      for (int mb = 0; mb < 2; mb++)
#pragma unroll
        for (int r = 0; r < 4; r++) mt = fmaxf(mt, sc[mb][r]);
      mt = xrow_max(mt);
      const float mn = fmaxf(m2, mt);
      const float msafe = (mn == -INFINITY) ? 0.0f : mn;
      const float corr = __builtin_amdgcn_exp2f(m2 - msafe);
      float ps = 0.0f;
#pragma unroll
      for (int mb = 0; mb < 2; mb++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          sc[mb][r] = __builtin_amdgcn_exp2f(sc[mb][r] - msafe);
          ps += sc[mb][r];
        }
      lsum = lsum * corr + ps;
      m2 = mn;
      // accumulator rows are columns 16 grp + 4 kb + r: their factors come
      // from the lanes of those columns
      if (__builtin_amdgcn_ballot_w64(corr != 1.0f) != 0) {
      if (kb == 0) corr_w[n] = corr;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const f4_t cr = *reinterpret_cast<const f4_t*>(corr_w + 4 * kb);
#pragma unroll
      for (int t = 0; t < 16; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) acc[t][r] *= cr[r];
      }
      // ---- values: A = p * value norm per 128-block, B = 32 keys x 16 dims
      h8_t pa[2];
#pragma unroll
      for (int mb = 0; mb < 2; mb++) {
        const int k0 = 32 * half + 16 * mb + 4 * kb;
        const f4_t v0 = *reinterpret_cast<const f4_t*>(nm + 128 + k0);
        const f4_t v1 = *reinterpret_cast<const f4_t*>(nm + 192 + k0);
#pragma unroll
        for (int r = 0; r < 4; r++) {
          pa[0][4 * mb + r] = (_Float16)(sc[mb][r] * v0[r]);
          pa[1][4 * mb + r] = (_Float16)(sc[mb][r] * v1[r]);
        }
      }
      const uint8_t* vbase = lds + mq::kLdsV + n * mq::kVRow + 16 * ((4 * half + kb) ^ (n & 7));   // dim 16t + n
      // operand reads four MFMAs ahead (five rotating buffers)
      h8_t vb[5];
#pragma unroll
      for (int t = 0; t < 4; t++) vb[t] = *reinterpret_cast<const h8_t*>(vbase + 16 * t * mq::kVRow);
#pragma unroll
      for (int t = 0; t < 16; t++) {
        if (t + 4 < 16) vb[(t + 4) % 5] = *reinterpret_cast<const h8_t*>(vbase + 16 * (t + 4) * mq::kVRow);
        __builtin_amdgcn_sched_barrier(0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[t >> 3], vb[t % 5], acc[t], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    __syncthreads();   // the tile areas are read and tile t + 1 is staged
  };
  for (int t = 0; t < n_tiles; t += 2) {
    tile_step(t, rb);
    if (t + 1 < n_tiles) tile_step(t + 1, ra);
  }
  lsum = xrow_sum(lsum);

  // ---- merge the two waves of each column group in LDS ----------------
  float* mo = reinterpret_cast<float*>(lds + mq::kLdsMo);
  float* ml = reinterpret_cast<float*>(lds + mq::kLdsMl);
  if (live) {
    // acc tile t: rows (columns) 4 kb + r of the group, dims 16t + n
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
      for (int t = 0; t < 16; t++) mo[(wave * 16 + 4 * kb + r) * mq::kMoPitch + 16 * t + n] = acc[t][r];
    if (kb == 0) {
      ml[wave * 16 + n] = m2;
      ml[kWaves * 16 + wave * 16 + n] = lsum;
    }
  }
  __syncthreads();
  const __amdgpu_buffer_rsrc_t rml = __builtin_amdgcn_make_buffer_rsrc(p.ws_ml, 0, p.ws_ml_bytes, kBufferRsrcWord3);
  const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(p.ws_o, 0, p.ws_o_bytes, kBufferRsrcWord3);
  int gqa_m = gqa;
  asm volatile("" : "+s"(gqa_m));
  if (has_work) {
    for (int idx = tid; idx < cols * 64; idx += kThreads) {
      const int R = idx >> 6, d4 = (idx & 63) * 4;
      const int wa = R >> 4, wb = wa + 4, rr = R & 15;
      const float ma = ml[wa * 16 + rr], mb2 = ml[wb * 16 + rr];
      const float M = fmaxf(ma, mb2);
      const float fa = (ma == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(ma - M);
      const float fb = (mb2 == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mb2 - M);
      const float Lr = fa * ml[kWaves * 16 + wa * 16 + rr] + fb * ml[kWaves * 16 + wb * 16 + rr];
      const f4_t oa = *reinterpret_cast<const f4_t*>(mo + (wa * 16 + rr) * mq::kMoPitch + d4);
      const f4_t ob = *reinterpret_cast<const f4_t*>(mo + (wb * 16 + rr) * mq::kMoPitch + d4);
      store_record_piece(p, rml, ro, h * gqa_m + R % gqa_m, t0 + R / gqa_m, chunk, d4, fa * oa + fb * ob, M, Lr);
    }
    publish_records(p, rml, h, gqa_m, t0, cols, chunk);
  } else {
    __syncthreads();   // (the barrier publish_records passes, so that mo is free for the mergers)
  }
  // (a multi-query call has at least two units per merger: 512 for the
  // 16-token verify at 16 q heads over 256 workgroups)
  merge_phase_paired<kThreads, true>(reinterpret_cast<float*>(lds + mq::kLdsMo),
                                     reinterpret_cast<f2_t*>(lds + mq::kLdsMl), p, rml, ro, out);
}

size_t tq3_attn_lds_bytes() { return kLdsTotal; }

#ifdef QKV_PHASE_TRACE
}  // namespace qkv
// Diagnostic build only: copies the phase stamps of the last fast-path
// launch (n <= kTraceMaxWgs * 8 * 16 values) to host memory.
extern "C" int qkv_debug_phase_stamps(uint64_t* host, size_t n) {
  if (host == nullptr || n > sizeof(qkv::qkv_phase_stamps) / 8) return -1;
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(qkv::qkv_phase_stamps), n * 8, 0, hipMemcpyDeviceToHost) ==
                 hipSuccess ? 0 : -6;
}
extern "C" int qkv_debug_phase_clear() {
  void* p = nullptr;
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(qkv::qkv_phase_stamps)) != hipSuccess) return -6;
  return qkv::launch_fill_zero(p, sizeof(qkv::qkv_phase_stamps), nullptr) == hipSuccess ? 0 : -6;
}
namespace qkv {
#endif

// ---- the allocation-free decode's scratch ----------------------------------
// One fixed-size array per GPU, holding the fast path's workspace layout
// (header, record scalars, record rows).  In host code `scratch` names a
// host-side stand-in, not a device address: kernels only ever receive the
// address hipGetSymbolAddress returns for the current device, kept per device.
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[64];
}  // namespace

hipError_t noalloc_scratch(int device, bool clear, hipStream_t stream, void** ptr) {
  if (device < 0 || device >= 64) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  bool fresh = false;
  if (g_scratch_ptr[device] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (p == nullptr) return hipErrorInvalidSymbol;
    g_scratch_ptr[device] = p;
    fresh = true;
  }
  *ptr = g_scratch_ptr[device];
  if (clear || fresh) return launch_fill_zero(*ptr, kNoAllocScratchBytes, stream);
  return hipSuccess;
}

hipError_t launch_tq3_attn(const AttnArgs& a, int mode, uint16_t* out, hipStream_t stream) {
  const int groups = (a.sub_n + a.qpw - 1) / a.qpw * a.n_chunks;
  const int n_wg = ((groups + 7) / 8) * 8 * a.num_kv;
  dim3 grid(n_wg), block(kThreads);
  if (mode == 0 && a.qpw * (a.num_q / a.num_kv) > 16)
    hipLaunchKernelGGL(tq3_mq_kernel, grid, block, 0, stream, QKV_ATTN_LEAD_ARGS(a), a, out);
  else if (mode == 0 && a.qpw * (a.num_q / a.num_kv) > 8)
    hipLaunchKernelGGL((tq3_attn_kernel<0, true>), grid, block, 0, stream, QKV_ATTN_LEAD_ARGS(a), a, out);
  else if (mode == 0 && a.k_new != nullptr)
    hipLaunchKernelGGL((tq3_attn_kernel<0, false, true>), grid, block, 0, stream, QKV_ATTN_LEAD_ARGS(a), a, out);
  else if (mode == 0)
    hipLaunchKernelGGL((tq3_attn_kernel<0>), grid, block, 0, stream, QKV_ATTN_LEAD_ARGS(a), a, out);
  else if (mode == 1)
    hipLaunchKernelGGL((tq3_attn_kernel<1>), grid, block, 0, stream, QKV_ATTN_LEAD_ARGS(a), a, out);
  else
    hipLaunchKernelGGL((tq3_attn_kernel<2>), grid, block, 0, stream, QKV_ATTN_LEAD_ARGS(a), a, out);
  return hipGetLastError();
}

}  // namespace qkv
