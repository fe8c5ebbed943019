// qkv_launch.h -- host launchers of the gfx950 kernels (internal; the public
// surface is include/qkv.h).  Arguments are validated by qkv_api.cpp.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qkv {

// Row mapping of a paged append: input block i (token i / blocks_per_row,
// slot token / n_tok, position positions[slot] + token % n_tok) goes to
// pool row block_tables[slot * max_blocks + pos / block_tokens] *
// block_tokens + pos % block_tokens; rows outside [0, pool_rows) are skipped.
struct PagedRows {
  const int32_t* block_tables;
  const int32_t* positions;
  int max_blocks, block_tokens, blocks_per_row, n_tok;
  long pool_rows;
};

// sc0/sc1 non-null: in0/in1 are DFK2 int8 rows with one fp16 scale per
// 128-element block (re-quantizing append)
hipError_t launch_tq3_append(const void* in0, void* out0, const void* in1, void* out1,
                             int n_blocks, int n_tensors, hipStream_t stream,
                             const PagedRows* paged = nullptr, const uint16_t* sc0 = nullptr,
                             const uint16_t* sc1 = nullptr);
hipError_t launch_tq3_dequant(const void* in, void* out, int n_blocks, hipStream_t stream);
hipError_t launch_q8_append(const void* in0, void* out0, const void* in1, void* out1,
                            int n_blocks, int n_tensors, hipStream_t stream,
                            const uint16_t* sc0 = nullptr, const uint16_t* sc1 = nullptr);
// DFK2 int8 rows (group-128 fp16 scales) to fp16; n_elems a multiple of 128
hipError_t launch_dfk2_dequant(const void* q, const uint16_t* sc, void* out, long n_elems,
                               hipStream_t stream);
hipError_t launch_q8_dequant(const void* in, void* out, int n_blocks, hipStream_t stream);
// Zero-fill of `bytes` (a multiple of 4) bytes by a kernel (graph-capture safe).
hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t stream);
hipError_t launch_ws_status(const void* workspace, int* status, int ok_value, int timeout_value,
                            hipStream_t stream);

// Token-row moves inside one slot of one layer's cache (kv_move.hip): row
// slot_row0 + to[i] := row slot_row0 + from[i] for i = 0..n-1, K and V.
constexpr int kMoveMax = 64;
struct MoveArgs {
  uint8_t* k;
  uint8_t* v;
  uint32_t k_row_bytes, v_row_bytes;   // multiples of 4
  long slot_row0;
  int n;
  int from[kMoveMax], to[kMoveMax];
};
hipError_t launch_kv_move(const MoveArgs& a, bool ordered, hipStream_t stream);

// Paged slot snapshot (gather) / restore (scatter), kv_move.hip.  Tensor t
// (0: K, 1: V) has rows of row_bytes[t] (a multiple of 4).
struct PageCopyArgs {
  uint8_t* pool[2];
  uint8_t* flat[2];
  uint32_t row_bytes[2];
  const int32_t* table;      // the slot's block-table row
  int max_blocks, block_tokens, n_rows, n_tensors;
  long pool_rows;
  bool aligned16;            // every pointer 16-byte aligned
};
hipError_t launch_kv_page_copy(const PageCopyArgs& a, bool scatter, hipStream_t stream);

// Block-sparse TQ3 verify (sparse_tq3.hip): K-pool signatures and the top-k
// block index.  Pools are fp16 [num_kv][stride][256].
struct KpoolArgs {
  const uint32_t* k;         // slot-base TQ3 key cache
  uint16_t* k_pool;
  uint16_t* k_pool_max;
  int num_kv, total_kv, blk_lo, cur_blocks, stride, bsn;
};
hipError_t launch_tq3_kpool(const KpoolArgs& a, hipStream_t stream);
struct BlockIndexArgs {
  const uint16_t* q;         // [sub_n][num_q][256]
  const uint16_t* k_pool;
  const uint16_t* k_pool_max;
  int32_t* block_index;      // [num_kv][sub_n_max][top_k]
  int num_q, num_kv, sub_n, sub_n_max, start_pos, top_k, bsn, n_blocks, stride;
  float beta;
  float inv_gqa;             // 1.0f / GQA (the reference's compile-time constant)
};
// scores: workspace of block_index_workspace_bytes (block scores [num_kv][sub_n][n_blocks])
hipError_t launch_block_index(const BlockIndexArgs& a, float* scores, hipStream_t stream);

// Chunked prefill over a TQ3 cache (prefill_tq3.hip).  Workspace pieces:
// kx  keys [num_kv][h_pad + n_pad][256] fp16: the history rows dequantized
//     exactly as the reference's bulk dequantization, padded to whole 64-row
//     tiles, then the chunk's own keys
// vt  values in 32-key tiles [num_kv][(h_pad + n_pad)/32][256 dims][32] fp16
// part_ml / part_o  key-split partials {m (log2 units), l} and o
//                   [n_split][n_tok][num_q] (x 256 for o)
struct PrefillArgs {
  const uint32_t* k_cache;   // slot-base TQ3 caches, rows 0 .. hist-1
  const uint32_t* v_cache;
  uint16_t* kx;
  uint16_t* vt;
  float* part_ml;
  float* part_o;
  int num_q, num_kv, start_pos, n_tok;
  int hist;                  // cache rows attended: start_pos, or start_pos + n_tok (verify)
  int h_pad;                 // hist rounded up to 64
  int n_pad;                 // chunk rows staged: n_tok rounded up to 64, 0 in verify mode
  int n_split;
  int from_cache;            // 1: the chunk's keys are cache rows too (verify)
  float scale_log2;
};
struct PrefillGeom {
  int n_pad, h_pad, n_split;
  size_t kx_off, vt_off, ml_off, o_off, total;
};
PrefillGeom prefill_geom(int num_q, int num_kv, int n_tok, int start_pos);
hipError_t launch_prefill_tq3(const PrefillArgs& a, int gqa, const uint16_t* q, const uint16_t* k,
                              const uint16_t* v, uint16_t* out, hipStream_t stream);

}  // namespace qkv
