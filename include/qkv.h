/*
 * qkv.h -- C ABI of the MI355X (gfx950) compressed KV-cache library libqkv.so.
 *
 * Drop-in for the reference's compressed-KV launches (Haru-neo/qengine,
 * paths relative to its tree).  The reference launches CUDA kernels directly
 * from QwenModel (src/model.cuh); every entry point below replaces one such
 * launch and keeps its argument list, buffer layouts and stream ordering.
 *
 * Conventions
 *  - fp16 tensors are passed as uint16_t bit patterns.
 *  - The caller owns every buffer; no entry point allocates or frees device
 *    memory.  Caches must be zero-initialised by the caller, as the reference
 *    does (model.cuh:1914-1920).
 *  - Every call is asynchronous on `stream` and never synchronises the host.
 *  - Return value: QKV_OK (0) or a negative qkv_status.  Invalid arguments are
 *    reported, never silently dropped (the reference returns void).
 */
#ifndef QKV_H
#define QKV_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* turboquant.cuh:73-77  struct block_tq3 { float norm; uint8_t qs[48]; }  (52 B, align 4)
 * 128 coordinates: L2 norm of the raw fp16 vector, then 3-bit Lloyd-Max codes of
 * the rotated unit vector, element e at bits 3e..3e+2 of the little-endian stream. */
typedef struct qkv_block_tq3 {
  float norm;
  uint8_t qs[48];
} qkv_block_tq3;

/* quant_gemv.cuh:19  block_q8_0_aligned { int8_t qs[32]; uint16_t pad; half d; }  (36 B) */
typedef struct qkv_block_q8 {
  int8_t qs[32];
  uint16_t pad;
  uint16_t d;
} qkv_block_q8;

typedef enum qkv_status {
  QKV_OK = 0,
  QKV_ERR_INVALID = -1,     /* bad size / shape / count                               */
  QKV_ERR_NULL = -2,        /* required pointer is NULL                               */
  QKV_ERR_UNSUPPORTED = -3, /* head_dim / GQA combination not compiled                */
  QKV_ERR_ALIGN = -4,       /* pointer not aligned as documented                       */
  QKV_ERR_DEVICE = -5,      /* no usable gfx950 device / HIP runtime error             */
  QKV_ERR_LAUNCH = -6,      /* kernel launch failed                                    */
  QKV_ERR_WORKSPACE = -7,   /* workspace missing or smaller than the query says         */
  QKV_ERR_TIMEOUT = -8      /* an in-kernel merge timed out; reset the workspace        */
} qkv_status;

/* Library version (major*10000 + minor*100 + patch). */
int qkv_version(void);

/* Static text for a status code. */
const char* qkv_status_string(int status);

/* ---------------------------------------------------------------------------
 * TQ3 codec
 * ------------------------------------------------------------------------- */

/* Replaces tq3_init_signs(gpu) (turboquant.cuh:288-302).  The sign vector is a
 * compile-time constant of this library (same seed and generator), so this call
 * validates `device` as a gfx950 GPU and prepares (zero-fills, synchronously)
 * the scratch of qkv_decode_attn_tq3_noalloc on it.  Optional before the
 * other calls; must not run while a qkv_decode_attn_tq3_noalloc call is in
 * flight on that device. */
int qkv_tq3_init(int device);

/* Replaces tq3_quantize_kernel<<<(n+31)/32, 32, 0, stream>>>(in, out, n_blocks)
 * (turboquant.cuh:112-165; launched at model.cuh:2329-2333, 5186-5190).
 * in:  n_blocks*128 fp16, contiguous (16-byte aligned).
 * out: n_blocks contiguous blocks (caller computes cache + (slot_off+pos)*bpt).
 * Codes and norms are bit-identical to the reference encoder. */
int qkv_tq3_append(const uint16_t* in_f16, qkv_block_tq3* out, int n_blocks,
                   hipStream_t stream);

/* K and V appends of one step in a single launch: equivalent to two
 * qkv_tq3_append calls (model.cuh:2329-2333 issues them back to back). */
int qkv_tq3_append_kv(const uint16_t* k_f16, const uint16_t* v_f16, qkv_block_tq3* k_out,
                      qkv_block_tq3* v_out, int n_blocks, hipStream_t stream);

/* Replaces tq3_dequantize_kernel (turboquant.cuh:169-200): fp16 output
 * half(((H*c)*rs)*sign*norm), bit-identical to the reference. */
int qkv_tq3_dequant(const qkv_block_tq3* in, uint16_t* out_f16, int n_blocks,
                    hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Q8_0 KV codec
 * ------------------------------------------------------------------------- */

/* Replaces quantize_kv_q8_0_kern<<<n_blocks, 32, 0, stream>>>(in, out, n_blocks)
 * (attention.cuh:2587-2609; launched at model.cuh:2316-2317).  `pad` is not
 * written.  in: n_blocks*32 fp16 (16-byte aligned). */
int qkv_q8_append(const uint16_t* in_f16, qkv_block_q8* out, int n_blocks,
                  hipStream_t stream);

/* K and V in one launch: the two quantize_kv_q8_0_kern launches of
 * model.cuh:2316-2333 (same blocks as two qkv_q8_append calls). */
int qkv_q8_append_kv(const uint16_t* k_f16, const uint16_t* v_f16, qkv_block_q8* k_out,
                     qkv_block_q8* v_out, int n_blocks, hipStream_t stream);

/* Replaces dequantize_kv_q8_0_kern (attention.cuh:2614-2626). */
int qkv_q8_dequant(const qkv_block_q8* in, uint16_t* out_f16, int n_blocks,
                   hipStream_t stream);

/* ---------------------------------------------------------------------------
 * KV inject from a DFK2 plane (int8 rows, one fp16 scale per 128 elements)
 * ------------------------------------------------------------------------- */

/* Replaces dfki2_dequant_kernel<<<(n + 255) / 256, 256>>>(q, scales, out, n,
 * kv_dim) (model.cuh:149-159; launched at model.cuh:3189-3192):
 * out[i] = half(float(q[i]) * float(scales[i / 128])), the scales of a row of
 * kv_dim elements being scales[row * kv_dim / 128 ...].  kv_dim a multiple of
 * 128, n a multiple of 8; q 8-byte and out 16-byte aligned. */
int qkv_dfk2_dequant(const int8_t* q, const uint16_t* scales, uint16_t* out_f16, long long n,
                     int kv_dim, hipStream_t stream);

/* The inject's dequantize-then-quantize pair fused into one launch: the
 * dfki2_dequant_kernel into the fp16 scratch followed by
 * tq3_quantize_kernel<<<(blocks + 31) / 32, 32>>>(scratch, dst, blocks)
 * (model.cuh:3189-3192, 3218-3226; the value planes, and key planes that need
 * no RoPE).  Block i is quantized from q[128 i .. 128 i + 127] with scale
 * scales[i]; the codes and norms are bit-identical to that pair's.  q 16-byte
 * aligned. */
int qkv_tq3_append_dfk2(const int8_t* q, const uint16_t* scales, qkv_block_tq3* out,
                        int n_blocks, hipStream_t stream);

/* The same for a Q8_0 cache (model.cuh:3189-3192 then 3227-3233 /
 * 3209-3217): 32-element block i from q[32 i ..] with scale scales[i / 4];
 * n_blocks a multiple of 4; q 8-byte aligned. */
int qkv_q8_append_dfk2(const int8_t* q, const uint16_t* scales, qkv_block_q8* out, int n_blocks,
                       hipStream_t stream);

/* Slot snapshot and restore over a paged pool.  The reference saves a slot's
 * first N rows of K and V with one device-to-host copy each
 * (save_prefix_snapshot, model.cuh:3394-3417: N * blocks_per_token blocks from
 * kv_slot_offset(slot) * blocks_per_token) and restores them with the reverse
 * copy (restore_snapshot_into_slot, model.cuh:3314-3335).  A contiguous slot
 * keeps those plain copies.  In a paged pool (qkv_decode_attn_tq3_paged) the
 * slot's logical row r is pool row
 *   block_table[r / block_tokens] * block_tokens + r % block_tokens,
 * and these two calls move rows 0 .. n_rows-1 between the pool and a flat
 * device buffer [n_rows][row_bytes] (then copied to / from the host as in the
 * reference).  Any packed format: row_bytes = blocks_per_token * 52 (TQ3),
 * * 36 (Q8_0) or kv_dim * 2 (fp16), a multiple of 4.  block_table is the
 * slot's row of max_blocks int32 entries (device).  Rows whose table entry is
 * negative or lands outside [0, pool_rows) are gathered as zeros and skipped
 * by the scatter.  v_pool and v_flat may both be NULL (keys only).  Rows of a
 * block shared with other slots (a common prefix) are written by the scatter
 * like any other row. */
int qkv_kv_gather_rows(const void* k_pool, const void* v_pool, void* k_flat, void* v_flat,
                       size_t k_row_bytes, size_t v_row_bytes, long pool_rows,
                       const int32_t* block_table, int max_blocks, int block_tokens, int n_rows,
                       hipStream_t stream);
int qkv_kv_scatter_rows(void* k_pool, void* v_pool, const void* k_flat, const void* v_flat,
                        size_t k_row_bytes, size_t v_row_bytes, long pool_rows,
                        const int32_t* block_table, int max_blocks, int block_tokens, int n_rows,
                        hipStream_t stream);

/* Token-row moves inside one slot of one layer's cache: replaces the per-token
 * device copies of kv_move_token (model.cuh:7430-7471; its tree-verify
 * acceptance calls it once per accepted token and layer).  For i = 0..n-1 in
 * list order, row slot_row0 + to[i] := row slot_row0 + from[i] in both k and
 * v, where from_to = {from0, to0, from1, to1, ...} (host array, 0 <= from, to
 * < slot_rows) and a row is k_row_bytes / v_row_bytes (blocks_per_token x
 * sizeof(qkv_block_tq3) or sizeof(qkv_block_q8); multiples of 4).  Works for
 * either cache format.  n <= 64 per call; a move with from == to does
 * nothing.  One launch; moves that touch no row another move writes run in
 * parallel, otherwise in list order. */
int qkv_kv_move_tokens(void* k, void* v, size_t k_row_bytes, size_t v_row_bytes, long slot_row0,
                       long slot_rows, const int32_t* from_to, int n, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Split-K flash decode over the packed caches
 *
 * Shapes: head_dim must be 256; GQA = num_q/num_kv in 1..8.
 * q        [sub_n][num_q][256] fp16 (16-byte aligned); query t sits at absolute
 *          position start_pos + t and attends keys [0, start_pos + t].
 * k, v     slot-base caches, token-major [pos][num_kv][2] blocks.
 * part_m/l [num_q][sub_n_max][k_splits] f32, part_o [..][k_splits][256] f32.
 * sink_tok/window_tok: 0/0 = dense; otherwise the reference's 32-key tile
 *          rule keeps tiles overlapping [0, sink) or the last `window` keys.
 * tree_mask: NULL = chain; else bit j of tree_mask[t] lets query t see key
 *          start_pos + j (sub_n <= 32).
 * ------------------------------------------------------------------------- */

/* Replaces flash_attn_chunk_fused_split_tq3<256, GQA, 32, 256, K_SPLITS>
 * <<<(num_kv, sub_n, K_SPLITS), 256>>> (attention.cuh:1905-2177; launched at
 * model.cuh:2472-2491 and 4663-4687).  Split z covers keys
 * [z*tps*32, min((z+1)*tps*32, start_pos+t+1)), tps = ceil(ceil(active_end_max/32)/k_splits);
 * writes the unnormalised partials (m, l, o) in the reference layout
 * (o in the original, unrotated coordinates).  Outputs agree with the
 * reference within the 2e-3 relative tolerance (fp32 accumulation). */
int qkv_attn_split_tq3(const uint16_t* q, const qkv_block_tq3* k, const qkv_block_tq3* v,
                       float* part_m, float* part_l, float* part_o, int num_q, int num_kv,
                       int head_dim, int start_pos, int sub_n, int sub_n_max,
                       int active_end_max, float scale, int k_splits, int sink_tok,
                       int window_tok, const uint32_t* tree_mask, hipStream_t stream);

/* Replaces flash_attn_chunk_fused_split_q8<256, GQA, 32, 256, K_SPLITS>
 * <<<(num_kv, sub_n, K_SPLITS), 256>>> (attention.cuh:2633-2801; launched at
 * model.cuh:2438-2457).  Same split rule and partial layout as
 * qkv_attn_split_tq3; K/V elements decode to half(q*d) (no masks: the
 * reference's Q8 kernel has none).  k, v: slot-base Q8_0 caches
 * [pos][num_kv][8] blocks.  Merge with qkv_attn_split_merge. */
int qkv_attn_split_q8(const uint16_t* q, const qkv_block_q8* k, const qkv_block_q8* v,
                      float* part_m, float* part_l, float* part_o, int num_q, int num_kv,
                      int head_dim, int start_pos, int sub_n, int sub_n_max, int active_end_max,
                      float scale, int k_splits, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Block-sparse TQ3 verify (the DFLASH_VERIFY_BLOCKSPARSE path of
 * model.cuh:4589-4662): per layer, a pool of 64-token key-block signatures is
 * kept up to date, each verify query picks its top_k blocks, and the split
 * kernel attends only those blocks; the partials merge with
 * qkv_attn_split_merge.
 * ------------------------------------------------------------------------- */

/* Replaces tq3_kpool_ms_update_kern<256, 256><<<dim3(num_kv, cur_blocks -
 * blk_lo), 256, block_size_n * 512>>>(k_tq, k_pool, k_pool_max, num_kv,
 * total_kv, blk_lo, n_blocks_stride, block_size_n) (attention.cuh:2445-2533;
 * launched at model.cuh:4616-4623).  For position blocks blk_lo ..
 * ceil(total_kv / block_size_n) - 1 of each kv head: the fp16 mean and the
 * sign-preserving max-abs over the block's dequantized keys, into
 * k_pool / k_pool_max [num_kv][n_blocks_stride][256] fp16.  Bit-identical to
 * the reference.  block_size_n <= 64. */
int qkv_tq3_kpool_update(const qkv_block_tq3* k_cache, uint16_t* k_pool, uint16_t* k_pool_max,
                         int num_kv, int head_dim, int total_kv, int blk_lo, int n_blocks_stride,
                         int block_size_n, hipStream_t stream);

/* Replaces build_block_index_ms_kern<256, GQA, 256><<<dim3(num_kv, sub_n),
 * 256, ...>>>(q, k_pool, k_pool_max, block_index, num_q, num_kv, sub_n,
 * sub_n_max, start_pos, top_k, block_size_n, n_blocks, n_blocks_stride, beta)
 * (sparse_attn/sparse_index.cuh:214-330; launched at model.cuh:4634-4637,
 * 4649-4652).  block_index [num_kv][sub_n_max][top_k] int32: per (kv head,
 * query t) the top_k blocks by max(q_avg . mean, beta * q_avg . maxabs) among
 * blocks 0 .. (start_pos + t) / block_size_n, ascending, -1 padded; ties go to
 * the lower block.  Bit-identical selection.  Unlike the reference (which
 * keeps one query's block scores in shared memory and rereads the pool per
 * query), the pool is read once for all sub_n queries and the scores pass
 * through a caller-provided workspace of
 * qkv_block_index_ms_workspace_bytes(num_kv, sub_n, n_blocks) bytes
 * (256-byte aligned, no initialisation needed).  k_pool / k_pool_max 16-byte
 * aligned. */
size_t qkv_block_index_ms_workspace_bytes(int num_kv, int sub_n, int n_blocks);
int qkv_block_index_ms(const uint16_t* q, const uint16_t* k_pool, const uint16_t* k_pool_max,
                       int32_t* block_index, int num_q, int num_kv, int head_dim, int sub_n,
                       int sub_n_max, int start_pos, int top_k, int block_size_n, int n_blocks,
                       int n_blocks_stride, float beta, void* workspace, size_t workspace_bytes,
                       hipStream_t stream);

/* Replaces flash_attn_chunk_block_sparse_split_tq3<256, GQA, 32, 256,
 * K_SPLITS><<<dim3(num_kv, sub_n, K_SPLITS), ...>>>(q, k_tq, v_tq,
 * block_index, part_m, part_l, part_o, num_q, num_kv, start_pos, sub_n,
 * sub_n_max, scale, top_k, block_size_n, tree_mask) (attention.cuh:2193-2433;
 * launched at model.cuh:4638-4644, 4653-4659): split z attends the blocks
 * block_index[...][z * ceil(top_k / k_splits) ...] (up to its first -1),
 * causal (and tree-masked) within the query's reach; partials in the
 * qkv_attn_split_tq3 layout.  block_size_n = 64; ceil(top_k / k_splits) <= 64. */
int qkv_attn_block_sparse_split_tq3(const uint16_t* q, const qkv_block_tq3* k,
                                    const qkv_block_tq3* v, const int32_t* block_index,
                                    float* part_m, float* part_l, float* part_o, int num_q,
                                    int num_kv, int head_dim, int start_pos, int sub_n,
                                    int sub_n_max, float scale, int top_k, int block_size_n,
                                    int k_splits, const uint32_t* tree_mask, hipStream_t stream);

/* Replaces flash_attn_split_merge<256, GQA, 256, K_SPLITS><<<(num_kv, sub_n), 256>>>
 * (attention.cuh:1837-1891).  out [sub_n][num_q][256] fp16; may alias q of the
 * preceding split call (model.cuh:2479-2482 merges in place). */
int qkv_attn_split_merge(const float* part_m, const float* part_l, const float* part_o,
                         uint16_t* out, int num_q, int num_kv, int head_dim, int sub_n,
                         int sub_n_max, int k_splits, hipStream_t stream);

/* Workspace bytes of qkv_decode_attn_tq3 for queries over up to
 * n_keys = start_pos + sub_n keys. */
size_t qkv_decode_attn_tq3_workspace_bytes(int num_q, int num_kv, int sub_n, int n_keys);

/* Fast path for the same computation as qkv_attn_split_tq3 + qkv_attn_split_merge
 * (model.cuh:2472-2491) in ONE launch: the key range is cut into chunks of
 * 512*k keys (the last one may also take a remainder of at most 64 keys),
 * partials stay in rotated coordinates and are merged inside the kernel (the
 * last workgroups of the grid do the merge), and each output row is rotated
 * back once.  The queries of a multi-token call (verify, sub_n > 1) share
 * passes over the cache: up to 16 (query, head) columns per pass, and calls
 * with more columns decode each tile once for up to 64 of them.
 * out [sub_n][num_q][256] fp16 (16-byte aligned).
 * workspace: caller-owned device memory of at least
 * qkv_decode_attn_tq3_workspace_bytes() bytes, 256-byte aligned, ZERO-FILLED
 * before its first use; every completed call leaves it ready for the next
 * one.  Calls sharing one workspace must be ordered (same stream). */
int qkv_decode_attn_tq3(const uint16_t* q, const qkv_block_tq3* k, const qkv_block_tq3* v,
                        uint16_t* out, int num_q, int num_kv, int head_dim, int start_pos,
                        int sub_n, float scale, int sink_tok, int window_tok,
                        const uint32_t* tree_mask, void* workspace, size_t workspace_bytes,
                        hipStream_t stream);

/* Health of a fast-path decode workspace (qkv_decode_attn_tq3, _q8, _q8_append,
 * _q8k_tq3v, _tq3_paged; for _tq3_noalloc see qkv_decode_noalloc_status
 * below).  The in-kernel merge waits for the records of its launch with
 * a bounded poll; if the bound runs out (a launch starved of GPU time for
 * seconds), the affected output rows are written as NaN and the workspace
 * header keeps an error word, after which every later call on that workspace
 * writes NaN rows until it is reset.  No counterpart in the reference (its
 * merge is a separate launch, attention.cuh:1837-1891).
 * qkv_decode_workspace_status synchronises `stream`, then returns QKV_OK or
 * QKV_ERR_TIMEOUT.  qkv_decode_workspace_reset zero-fills `bytes` bytes of
 * the workspace on `stream` (a fill kernel, no memset node: safe to capture). */
int qkv_decode_workspace_status(const void* workspace, hipStream_t stream);
int qkv_decode_workspace_reset(void* workspace, size_t bytes, hipStream_t stream);

/* The same health check without synchronising (serving loops, HIP graph
 * capture): enqueues on `stream` one single-thread kernel that writes QKV_OK or
 * QKV_ERR_TIMEOUT to *status -- device memory, or host memory the device can
 * write (hipHostMalloc) -- once every earlier call on the stream is done.
 * Read *status after the stream has passed that point.  Returns the launch
 * status (QKV_OK when the check was enqueued).  No counterpart in the
 * reference. */
int qkv_decode_workspace_status_async(const void* workspace, int* status, hipStream_t stream);

/* Test hook, no counterpart in the reference: the merger poll limit of every
 * later fast-path decode launch in this process (limit >= 0; a negative value
 * restores the default of 2^22 polls).  A limit of 0 makes every merger time
 * out, so the error path can be exercised without a GPU fault or hang. */
int qkv_debug_set_merge_spin_limit(int limit);

/* TQ3 append and decode of a multi-token (verify) block in one call.
 * Replaces the reference's verify-step sequence: the block's K and V encoded
 * into the cache (tq3_quantize_kernel, K then V, model.cuh:4566-4571;
 * turboquant.cuh:112-165) followed by the split attention of its sub_n
 * queries and the merge (model.cuh:4663-4687).  k_new, v_new are the block's
 * fp16 K and V rows [sub_n][num_kv][256] (16-byte aligned); they are encoded
 * exactly as qkv_tq3_append_kv encodes them and written to rows start_pos ..
 * start_pos + sub_n - 1 of k and v, and the attention is that of
 * qkv_decode_attn_tq3 with the same arguments.  It is ONE launch for a
 * decode step (sub_n = 1: the wave whose tile holds the new key encodes it)
 * and for calls with more than 16 (query, head) columns and sub_n <= 64 (the
 * shared-decode kernel encodes the new rows it reads); both write the rows to
 * the caches.  Other shapes take the append's launch, then the decode's.  Caches and output equal those of
 * qkv_tq3_append_kv followed by qkv_decode_attn_tq3; same workspace
 * (qkv_decode_attn_tq3_workspace_bytes(num_q, num_kv, sub_n,
 * start_pos + sub_n)) and errors. */
int qkv_decode_attn_tq3_append(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                               qkv_block_tq3* k, qkv_block_tq3* v, uint16_t* out, int num_q,
                               int num_kv, int head_dim, int start_pos, int sub_n, float scale,
                               int sink_tok, int window_tok, const uint32_t* tree_mask,
                               void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Allocation-free variant of qkv_decode_attn_tq3 (same arguments without the
 * workspace, same results).  No counterpart in the reference: it is for
 * callers that cannot allocate or own device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * workspace lives in a fixed 8 MiB scratch array that the library holds on
 * each GPU it runs on until the process ends; the call itself allocates
 * nothing.  qkv_tq3_init(device) looks the array up and zero-fills it (so
 * does the first call on a device if init was not called; it also re-clears
 * it, the reset after a merge timeout).  Shapes whose workspace
 * (qkv_decode_attn_tq3_workspace_bytes) exceeds 8 MiB return
 * QKV_ERR_WORKSPACE.  Every call on one GPU shares that GPU's scratch, which
 * each completed call leaves ready for the next: calls that overlap on one
 * GPU (different streams, or a concurrent qkv_tq3_init) race and must not be
 * issued. */
int qkv_decode_attn_tq3_noalloc(const uint16_t* q, const qkv_block_tq3* k,
                                const qkv_block_tq3* v, uint16_t* out, int num_q, int num_kv,
                                int head_dim, int start_pos, int sub_n, float scale, int sink_tok,
                                int window_tok, const uint32_t* tree_mask, hipStream_t stream);

/* Health and reset of the allocation-free decode's scratch on `device` (the
 * same error word as qkv_decode_workspace_status, for callers that never see
 * the scratch's address).  No counterpart in the reference.
 * qkv_decode_noalloc_status synchronises `stream` (a stream of `device`),
 * then returns QKV_OK or QKV_ERR_TIMEOUT; qkv_decode_noalloc_reset zero-fills
 * the scratch on `stream` (a fill kernel), clearing a sticky merge error.
 * Both make `device` current for the call and restore the caller's device. */
int qkv_decode_noalloc_status(int device, hipStream_t stream);
/* qkv_decode_workspace_status_async for the scratch of `device` (`stream` a
 * stream of `device`); no counterpart in the reference. */
int qkv_decode_noalloc_status_async(int device, int* status, hipStream_t stream);
int qkv_decode_noalloc_reset(int device, hipStream_t stream);

/* Fast path for qkv_attn_split_q8 + qkv_attn_split_merge over the Q8_0 cache
 * (decode launch model.cuh:2430-2463; attention.cuh:2633-2801 and 1837-1891) in ONE launch:
 * chunks of 128*k keys, records merged inside the kernel as for
 * qkv_decode_attn_tq3 (values are not rotated).  Same argument meaning as
 * qkv_attn_split_q8 (no sink/window/tree rules, as in the reference) with the
 * merged fp16 output and a workspace of qkv_decode_attn_q8_workspace_bytes()
 * bytes (256-byte aligned, zero-filled before first use, reused in order). */
size_t qkv_decode_attn_q8_workspace_bytes(int num_q, int num_kv, int sub_n, int n_keys);
int qkv_decode_attn_q8(const uint16_t* q, const qkv_block_q8* k, const qkv_block_q8* v,
                       uint16_t* out, int num_q, int num_kv, int head_dim, int start_pos,
                       int sub_n, float scale, void* workspace, size_t workspace_bytes,
                       hipStream_t stream);

/* Q8_0 append and decode of one new token in one launch.  Replaces the
 * reference's decode-step pair quantize_kv_q8_0_kern (K, then V; append,
 * model.cuh:2316-2333, attention.cuh:2587-2609) followed by the decode
 * attention (model.cuh:2430-2463): k_new, v_new are the token's fp16 K and V
 * rows [num_kv][256] (16-byte aligned); the kernel quantizes them exactly as
 * qkv_q8_append does, writes them to row start_pos of k and v (pad fields
 * untouched) and uses them as key start_pos of the attention of the one query
 * q over keys 0..start_pos.  The result and the caches equal those of
 * qkv_q8_append (K and V) followed by qkv_decode_attn_q8 with sub_n 1; same
 * workspace (qkv_decode_attn_q8_workspace_bytes(num_q, num_kv, 1,
 * start_pos + 1)) and errors. */
int qkv_decode_attn_q8_append(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                              qkv_block_q8* k, qkv_block_q8* v, uint16_t* out, int num_q,
                              int num_kv, int head_dim, int start_pos, float scale,
                              void* workspace, size_t workspace_bytes, hipStream_t stream);

/* V-only TurboQuant (TQ_KEYS_Q8=1): keys in Q8_0 (k, 8 blocks per kv head and
 * token), values in TQ3 (v, 2 blocks per kv head and token).  Replaces the
 * reference's unfused sequence for that mode (model.cuh:2574-2588:
 * dequantize_kv_q8_0_kern into fp16 scratch, attn_score_kernel_h, softmax,
 * then attn_value_kernel_tq3 over the TQ3 values; cache layout
 * model.cuh:1735-1748, append model.cuh:2323-2333) with one fused launch:
 * the qkv_decode_attn_q8 schedule, values accumulated in rotated coordinates
 * and rotated back by the in-kernel mergers.  Same arguments, errors and
 * workspace rules as qkv_decode_attn_q8. */
size_t qkv_decode_attn_q8k_tq3v_workspace_bytes(int num_q, int num_kv, int sub_n, int n_keys);
int qkv_decode_attn_q8k_tq3v(const uint16_t* q, const qkv_block_q8* k, const qkv_block_tq3* v,
                             uint16_t* out, int num_q, int num_kv, int head_dim, int start_pos,
                             int sub_n, float scale, void* workspace, size_t workspace_bytes,
                             hipStream_t stream);

/* Paged, ragged decode: one query per slot over per-slot block tables
 * This generalises the reference, which keeps every
 * slot contiguous and hands the attention launch a slot-base pointer
 * (model.cuh:1708-1715 kv_slot_offset, model.cuh:2466-2468); a block table
 * that maps block b of a slot to pool block base + b reproduces that call.
 * q, out: [n_slots][num_q][256] fp16 (16-byte aligned).
 * k_pool, v_pool: pool_rows token rows of num_kv*256/128 TQ3 blocks (the
 * contiguous cache's row layout).  Key k of slot s lives in pool row
 * block_tables[s*max_blocks + k/block_tokens]*block_tokens + k%block_tokens.
 * ctx_lens: device int32 [n_slots]; slot s attends to its keys
 * 0..ctx_lens[s]-1 (clamped to [0, max_ctx]; a slot without keys gets a zero
 * row).  block_tokens: a multiple of 64; max_ctx <= max_blocks*block_tokens.
 * Table entries pointing outside the pool read as zero keys.  Workspace: as
 * for qkv_decode_attn_tq3 (zero-filled before first use, reused in order). */
size_t qkv_decode_attn_tq3_paged_workspace_bytes(int num_q, int num_kv, int n_slots, int max_ctx);
int qkv_decode_attn_tq3_paged(const uint16_t* q, const qkv_block_tq3* k_pool,
                              const qkv_block_tq3* v_pool, uint16_t* out, int num_q, int num_kv,
                              int head_dim, int n_slots, const int32_t* block_tables,
                              int max_blocks, int block_tokens, int pool_rows,
                              const int32_t* ctx_lens, int max_ctx, float scale, void* workspace,
                              size_t workspace_bytes, hipStream_t stream);

/* Paged append of K and V (tq3_quantize_kernel, turboquant.cuh:112-165, with
 * the destination row of each token taken from the slot's block table):
 * k_f16, v_f16: [n_slots][n_tok][num_kv][256] fp16; token t of slot s is
 * written at position positions[s] + t of that slot (row rule as in
 * qkv_decode_attn_tq3_paged).  Tokens whose row falls outside
 * [0, pool_rows) or whose block index is >= max_blocks are not written. */
int qkv_tq3_append_kv_paged(const uint16_t* k_f16, const uint16_t* v_f16, qkv_block_tq3* k_pool,
                            qkv_block_tq3* v_pool, int n_slots, int n_tok, int num_kv,
                            int head_dim, const int32_t* block_tables, int max_blocks,
                            int block_tokens, int pool_rows, const int32_t* positions,
                            hipStream_t stream);

/* Chunked prefill attention over a TQ3 cache (BASELINE config 5(i)).
 * Replaces, for one slot, the reference's per-chunk sequence: bulk dequant of
 * the history into an fp16 scratch plus a copy of the chunk's fp16 K/V after
 * it (model.cuh:5189-5214), then per 16-token sub-chunk the split-K kernel
 * flash_attn_chunk_fused_split_ntb and flash_attn_split_merge over that
 * scratch (model.cuh:5256-5330, 5680-5721; attention.cuh:1690-1831,
 * 1837-1891).  The history is read from the packed cache directly.
 * q: [n_tok][num_q][256] fp16 (post-RoPE queries of chunk positions
 *    start_pos .. start_pos + n_tok - 1);
 * k_cache, v_cache: slot-base TQ3 caches whose rows 0 .. start_pos-1 hold
 *    the history (rows from start_pos on are not read);
 * k_chunk, v_chunk: [n_tok][num_kv][256] fp16, the chunk's own keys and
 *    values, attended unquantized as in the reference;
 * out: [n_tok][num_q][256] fp16.  Query token t attends to keys
 * 0 .. start_pos + t.  The append of the chunk into the cache is a separate
 * qkv_tq3_append_kv call (model.cuh:5176-5190).
 * Multi-token verify (model.cuh:4566-4571, 4663-4687: the verify block is
 * quantized first and attended from the cache): pass k_chunk = v_chunk =
 * NULL; every key, the block's own included, is then read from cache rows
 * 0 .. start_pos + n_tok - 1 (causal within the block; no tree mask -- tree,
 * sink and window rules stay with qkv_decode_attn_tq3).  GQA 4 and 6.  workspace:
 * caller-owned device memory of qkv_prefill_attn_tq3_workspace_bytes() bytes,
 * 256-byte aligned (no initialisation needed). */
size_t qkv_prefill_attn_tq3_workspace_bytes(int num_q, int num_kv, int n_tok, int start_pos);
int qkv_prefill_attn_tq3(const uint16_t* q, const qkv_block_tq3* k_cache,
                         const qkv_block_tq3* v_cache, const uint16_t* k_chunk,
                         const uint16_t* v_chunk, uint16_t* out, int num_q, int num_kv,
                         int head_dim, int start_pos, int n_tok, float scale, void* workspace,
                         size_t workspace_bytes, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* QKV_H */
