/*
 * qkv_oracle.h -- CPU restatement of the reference's compressed-KV path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP
 * kernels in qengine_amd/csrc: only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it.  The product path never calls it.
 *
 * Every function names the reference file:line it restates (paths relative to
 * the reference tree: src/turboquant.cuh, src/attention.cuh, src/quant_gemv.cuh).
 *
 * Pinning status (what independent check fixes each function) is listed in the
 * header of qkv_oracle.c.
 */
#ifndef QKV_ORACLE_H
#define QKV_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OR_TQ_BLOCK 128      /* turboquant.cuh:16  TQ_BLOCK_SIZE            */
#define OR_TQ_QS_BYTES 48    /* turboquant.cuh:75  128*3/8                  */
#define OR_Q8_BLOCK 32       /* quant_gemv.cuh:8   QK8                      */

/* turboquant.cuh:73-77: { float norm; uint8_t qs[48]; } -- 52 bytes. */
typedef struct {
    float norm;
    uint8_t qs[OR_TQ_QS_BYTES];
} or_block_tq3;

/* quant_gemv.cuh:19: { int8_t qs[32]; uint16_t pad; half d; } -- 36 bytes. */
typedef struct {
    int8_t qs[OR_Q8_BLOCK];
    uint16_t pad;
    uint16_t d; /* fp16 bits */
} or_block_q8;

/* ---- scalar helpers -------------------------------------------------- */
float or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);             /* round-to-nearest-even */
void or_f16_to_f32_n(const uint16_t* h, float* f, int64_t n);
void or_f32_to_f16_n(const float* f, uint16_t* h, int64_t n);

/* ---- codec constants ------------------------------------------------- */
void or_tq3_signs(float out[OR_TQ_BLOCK]);   /* turboquant.cuh:288-302 */
void or_tq3_centroids(float out[8]);         /* turboquant.cuh:27-30   */
void or_tq3_bounds(float out[7]);            /* turboquant.cuh:34-37   */
float or_tq3_wht_scale(void);                /* turboquant.cuh:61      */

/* ---- codec building blocks ------------------------------------------- */
void or_wht128(float* x);                                 /* turboquant.cuh:48-64   */
uint8_t or_tq3_find_bin(float v);                         /* turboquant.cuh:79-87   */
int64_t or_tq3_prescale_threshold_mismatches(const uint32_t* thr, int64_t lo, int64_t hi,
                                             int negated, int nthreads);
int64_t or_tq3_fold_mismatches(uint32_t a_bits, const uint32_t* q, int64_t lo, int64_t hi,
                               int negated, int nthreads);
void or_pack_3bit_8(uint8_t* dst, const uint8_t* idx8);   /* turboquant.cuh:90-100  */
void or_unpack_3bit_8(const uint8_t* src, uint8_t* idx8); /* turboquant.cuh:103-108 */

/* ---- TQ3 encode / decode (the append path) --------------------------- */
/* turboquant.cuh:112-165 */
void or_tq3_encode(const uint16_t* in_f16, or_block_tq3* out, int64_t n_blocks, int nthreads);
/* turboquant.cuh:112-165, but also returns the rotated, scaled coordinates
 * (y = rs*H*D*x/|x|) the bin search saw, for near-boundary reporting. */
void or_tq3_encode_rotated(const uint16_t* in_f16, or_block_tq3* out, float* rot,
                           int64_t n_blocks);
/* turboquant.cuh:169-200 (fp16 output) */
void or_tq3_decode(const or_block_tq3* in, uint16_t* out_f16, int64_t n_blocks, int nthreads);
/* turboquant.cuh:253-284 (fp32 output) */
void or_tq3_decode_f32(const or_block_tq3* in, float* out, int64_t n_blocks);

/* ---- Q8_0 KV encode / decode ----------------------------------------- */
/* attention.cuh:2587-2609 */
void or_q8_encode(const uint16_t* in_f16, or_block_q8* out, int64_t n_blocks, int nthreads);
/* attention.cuh:2614-2626 */
void or_q8_decode(const or_block_q8* in, uint16_t* out_f16, int64_t n_blocks, int nthreads);

/* ---- split-K flash decode and merge ---------------------------------- */
enum { OR_KV_TQ3 = 0, OR_KV_Q8 = 1, OR_KV_F16 = 2 };

/*
 * attention.cuh:1905-2177 (kind=OR_KV_TQ3), attention.cuh:2633-2801
 * (kind=OR_KV_Q8).  Same argument meaning and partial layouts:
 *   q      [sub_n][num_q][hd] fp16
 *   k, v   slot-base caches, token-major [pos][num_kv][hd/blk] blocks
 *   part_m, part_l [num_q][sub_n_max][k_splits] f32
 *   part_o [num_q][sub_n_max][k_splits][hd] f32
 * Tile size BM=32 tokens as in the reference instantiations
 * (model.cuh:2365, BM=32).  tree_mask may be NULL.
 */
void or_attn_split(int kind, const uint16_t* q, const void* k, const void* v,
                   float* part_m, float* part_l, float* part_o,
                   int num_q, int num_kv, int hd, int start_pos, int sub_n,
                   int sub_n_max, int active_end_max, float scale, int k_splits,
                   int sink_tok, int window_tok, const uint32_t* tree_mask,
                   int nthreads);

/* attention.cuh:1837-1891 */
void or_attn_split_merge(const float* part_m, const float* part_l, const float* part_o,
                         uint16_t* out, int num_q, int num_kv, int hd, int sub_n,
                         int sub_n_max, int k_splits);

/*
 * Independent fp64 attention over already-decoded fp16 K/V
 * (pattern of tools/dflash_attn_bench.cu:185-211): for query t, keys
 * [0, start_pos+t] filtered by the same visibility rule (causal, tree mask,
 * sink/window tile rule); softmax in double.  out [sub_n][num_q][hd] f64.
 */
void or_attn_ref_f64(const uint16_t* q, const uint16_t* k_f16, const uint16_t* v_f16,
                     double* out, int num_q, int num_kv, int hd, int start_pos,
                     int sub_n, double scale, int sink_tok, int window_tok,
                     const uint32_t* tree_mask);
/* The same fp64 attention over float K/V (e.g. the exact TQ3 dequantization
 * before its fp16 rounding): the truth the rotated-domain kernels are held to. */
void or_attn_ref_f64_f32kv(const uint16_t* q, const float* k, const float* v, double* out,
                           int num_q, int num_kv, int hd, int start_pos, int sub_n, double scale,
                           int sink_tok, int window_tok, const uint32_t* tree_mask);

/* Visibility rule shared by the split kernel and the fp64 reference:
 * attention.cuh:1941-1951 (causal), 1985-1994 (sink/window tile skip),
 * 2101-2105 (tree bits).  Returns 1 if query t_idx sees key `key`. */
int or_key_visible(int key, int start_pos, int t_idx, int sink_tok, int window_tok,
                   const uint32_t* tree_mask);

/* Legacy short-context decode of one query token over seq_len rows
 * (model.cuh:2544-2664): fp16 scratch + attn_score_kernel_h + softmax_kernel +
 * attn_value_kernel_h, or with tq_fused the fp32 TQ3 kernels
 * (attention.cuh:400-483, 920-989) for TQ3 operands.  k_kind / v_kind are
 * OR_KV_*; q [num_q][hd] fp16; out [num_q][hd] fp16; probs (optional)
 * receives the normalized softmax rows [num_q][seq_len].  Returns 0, or -1 for
 * an unsupported shape. */
int or_legacy_decode(int k_kind, int v_kind, int tq_fused, const uint16_t* q, const void* k,
                     const void* v, uint16_t* out, float* probs, int num_q, int num_kv, int hd,
                     int seq_len, float scale);

/* dfki2_dequant_kernel (model.cuh:149-159): DFK2 int8 plane rows of kv_dim
 * elements with one fp16 scale per 128 to fp16. */
void or_dfk2_dequant(const int8_t* q, const uint16_t* s, uint16_t* out, int64_t n, int kv_dim);

/* Block-sparse TQ3 verify: K-pool signatures (attention.cuh:2445-2533), the
 * MS top-k block index (sparse_attn/sparse_index.cuh:214-330) and the sparse
 * split kernel (attention.cuh:2193-2433; merge with or_attn_split_merge). */
void or_tq3_kpool_update(const or_block_tq3* k, uint16_t* k_pool, uint16_t* k_pool_max,
                         int num_kv, int hd, int total_kv, int blk_lo, int n_blocks_stride,
                         int bsn);
/* block scores [num_kv][sub_n][n_blocks] of build_block_index_ms_kern
 * (sparse_index.cuh:243-290): the first half of or_block_index_ms. */
void or_block_scores_ms(const uint16_t* q, const uint16_t* k_pool, const uint16_t* k_pool_max,
                        float* scores, int num_q, int num_kv, int hd, int sub_n, int start_pos,
                        int bsn, int n_blocks, int n_blocks_stride, float beta);
void or_block_index_ms(const uint16_t* q, const uint16_t* k_pool, const uint16_t* k_pool_max,
                       int32_t* block_index, int num_q, int num_kv, int hd, int sub_n,
                       int sub_n_max, int start_pos, int top_k, int bsn, int n_blocks,
                       int n_blocks_stride, float beta);
void or_attn_block_sparse_split(const uint16_t* q, const or_block_tq3* k, const or_block_tq3* v,
                                const int32_t* block_index, float* part_m, float* part_l,
                                float* part_o, int num_q, int num_kv, int hd, int start_pos,
                                int sub_n, int sub_n_max, float scale, int top_k, int bsn,
                                int k_splits, const uint32_t* tree_mask);

#ifdef __cplusplus
}
#endif
#endif
