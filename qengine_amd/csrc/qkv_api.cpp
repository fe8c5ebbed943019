// qkv_api.cpp -- the extern "C" surface of libqkv.so (declared in include/qkv.h).
//
// Each entry point validates its arguments, then launches on the caller's
// stream.  Nothing here allocates device memory or synchronises the host.
#include "../../include/qkv.h"

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstring>
#include <mutex>

#include "attn_common.h"
#include "qkv_launch.h"

namespace {

constexpr int kVersion = 100;  // 0.1.0

inline bool aligned(const void* p, size_t a) {
  return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

inline int launch_status(hipError_t e) { return e == hipSuccess ? QKV_OK : QKV_ERR_LAUNCH; }

std::mutex g_init_mu;
bool g_init_ok[64];
std::atomic<int> g_spin_limit{qkv::kMergeSpinLimit};

}  // namespace

extern "C" {

int qkv_version(void) { return kVersion; }

const char* qkv_status_string(int s) {
  switch (s) {
    case QKV_OK: return "ok";
    case QKV_ERR_INVALID: return "invalid argument";
    case QKV_ERR_NULL: return "null pointer";
    case QKV_ERR_UNSUPPORTED: return "unsupported head_dim/GQA combination";
    case QKV_ERR_ALIGN: return "misaligned pointer";
    case QKV_ERR_DEVICE: return "no usable gfx950 device";
    case QKV_ERR_LAUNCH: return "kernel launch failed";
    case QKV_ERR_WORKSPACE: return "workspace missing or too small";
    case QKV_ERR_TIMEOUT: return "in-kernel merge timed out; reset the workspace";
    default: return "unknown status";
  }
}

int qkv_tq3_init(int device) {
  if (device < 0 || device >= 64) return QKV_ERR_INVALID;
  std::lock_guard<std::mutex> lk(g_init_mu);
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || device >= n) return QKV_ERR_DEVICE;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return QKV_ERR_DEVICE;
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) return QKV_ERR_DEVICE;
  g_init_ok[device] = true;
  // the allocation-free decode's scratch on this device: looked up and zero-filled
  int cur = 0;
  if (hipGetDevice(&cur) != hipSuccess) return QKV_ERR_DEVICE;
  if (hipSetDevice(device) != hipSuccess) return QKV_ERR_DEVICE;
  void* ptr = nullptr;
  const bool ok = qkv::noalloc_scratch(device, true, nullptr, &ptr) == hipSuccess &&
                  hipStreamSynchronize(nullptr) == hipSuccess;
  if (hipSetDevice(cur) != hipSuccess || !ok) return QKV_ERR_DEVICE;
  return QKV_OK;
}

int qkv_tq3_append(const uint16_t* in_f16, qkv_block_tq3* out, int n_blocks, hipStream_t stream) {
  if (n_blocks < 0) return QKV_ERR_INVALID;
  if (n_blocks == 0) return QKV_OK;
  if (!in_f16 || !out) return QKV_ERR_NULL;
  if (!aligned(in_f16, 16) || !aligned(out, 4)) return QKV_ERR_ALIGN;
  return launch_status(qkv::launch_tq3_append(in_f16, out, in_f16, out, n_blocks, 1, stream));
}

int qkv_tq3_append_kv(const uint16_t* k_f16, const uint16_t* v_f16, qkv_block_tq3* k_out,
                      qkv_block_tq3* v_out, int n_blocks, hipStream_t stream) {
  if (n_blocks < 0) return QKV_ERR_INVALID;
  if (n_blocks == 0) return QKV_OK;
  if (!k_f16 || !v_f16 || !k_out || !v_out) return QKV_ERR_NULL;
  if (!aligned(k_f16, 16) || !aligned(v_f16, 16) || !aligned(k_out, 4) || !aligned(v_out, 4))
    return QKV_ERR_ALIGN;
  return launch_status(qkv::launch_tq3_append(k_f16, k_out, v_f16, v_out, n_blocks, 2, stream));
}

int qkv_tq3_append_kv_paged(const uint16_t* k_f16, const uint16_t* v_f16, qkv_block_tq3* k_pool,
                            qkv_block_tq3* v_pool, int n_slots, int n_tok, int num_kv,
                            int head_dim, const int32_t* block_tables, int max_blocks,
                            int block_tokens, int pool_rows, const int32_t* positions,
                            hipStream_t stream) {
  if (head_dim != 256) return QKV_ERR_UNSUPPORTED;
  if (n_slots < 0 || n_tok < 0 || num_kv <= 0 || max_blocks <= 0 || block_tokens <= 0 ||
      pool_rows < 0)
    return QKV_ERR_INVALID;
  if (n_slots == 0 || n_tok == 0) return QKV_OK;
  if (!k_f16 || !v_f16 || !k_pool || !v_pool || !block_tables || !positions) return QKV_ERR_NULL;
  if (!aligned(k_f16, 16) || !aligned(v_f16, 16) || !aligned(k_pool, 4) || !aligned(v_pool, 4) ||
      !aligned(block_tables, 4) || !aligned(positions, 4))
    return QKV_ERR_ALIGN;
  const int bpr = num_kv * head_dim / 128;
  const long n_blocks = (long)n_slots * n_tok * bpr;
  if (n_blocks > 0x7fffffffL) return QKV_ERR_UNSUPPORTED;
  qkv::PagedRows pr{};
  pr.block_tables = block_tables;
  pr.positions = positions;
  pr.max_blocks = max_blocks;
  pr.block_tokens = block_tokens;
  pr.blocks_per_row = bpr;
  pr.n_tok = n_tok;
  pr.pool_rows = pool_rows;
  return launch_status(
      qkv::launch_tq3_append(k_f16, k_pool, v_f16, v_pool, (int)n_blocks, 2, stream, &pr));
}

int qkv_tq3_dequant(const qkv_block_tq3* in, uint16_t* out_f16, int n_blocks, hipStream_t stream) {
  if (n_blocks < 0) return QKV_ERR_INVALID;
  if (n_blocks == 0) return QKV_OK;
  if (!in || !out_f16) return QKV_ERR_NULL;
  if (!aligned(in, 4) || !aligned(out_f16, 16)) return QKV_ERR_ALIGN;
  return launch_status(qkv::launch_tq3_dequant(in, out_f16, n_blocks, stream));
}

int qkv_q8_append(const uint16_t* in_f16, qkv_block_q8* out, int n_blocks, hipStream_t stream) {
  if (n_blocks < 0) return QKV_ERR_INVALID;
  if (n_blocks == 0) return QKV_OK;
  if (!in_f16 || !out) return QKV_ERR_NULL;
  if (!aligned(in_f16, 16) || !aligned(out, 4)) return QKV_ERR_ALIGN;
  return launch_status(qkv::launch_q8_append(in_f16, out, in_f16, out, n_blocks, 1, stream));
}

int qkv_q8_append_kv(const uint16_t* k_f16, const uint16_t* v_f16, qkv_block_q8* k_out,
                     qkv_block_q8* v_out, int n_blocks, hipStream_t stream) {
  if (n_blocks < 0) return QKV_ERR_INVALID;
  if (n_blocks == 0) return QKV_OK;
  if (!k_f16 || !v_f16 || !k_out || !v_out) return QKV_ERR_NULL;
  if (!aligned(k_f16, 16) || !aligned(v_f16, 16) || !aligned(k_out, 4) || !aligned(v_out, 4))
    return QKV_ERR_ALIGN;
  return launch_status(qkv::launch_q8_append(k_f16, k_out, v_f16, v_out, n_blocks, 2, stream));
}
int qkv_dfk2_dequant(const int8_t* q, const uint16_t* scales, uint16_t* out_f16, long long n,
                     int kv_dim, hipStream_t stream) {
  if (n < 0 || kv_dim <= 0) return QKV_ERR_INVALID;
  if (kv_dim % 128 != 0 || n % 8 != 0) return QKV_ERR_UNSUPPORTED;
  if (n == 0) return QKV_OK;
  if (!q || !scales || !out_f16) return QKV_ERR_NULL;
  if (!aligned(q, 8) || !aligned(scales, 2) || !aligned(out_f16, 16)) return QKV_ERR_ALIGN;
  return launch_status(qkv::launch_dfk2_dequant(q, scales, out_f16, (long)n, stream));
}

int qkv_tq3_append_dfk2(const int8_t* q, const uint16_t* scales, qkv_block_tq3* out,
                        int n_blocks, hipStream_t stream) {
  if (n_blocks < 0) return QKV_ERR_INVALID;
  if (n_blocks == 0) return QKV_OK;
  if (!q || !scales || !out) return QKV_ERR_NULL;
  if (!aligned(q, 16) || !aligned(scales, 2) || !aligned(out, 4)) return QKV_ERR_ALIGN;
  return launch_status(
      qkv::launch_tq3_append(q, out, q, out, n_blocks, 1, stream, nullptr, scales, scales));
}

int qkv_q8_append_dfk2(const int8_t* q, const uint16_t* scales, qkv_block_q8* out, int n_blocks,
                       hipStream_t stream) {
  if (n_blocks < 0) return QKV_ERR_INVALID;
  if (n_blocks % 4 != 0) return QKV_ERR_UNSUPPORTED;
  if (n_blocks == 0) return QKV_OK;
  if (!q || !scales || !out) return QKV_ERR_NULL;
  if (!aligned(q, 8) || !aligned(scales, 2) || !aligned(out, 4)) return QKV_ERR_ALIGN;
  return launch_status(qkv::launch_q8_append(q, out, q, out, n_blocks, 1, stream, scales, scales));
}

int qkv_kv_move_tokens(void* k, void* v, size_t k_row_bytes, size_t v_row_bytes, long slot_row0,
                       long slot_rows, const int32_t* from_to, int n, hipStream_t stream) {
  if (n < 0 || n > qkv::kMoveMax) return QKV_ERR_INVALID;
  if (n == 0) return QKV_OK;
  if (!k || !v || !from_to) return QKV_ERR_NULL;
  if (k_row_bytes == 0 || v_row_bytes == 0 || k_row_bytes % 4 || v_row_bytes % 4 ||
      k_row_bytes > 0xffffffffULL || v_row_bytes > 0xffffffffULL || slot_row0 < 0 || slot_rows <= 0)
    return QKV_ERR_INVALID;
  if (!aligned(k, 4) || !aligned(v, 4)) return QKV_ERR_ALIGN;
  qkv::MoveArgs a{};
  a.k = static_cast<uint8_t*>(k);
  a.v = static_cast<uint8_t*>(v);
  a.k_row_bytes = (uint32_t)k_row_bytes;
  a.v_row_bytes = (uint32_t)v_row_bytes;
  a.slot_row0 = slot_row0;
  a.n = n;
  for (int i = 0; i < n; i++) {
    a.from[i] = from_to[2 * i];
    a.to[i] = from_to[2 * i + 1];
    if (a.from[i] < 0 || a.from[i] >= slot_rows || a.to[i] < 0 || a.to[i] >= slot_rows)
      return QKV_ERR_INVALID;
  }
  // in list order unless no row written by one move is read or written by another
  bool ordered = false;
  for (int i = 0; i < n && !ordered; i++) {
    if (a.from[i] == a.to[i]) continue;
    for (int j = 0; j < n; j++)
      if (j != i && a.from[j] != a.to[j] && (a.to[i] == a.from[j] || a.to[i] == a.to[j])) {
        ordered = true;
        break;
      }
  }
  return launch_status(qkv::launch_kv_move(a, ordered, stream));
}

static int kv_page_copy(void* k_pool, void* v_pool, void* k_flat, void* v_flat,
                        size_t k_row_bytes, size_t v_row_bytes, long pool_rows,
                        const int32_t* block_table, int max_blocks, int block_tokens, int n_rows,
                        bool scatter, hipStream_t stream) {
  if (n_rows < 0 || max_blocks <= 0 || block_tokens <= 0 || pool_rows < 0) return QKV_ERR_INVALID;
  if (n_rows == 0) return QKV_OK;
  if (!k_pool || !k_flat || !block_table) return QKV_ERR_NULL;
  if ((v_pool == nullptr) != (v_flat == nullptr)) return QKV_ERR_NULL;
  const int n_tensors = v_pool ? 2 : 1;
  if (k_row_bytes == 0 || k_row_bytes % 4 || k_row_bytes > 0x7fffffffULL) return QKV_ERR_INVALID;
  if (n_tensors == 2 && (v_row_bytes == 0 || v_row_bytes % 4 || v_row_bytes > 0x7fffffffULL))
    return QKV_ERR_INVALID;
  if ((long)(n_rows - 1) / block_tokens >= max_blocks) return QKV_ERR_INVALID;
  if (!aligned(k_pool, 4) || !aligned(k_flat, 4) || !aligned(block_table, 4) ||
      (n_tensors == 2 && (!aligned(v_pool, 4) || !aligned(v_flat, 4))))
    return QKV_ERR_ALIGN;
  qkv::PageCopyArgs a{};
  a.pool[0] = static_cast<uint8_t*>(k_pool);
  a.flat[0] = static_cast<uint8_t*>(k_flat);
  a.row_bytes[0] = (uint32_t)k_row_bytes;
  a.pool[1] = n_tensors == 2 ? static_cast<uint8_t*>(v_pool) : a.pool[0];
  a.flat[1] = n_tensors == 2 ? static_cast<uint8_t*>(v_flat) : a.flat[0];
  a.row_bytes[1] = n_tensors == 2 ? (uint32_t)v_row_bytes : a.row_bytes[0];
  a.table = block_table;
  a.max_blocks = max_blocks;
  a.block_tokens = block_tokens;
  a.n_rows = n_rows;
  a.n_tensors = n_tensors;
  a.pool_rows = pool_rows;
  a.aligned16 = aligned(a.pool[0], 16) && aligned(a.pool[1], 16) && aligned(a.flat[0], 16) &&
                aligned(a.flat[1], 16);
  return launch_status(qkv::launch_kv_page_copy(a, scatter, stream));
}

int qkv_kv_gather_rows(const void* k_pool, const void* v_pool, void* k_flat, void* v_flat,
                       size_t k_row_bytes, size_t v_row_bytes, long pool_rows,
                       const int32_t* block_table, int max_blocks, int block_tokens, int n_rows,
                       hipStream_t stream) {
  return kv_page_copy(const_cast<void*>(k_pool), const_cast<void*>(v_pool), k_flat, v_flat,
                      k_row_bytes, v_row_bytes, pool_rows, block_table, max_blocks, block_tokens,
                      n_rows, false, stream);
}

int qkv_kv_scatter_rows(void* k_pool, void* v_pool, const void* k_flat, const void* v_flat,
                        size_t k_row_bytes, size_t v_row_bytes, long pool_rows,
                        const int32_t* block_table, int max_blocks, int block_tokens, int n_rows,
                        hipStream_t stream) {
  return kv_page_copy(k_pool, v_pool, const_cast<void*>(k_flat), const_cast<void*>(v_flat),
                      k_row_bytes, v_row_bytes, pool_rows, block_table, max_blocks, block_tokens,
                      n_rows, true, stream);
}

int qkv_q8_dequant(const qkv_block_q8* in, uint16_t* out_f16, int n_blocks, hipStream_t stream) {
  if (n_blocks < 0) return QKV_ERR_INVALID;
  if (n_blocks == 0) return QKV_OK;
  if (!in || !out_f16) return QKV_ERR_NULL;
  if (!aligned(in, 4) || !aligned(out_f16, 16)) return QKV_ERR_ALIGN;
  return launch_status(qkv::launch_q8_dequant(in, out_f16, n_blocks, stream));
}

}  // extern "C"

// ---------------------------------------------------------------------------
// attention
// ---------------------------------------------------------------------------
namespace {

constexpr int kChunkKeys = 512;     // TQ3 fast path: 8 waves x 64-key tiles
constexpr int kChunkKeysQ8 = 128;   // Q8 fast path: 4 waves x 32-key tiles
constexpr long kMaxFastWgs = 256;   // TQ3 fast path: one workgroup per CU of an MI355X

int check_attn_shape(int num_q, int num_kv, int head_dim, int start_pos, int sub_n,
                     const uint32_t* tree_mask) {
  if (head_dim != 256) return QKV_ERR_UNSUPPORTED;
  if (num_kv <= 0 || num_q <= 0 || num_q % num_kv != 0) return QKV_ERR_INVALID;
  if (num_q / num_kv > 8 || num_q > qkv::kLeadMaxHeads) return QKV_ERR_UNSUPPORTED;
  if (start_pos < 0 || sub_n < 1) return QKV_ERR_INVALID;
  if (tree_mask && sub_n > 32) return QKV_ERR_INVALID;
  return QKV_OK;
}

}  // namespace

extern "C" {

int qkv_attn_split_tq3(const uint16_t* q, const qkv_block_tq3* k, const qkv_block_tq3* v,
                       float* part_m, float* part_l, float* part_o, int num_q, int num_kv,
                       int head_dim, int start_pos, int sub_n, int sub_n_max,
                       int active_end_max, float scale, int k_splits, int sink_tok,
                       int window_tok, const uint32_t* tree_mask, hipStream_t stream) {
  int st = check_attn_shape(num_q, num_kv, head_dim, start_pos, sub_n, tree_mask);
  if (st) return st;
  if (sub_n > sub_n_max || k_splits < 1 || k_splits > 65536 || active_end_max < 1 ||
      sink_tok < 0 || window_tok < 0)
    return QKV_ERR_INVALID;
  if (!q || !k || !v || !part_m || !part_l || !part_o) return QKV_ERR_NULL;
  if (!aligned(q, 16) || !aligned(k, 4) || !aligned(v, 4) || !aligned(part_m, 4) ||
      !aligned(part_l, 4) || !aligned(part_o, 4))
    return QKV_ERR_ALIGN;
  qkv::AttnArgs a{};
  a.q = q;
  a.k = reinterpret_cast<const uint32_t*>(k);
  a.v = reinterpret_cast<const uint32_t*>(v);
  a.num_q = num_q;
  a.num_kv = num_kv;
  a.start_pos = start_pos;
  a.sub_n = sub_n;
  a.sub_n_max = sub_n_max;
  a.qpw = 8 / (num_q / num_kv);   // queries share MFMA columns 0..7 (8..15: query remainders)
  {
    const uint64_t extent = (uint64_t)(start_pos + sub_n) * num_kv * 104;
    a.kv_bytes = extent;
  }
  a.active_end_max = active_end_max;
  a.k_splits = k_splits;
  a.n_chunks = k_splits;
  a.scale_log2 = scale * qkv::kLog2e;
  a.sink_tok = sink_tok;
  a.window_tok = window_tok;
  a.tree_mask = tree_mask;
  a.part_m = part_m;
  a.part_l = part_l;
  a.part_o = part_o;
  return launch_status(qkv::launch_tq3_attn(a, 1, nullptr, stream));
}

int qkv_tq3_kpool_update(const qkv_block_tq3* k_cache, uint16_t* k_pool, uint16_t* k_pool_max,
                         int num_kv, int head_dim, int total_kv, int blk_lo, int n_blocks_stride,
                         int block_size_n, hipStream_t stream) {
  if (head_dim != 256) return QKV_ERR_UNSUPPORTED;
  if (block_size_n < 1 || block_size_n > 64) return QKV_ERR_UNSUPPORTED;
  if (num_kv <= 0 || total_kv < 0 || blk_lo < 0 || n_blocks_stride <= 0) return QKV_ERR_INVALID;
  const int cur_blocks = (int)(((long)total_kv + block_size_n - 1) / block_size_n);
  if (cur_blocks > n_blocks_stride) return QKV_ERR_INVALID;
  if (blk_lo >= cur_blocks) return QKV_OK;
  if ((long)num_kv * (cur_blocks - blk_lo) > 0x7fffffffL) return QKV_ERR_UNSUPPORTED;
  if (!k_cache || !k_pool || !k_pool_max) return QKV_ERR_NULL;
  if (!aligned(k_cache, 4) || !aligned(k_pool, 2) || !aligned(k_pool_max, 2)) return QKV_ERR_ALIGN;
  qkv::KpoolArgs a{};
  a.k = reinterpret_cast<const uint32_t*>(k_cache);
  a.k_pool = k_pool;
  a.k_pool_max = k_pool_max;
  a.num_kv = num_kv;
  a.total_kv = total_kv;
  a.blk_lo = blk_lo;
  a.cur_blocks = cur_blocks;
  a.stride = n_blocks_stride;
  a.bsn = block_size_n;
  return launch_status(qkv::launch_tq3_kpool(a, stream));
}

size_t qkv_block_index_ms_workspace_bytes(int num_kv, int sub_n, int n_blocks) {
  if (num_kv <= 0 || sub_n <= 0 || n_blocks <= 0) return 0;
  return ((size_t)num_kv * sub_n * n_blocks * 4 + 255) & ~(size_t)255;
}

int qkv_block_index_ms(const uint16_t* q, const uint16_t* k_pool, const uint16_t* k_pool_max,
                       int32_t* block_index, int num_q, int num_kv, int head_dim, int sub_n,
                       int sub_n_max, int start_pos, int top_k, int block_size_n, int n_blocks,
                       int n_blocks_stride, float beta, void* workspace, size_t workspace_bytes,
                       hipStream_t stream) {
  if (head_dim != 256) return QKV_ERR_UNSUPPORTED;
  if (num_kv <= 0 || num_q <= 0 || num_q % num_kv != 0 || sub_n < 1 || sub_n > sub_n_max ||
      start_pos < 0 || top_k < 1 || block_size_n < 1 || n_blocks < 1 ||
      n_blocks > n_blocks_stride)
    return QKV_ERR_INVALID;
  if (!q || !k_pool || !k_pool_max || !block_index) return QKV_ERR_NULL;
  if (!aligned(q, 4) || !aligned(k_pool, 16) || !aligned(k_pool_max, 16) ||
      !aligned(block_index, 4))
    return QKV_ERR_ALIGN;
  if (!workspace || workspace_bytes < qkv_block_index_ms_workspace_bytes(num_kv, sub_n, n_blocks))
    return QKV_ERR_WORKSPACE;
  if (!aligned(workspace, 256)) return QKV_ERR_ALIGN;
  qkv::BlockIndexArgs a{};
  a.q = q;
  a.k_pool = k_pool;
  a.k_pool_max = k_pool_max;
  a.block_index = block_index;
  a.num_q = num_q;
  a.num_kv = num_kv;
  a.sub_n = sub_n;
  a.sub_n_max = sub_n_max;
  a.start_pos = start_pos;
  a.top_k = top_k;
  a.bsn = block_size_n;
  a.n_blocks = n_blocks;
  a.stride = n_blocks_stride;
  a.beta = beta;
  a.inv_gqa = 1.0f / (float)(num_q / num_kv);
  return launch_status(qkv::launch_block_index(a, static_cast<float*>(workspace), stream));
}

int qkv_attn_block_sparse_split_tq3(const uint16_t* q, const qkv_block_tq3* k,
                                    const qkv_block_tq3* v, const int32_t* block_index,
                                    float* part_m, float* part_l, float* part_o, int num_q,
                                    int num_kv, int head_dim, int start_pos, int sub_n,
                                    int sub_n_max, float scale, int top_k, int block_size_n,
                                    int k_splits, const uint32_t* tree_mask, hipStream_t stream) {
  int st = check_attn_shape(num_q, num_kv, head_dim, start_pos, sub_n, tree_mask);
  if (st) return st;
  if (block_size_n != 64) return QKV_ERR_UNSUPPORTED;   // one 64-key tile per block
  if (sub_n > sub_n_max || top_k < 1 || k_splits < 1 || k_splits > 65536) return QKV_ERR_INVALID;
  if ((top_k + k_splits - 1) / k_splits > 64) return QKV_ERR_UNSUPPORTED;   // <= 64 blocks per split
  if (!q || !k || !v || !block_index || !part_m || !part_l || !part_o) return QKV_ERR_NULL;
  if (!aligned(q, 16) || !aligned(k, 4) || !aligned(v, 4) || !aligned(block_index, 4) ||
      !aligned(part_m, 4) || !aligned(part_l, 4) || !aligned(part_o, 4))
    return QKV_ERR_ALIGN;
  qkv::AttnArgs a{};
  a.q = q;
  a.k = reinterpret_cast<const uint32_t*>(k);
  a.v = reinterpret_cast<const uint32_t*>(v);
  a.num_q = num_q;
  a.num_kv = num_kv;
  a.start_pos = start_pos;
  a.sub_n = sub_n;
  a.sub_n_max = sub_n_max;
  a.qpw = 1;   // every query has its own block list
  a.kv_bytes = (uint64_t)(start_pos + sub_n) * num_kv * 104;
  a.active_end_max = start_pos + sub_n;
  a.k_splits = k_splits;
  a.n_chunks = k_splits;
  a.scale_log2 = scale * qkv::kLog2e;
  a.tree_mask = tree_mask;
  a.block_index = block_index;
  a.top_k = top_k;
  a.part_m = part_m;
  a.part_l = part_l;
  a.part_o = part_o;
  return launch_status(qkv::launch_tq3_attn(a, 2, nullptr, stream));
}

int qkv_attn_split_q8(const uint16_t* q, const qkv_block_q8* k, const qkv_block_q8* v,
                      float* part_m, float* part_l, float* part_o, int num_q, int num_kv,
                      int head_dim, int start_pos, int sub_n, int sub_n_max, int active_end_max,
                      float scale, int k_splits, hipStream_t stream) {
  int st = check_attn_shape(num_q, num_kv, head_dim, start_pos, sub_n, nullptr);
  if (st) return st;
  if (sub_n > sub_n_max || k_splits < 1 || k_splits > 65536 || active_end_max < 1)
    return QKV_ERR_INVALID;
  if ((int64_t)num_kv * sub_n * k_splits > 0x7fffffff) return QKV_ERR_INVALID;
  if (!q || !k || !v || !part_m || !part_l || !part_o) return QKV_ERR_NULL;
  if (!aligned(q, 16) || !aligned(k, 4) || !aligned(v, 4) || !aligned(part_m, 4) ||
      !aligned(part_l, 4) || !aligned(part_o, 4))
    return QKV_ERR_ALIGN;
  qkv::AttnArgs a{};
  a.q = q;
  a.k = reinterpret_cast<const uint32_t*>(k);
  a.v = reinterpret_cast<const uint32_t*>(v);
  a.num_q = num_q;
  a.num_kv = num_kv;
  a.start_pos = start_pos;
  a.sub_n = sub_n;
  a.sub_n_max = sub_n_max;
  {
    const uint64_t extent = (uint64_t)(start_pos + sub_n) * num_kv * 8 * sizeof(qkv_block_q8);
    a.kv_bytes = extent;
  }
  a.active_end_max = active_end_max;
  a.k_splits = k_splits;
  a.n_chunks = k_splits;
  a.scale_log2 = scale * qkv::kLog2e;
  a.part_m = part_m;
  a.part_l = part_l;
  a.part_o = part_o;
  return launch_status(qkv::launch_q8_attn_split(a, stream));
}

int qkv_attn_split_merge(const float* part_m, const float* part_l, const float* part_o,
                         uint16_t* out, int num_q, int num_kv, int head_dim, int sub_n,
                         int sub_n_max, int k_splits, hipStream_t stream) {
  if (head_dim != 256) return QKV_ERR_UNSUPPORTED;
  if (num_q <= 0 || num_kv <= 0 || num_q % num_kv || sub_n < 1 || sub_n > sub_n_max ||
      k_splits < 1 || k_splits > 65536)
    return QKV_ERR_INVALID;
  if (!part_m || !part_l || !part_o || !out) return QKV_ERR_NULL;
  if (!aligned(part_m, 4) || !aligned(part_l, 4) || !aligned(part_o, 4) || !aligned(out, 2))
    return QKV_ERR_ALIGN;
  return launch_status(
      qkv::launch_split_merge(part_m, part_l, part_o, out, num_q, sub_n, sub_n_max, k_splits, stream));
}

namespace {
struct FastGeom {
  int chunk_keys, n_chunks, n_slots;
  size_t header_off, ml_off, o_off, total;
};
// Chunks of base*tpw keys, at most 128 per (kv head, query): one record per
// chunk and q head, merged by the designated merger workgroups.
// Query groups of a contiguous TQ3 fast-path launch (16 / GQA queries share a
// workgroup's MFMA columns).
int tq3_fast_qpw(int num_q, int num_kv, int sub_n) {
  const int gqa = num_q / num_kv;
  // more than 16 (query, head) columns: up to 64 columns per workgroup, every
  // tile decoded once for all of them (tq3_mq_kernel)
  if (sub_n * gqa > 16) return std::min(sub_n, 64 / gqa);
  // one query group of rounded queries + remainders in the 16 MFMA columns, or,
  // when the call has more queries than that, 16 / GQA queries per group with
  // the remainders in a chained product (tq3_attn_kernel<0, true>)
  return sub_n > 8 / gqa ? 16 / gqa : 8 / gqa;
}
int tq3_groups(int num_q, int num_kv, int sub_n) {
  const int qpw = tq3_fast_qpw(num_q, num_kv, sub_n);
  return (sub_n + qpw - 1) / qpw;
}
// Chunk size (in 512-key steps) from which a contiguous TQ3 launch joins a
// last chunk of at most one 64-key tile to the previous chunk (its kernel runs
// the last chunk to the end of the keys).  tq3_attn_kernel spreads a chunk
// over its 8 waves, so the join pays from 4 tiles per wave on (one wave takes
// one more tile instead of every wave one more round: a 16-token verify over
// 131,072 + 16 keys, 16 chunks of 16 tiles per wave and a 16-key tile, not 16
// chunks of 17); tq3_mq_kernel runs a chunk's tiles one after another with all
// of its waves, so one more tile never costs a round (32,768 + 16 keys: 64
// chunks of 8 tiles, one with a ninth, not 33 chunks on half of the GPU).
int tq3_join_min(int num_q, int num_kv, int sub_n) {
  return sub_n * (num_q / num_kv) > 16 ? 1 : 4;
}

FastGeom fast_geom(int num_q, int num_kv, int sub_n, int n_keys, int base = kChunkKeys,
                   int groups = 0, int join_min = 0) {
  FastGeom g{};
  const int cb = (n_keys + base - 1) / base;
  int tpw = (cb + 127) / 128;
  // chunks of base * t keys; from t = join_min on (0: never) a last chunk of
  // at most one 64-key tile joins the previous one (tq3_join_min)
  auto chunks_from = [&](int t, int jmin) {
    const long ck = (long)base * t;
    int n = (int)((n_keys + ck - 1) / ck);
    if (jmin > 0 && n > 1 && t >= jmin && n_keys - (n - 1) * ck <= 64) n--;
    return n;
  };
  // Long contexts and many queries: grow the chunks until the launch fits one
  // round of the GPU (kMaxFastWgs workgroups, one per CU), so that each
  // workgroup pays its setup and merge once for several tiles (config 4:
  // 189 -> 119 us per step; a 16-token verify over 131K keys: 148 -> 108 us).
  auto fit = [&](int jmin) {
    int t = tpw;
    while (groups > 0 && (long)groups * chunks_from(t, jmin) * num_kv > kMaxFastWgs && t < cb) t++;
    return t;
  };
  // A remainder of at most one tile also joins below join_min when leaving it
  // alone would take longer chunks (a decode step over 32,769 keys: 64 chunks
  // of 512 keys with one wave taking a second tile instead of 33 chunks of
  // 1,024 on half the CUs, 20.8 -> 17.9 us); otherwise an extra chunk is the
  // cheaper (4,097 keys: 9 chunks, 14.2 us, against 16.3 joined).
  if (join_min > 1 && groups > 0 && fit(1) < fit(join_min)) join_min = 1;
  auto chunks = [&](int t) { return chunks_from(t, join_min); };
  tpw = fit(join_min);
  g.chunk_keys = base * tpw;
  g.n_chunks = chunks(tpw);
  g.n_slots = g.n_chunks;
  const size_t rows = (size_t)num_q * sub_n * g.n_slots;
  g.header_off = 0;
  g.ml_off = qkv::kWsHeaderBytes;
  (void)num_kv;
  g.o_off = (g.ml_off + rows * qkv::kRecMlBytes + 255) & ~(size_t)255;
  g.total = g.o_off + rows * 256 * sizeof(float);
  return g;
}

// Workspace for every call over at most n_keys keys.  The record area is not
// monotone in the key count: a longer context takes longer chunks, hence fewer
// of them (16,384 Q8 keys: 128 chunks, 16,385: 65; a 16-query TQ3 verify over
// 32,768 keys: 16, over 32,833: 13), so the size for n_keys alone can be less
// than a shorter call needs.  The chunk count depends on the key count only
// through whole 64-key tiles (base, every chunk and the joined tail are whole
// tiles), so one evaluation per tile covers every count.
size_t fast_ws_upto(int num_q, int num_kv, int sub_n, int n_keys, int base, int groups,
                    int join_min) {
  size_t best = 0;
  for (long n = 64;; n += 64) {
    const int nk = (int)std::min<long>(n, n_keys);
    best = std::max(best, fast_geom(num_q, num_kv, sub_n, nk, base, groups, join_min).total);
    if (nk == n_keys) break;
  }
  return best;
}
}  // namespace

size_t qkv_decode_attn_tq3_workspace_bytes(int num_q, int num_kv, int sub_n, int n_keys) {
  if (num_q <= 0 || num_kv <= 0 || sub_n <= 0 || n_keys <= 0) return 0;
  return fast_ws_upto(num_q, num_kv, sub_n, n_keys, kChunkKeys, tq3_groups(num_q, num_kv, sub_n),
                      tq3_join_min(num_q, num_kv, sub_n));
}

// The TQ3 fast path with its workspace at `workspace` (caller-owned, or the
// allocation-free entry point's scratch when `noalloc`).
static int decode_tq3(const uint16_t* q, const qkv_block_tq3* k, const qkv_block_tq3* v,
                      uint16_t* out, int num_q, int num_kv, int head_dim, int start_pos, int sub_n,
                      float scale, int sink_tok, int window_tok, const uint32_t* tree_mask,
                      void* workspace, size_t workspace_bytes, bool noalloc, hipStream_t stream,
                      const uint16_t* k_new = nullptr, const uint16_t* v_new = nullptr) {
  int st = check_attn_shape(num_q, num_kv, head_dim, start_pos, sub_n, tree_mask);
  if (st) return st;
  if (sink_tok < 0 || window_tok < 0) return QKV_ERR_INVALID;
  if (!q || !k || !v || !out) return QKV_ERR_NULL;
  if (!aligned(q, 16) || !aligned(k, 4) || !aligned(v, 4) || !aligned(out, 16))
    return QKV_ERR_ALIGN;
  const int n_keys = start_pos + sub_n;
  const FastGeom g = fast_geom(num_q, num_kv, sub_n, n_keys, kChunkKeys, tq3_groups(num_q, num_kv, sub_n),
                               tq3_join_min(num_q, num_kv, sub_n));
  if (noalloc) {
    // no allocation: this device's scratch (looked up, and zero-filled on
    // `stream`, by the device's first qkv_tq3_init or first call here)
    if (g.total > qkv::kNoAllocScratchBytes) return QKV_ERR_WORKSPACE;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return QKV_ERR_DEVICE;
    if (qkv::noalloc_scratch(dev, false, stream, &workspace) != hipSuccess) return QKV_ERR_DEVICE;
    workspace_bytes = qkv::kNoAllocScratchBytes;
  }
  if (!workspace || workspace_bytes < g.total) return QKV_ERR_WORKSPACE;
  if (!aligned(workspace, 256)) return QKV_ERR_ALIGN;
  char* ws = static_cast<char*>(workspace);
  qkv::AttnArgs a{};
  a.q = q;
  a.k = reinterpret_cast<const uint32_t*>(k);
  a.v = reinterpret_cast<const uint32_t*>(v);
  a.num_q = num_q;
  a.num_kv = num_kv;
  a.start_pos = start_pos;
  a.sub_n = sub_n;
  a.sub_n_max = sub_n;
  a.qpw = tq3_fast_qpw(num_q, num_kv, sub_n);
  {
    const uint64_t extent = (uint64_t)n_keys * num_kv * 104;
    a.kv_bytes = extent;
  }
  a.active_end_max = n_keys;
  a.k_splits = 1;
  a.n_chunks = g.n_chunks;
  a.chunk_keys = g.chunk_keys;
  a.n_slots = g.n_slots;
  a.scale_log2 = scale * qkv::kLog2e;
  a.sink_tok = sink_tok;
  a.window_tok = window_tok;
  a.tree_mask = tree_mask;
  a.ws_header = reinterpret_cast<int*>(ws + g.header_off);
  a.spin_limit = g_spin_limit.load(std::memory_order_relaxed);
  a.ws_ml = reinterpret_cast<float*>(ws + g.ml_off);
  a.ws_o = reinterpret_cast<float*>(ws + g.o_off);
  if (g.total > 0xffffffffULL) return QKV_ERR_UNSUPPORTED;   // 32-bit buffer offsets
  a.ws_ml_bytes = (uint32_t)(g.o_off - g.ml_off);
  a.ws_o_bytes = (uint32_t)(g.total - g.o_off);
  if (k_new) {
    // the block's rows start_pos .. start_pos + sub_n - 1: encoded inside the
    // decode launch when it takes the shared-decode kernel (more than 16
    // query-head columns) and the block has at most 64 rows (the kernel's
    // encode area: a workgroup encodes the new rows it reads, at most
    // min(sub_n, 64)), or when it is one query (a decode step: the wave whose
    // tile holds the new key encodes it); else appended by their own launch
    const int cols = a.qpw * (num_q / num_kv);
    if ((cols > 16 && sub_n <= 64) || (sub_n == 1 && cols <= 8)) {
      a.k_new = k_new;
      a.v_new = v_new;
      a.k_w = reinterpret_cast<uint8_t*>(const_cast<qkv_block_tq3*>(k));
      a.v_w = reinterpret_cast<uint8_t*>(const_cast<qkv_block_tq3*>(v));
    } else {
      const long first = (long)start_pos * num_kv * 2;
      const hipError_t e = qkv::launch_tq3_append(k_new, const_cast<qkv_block_tq3*>(k) + first, v_new,
                                                  const_cast<qkv_block_tq3*>(v) + first, sub_n * num_kv * 2,
                                                  2, stream);
      if (e != hipSuccess) return launch_status(e);
    }
  }
  return launch_status(qkv::launch_tq3_attn(a, 0, out, stream));
}

int qkv_decode_attn_tq3(const uint16_t* q, const qkv_block_tq3* k, const qkv_block_tq3* v,
                        uint16_t* out, int num_q, int num_kv, int head_dim, int start_pos,
                        int sub_n, float scale, int sink_tok, int window_tok,
                        const uint32_t* tree_mask, void* workspace, size_t workspace_bytes,
                        hipStream_t stream) {
  return decode_tq3(q, k, v, out, num_q, num_kv, head_dim, start_pos, sub_n, scale, sink_tok,
                    window_tok, tree_mask, workspace, workspace_bytes, false, stream);
}

int qkv_decode_attn_tq3_append(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                               qkv_block_tq3* k, qkv_block_tq3* v, uint16_t* out, int num_q,
                               int num_kv, int head_dim, int start_pos, int sub_n, float scale,
                               int sink_tok, int window_tok, const uint32_t* tree_mask,
                               void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (!k_new || !v_new) return QKV_ERR_NULL;
  if (!aligned(k_new, 16) || !aligned(v_new, 16)) return QKV_ERR_ALIGN;
  return decode_tq3(q, k, v, out, num_q, num_kv, head_dim, start_pos, sub_n, scale, sink_tok,
                    window_tok, tree_mask, workspace, workspace_bytes, false, stream, k_new, v_new);
}

int qkv_decode_attn_tq3_noalloc(const uint16_t* q, const qkv_block_tq3* k,
                                const qkv_block_tq3* v, uint16_t* out, int num_q, int num_kv,
                                int head_dim, int start_pos, int sub_n, float scale, int sink_tok,
                                int window_tok, const uint32_t* tree_mask, hipStream_t stream) {
  return decode_tq3(q, k, v, out, num_q, num_kv, head_dim, start_pos, sub_n, scale, sink_tok,
                    window_tok, tree_mask, nullptr, 0, true, stream);
}

size_t qkv_decode_attn_q8_workspace_bytes(int num_q, int num_kv, int sub_n, int n_keys) {
  if (num_q <= 0 || num_kv <= 0 || sub_n <= 0 || n_keys <= 0) return 0;
  return fast_ws_upto(num_q, num_kv, sub_n, n_keys, kChunkKeysQ8, 0, 0);
}

// Fast path over Q8_0 keys; values Q8_0 (v_tq3 false) or TQ3 (v_tq3 true).
static int decode_q8_keys(const uint16_t* q, const void* k, const void* v, uint16_t* out,
                          int num_q, int num_kv, int head_dim, int start_pos, int sub_n,
                          float scale, void* workspace, size_t workspace_bytes, bool v_tq3,
                          hipStream_t stream, const uint16_t* k_new = nullptr,
                          const uint16_t* v_new = nullptr) {
  int st = check_attn_shape(num_q, num_kv, head_dim, start_pos, sub_n, nullptr);
  if (st) return st;
  if (!q || !k || !v || !out) return QKV_ERR_NULL;
  if (!aligned(q, 16) || !aligned(k, 4) || !aligned(v, 4) || !aligned(out, 16))
    return QKV_ERR_ALIGN;
  const int n_keys = start_pos + sub_n;
  const FastGeom g = fast_geom(num_q, num_kv, sub_n, n_keys, kChunkKeysQ8);
  if (!workspace || workspace_bytes < g.total) return QKV_ERR_WORKSPACE;
  if (!aligned(workspace, 256)) return QKV_ERR_ALIGN;
  char* ws = static_cast<char*>(workspace);
  qkv::AttnArgs a{};
  a.q = q;
  a.k = reinterpret_cast<const uint32_t*>(k);
  a.v = reinterpret_cast<const uint32_t*>(v);
  a.num_q = num_q;
  a.num_kv = num_kv;
  a.start_pos = start_pos;
  a.sub_n = sub_n;
  a.sub_n_max = sub_n;
  a.qpw = 1;
  {
    const uint64_t extent = (uint64_t)n_keys * num_kv * 8 * sizeof(qkv_block_q8);
    a.kv_bytes = extent;
    a.v_bytes = (uint64_t)n_keys * num_kv * 2 * sizeof(qkv_block_tq3);
  }
  a.active_end_max = n_keys;
  a.k_splits = 1;
  a.n_chunks = g.n_chunks;
  a.chunk_keys = g.chunk_keys;
  a.n_slots = g.n_slots;
  a.scale_log2 = scale * qkv::kLog2e;
  a.ws_header = reinterpret_cast<int*>(ws + g.header_off);
  a.spin_limit = g_spin_limit.load(std::memory_order_relaxed);
  a.ws_ml = reinterpret_cast<float*>(ws + g.ml_off);
  a.ws_o = reinterpret_cast<float*>(ws + g.o_off);
  if (g.total > 0xffffffffULL) return QKV_ERR_UNSUPPORTED;   // 32-bit buffer offsets
  a.ws_ml_bytes = (uint32_t)(g.o_off - g.ml_off);
  a.ws_o_bytes = (uint32_t)(g.total - g.o_off);
  if (k_new) {
    a.k_new = k_new;
    a.v_new = v_new;
    a.k_w = static_cast<uint8_t*>(const_cast<void*>(k));
    a.v_w = static_cast<uint8_t*>(const_cast<void*>(v));
    return launch_status(qkv::launch_q8_attn_fast_append(a, out, stream));
  }
  return launch_status(v_tq3 ? qkv::launch_q8k_tq3v_attn_fast(a, out, stream)
                             : qkv::launch_q8_attn_fast(a, out, stream));
}

int qkv_decode_attn_q8_append(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                              qkv_block_q8* k, qkv_block_q8* v, uint16_t* out, int num_q,
                              int num_kv, int head_dim, int start_pos, float scale,
                              void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (!k_new || !v_new) return QKV_ERR_NULL;
  if (!aligned(k_new, 16) || !aligned(v_new, 16)) return QKV_ERR_ALIGN;
  return decode_q8_keys(q, k, v, out, num_q, num_kv, head_dim, start_pos, 1, scale, workspace,
                        workspace_bytes, false, stream, k_new, v_new);
}

int qkv_decode_attn_q8(const uint16_t* q, const qkv_block_q8* k, const qkv_block_q8* v,
                       uint16_t* out, int num_q, int num_kv, int head_dim, int start_pos,
                       int sub_n, float scale, void* workspace, size_t workspace_bytes,
                       hipStream_t stream) {
  return decode_q8_keys(q, k, v, out, num_q, num_kv, head_dim, start_pos, sub_n, scale,
                        workspace, workspace_bytes, false, stream);
}

size_t qkv_decode_attn_q8k_tq3v_workspace_bytes(int num_q, int num_kv, int sub_n, int n_keys) {
  return qkv_decode_attn_q8_workspace_bytes(num_q, num_kv, sub_n, n_keys);
}

int qkv_decode_attn_q8k_tq3v(const uint16_t* q, const qkv_block_q8* k, const qkv_block_tq3* v,
                             uint16_t* out, int num_q, int num_kv, int head_dim, int start_pos,
                             int sub_n, float scale, void* workspace, size_t workspace_bytes,
                             hipStream_t stream) {
  return decode_q8_keys(q, k, v, out, num_q, num_kv, head_dim, start_pos, sub_n, scale,
                        workspace, workspace_bytes, true, stream);
}

size_t qkv_decode_attn_tq3_paged_workspace_bytes(int num_q, int num_kv, int n_slots,
                                                 int max_ctx) {
  if (num_q <= 0 || num_kv <= 0 || n_slots <= 0 || max_ctx <= 0) return 0;
  return fast_geom(num_q, num_kv, n_slots, max_ctx, kChunkKeys, n_slots).total;
}

int qkv_decode_attn_tq3_paged(const uint16_t* q, const qkv_block_tq3* k_pool,
                              const qkv_block_tq3* v_pool, uint16_t* out, int num_q, int num_kv,
                              int head_dim, int n_slots, const int32_t* block_tables,
                              int max_blocks, int block_tokens, int pool_rows,
                              const int32_t* ctx_lens, int max_ctx, float scale, void* workspace,
                              size_t workspace_bytes, hipStream_t stream) {
  int st = check_attn_shape(num_q, num_kv, head_dim, 0, 1, nullptr);
  if (st) return st;
  if (n_slots < 1 || max_ctx < 1 || max_blocks < 1 || pool_rows < 1) return QKV_ERR_INVALID;
  if (block_tokens < 64 || block_tokens % 64 != 0) return QKV_ERR_UNSUPPORTED;
  if ((long)max_blocks * block_tokens < max_ctx) return QKV_ERR_INVALID;
  if (!q || !k_pool || !v_pool || !out || !block_tables || !ctx_lens) return QKV_ERR_NULL;
  if (!aligned(q, 16) || !aligned(k_pool, 4) || !aligned(v_pool, 4) || !aligned(out, 16) ||
      !aligned(block_tables, 4) || !aligned(ctx_lens, 4))
    return QKV_ERR_ALIGN;
  const FastGeom g = fast_geom(num_q, num_kv, n_slots, max_ctx, kChunkKeys, n_slots);
  if (!workspace || workspace_bytes < g.total) return QKV_ERR_WORKSPACE;
  if (!aligned(workspace, 256)) return QKV_ERR_ALIGN;
  char* ws = static_cast<char*>(workspace);
  qkv::AttnArgs a{};
  a.q = q;
  a.k = reinterpret_cast<const uint32_t*>(k_pool);
  a.v = reinterpret_cast<const uint32_t*>(v_pool);
  a.num_q = num_q;
  a.num_kv = num_kv;
  a.start_pos = 0;
  a.sub_n = n_slots;
  a.sub_n_max = n_slots;
  a.qpw = 1;   // slots read different caches
  {
    const uint64_t extent = (uint64_t)pool_rows * num_kv * 104;
    a.kv_bytes = extent;
  }
  a.active_end_max = max_ctx;
  a.k_splits = 1;
  a.n_chunks = g.n_chunks;
  a.chunk_keys = g.chunk_keys;
  a.n_slots = g.n_slots;
  a.scale_log2 = scale * qkv::kLog2e;
  a.block_tables = block_tables;
  a.bt_stride = max_blocks;
  a.block_tokens = block_tokens;
  a.ctx_lens = ctx_lens;
  a.ctx_max = max_ctx;
  a.ws_header = reinterpret_cast<int*>(ws + g.header_off);
  a.spin_limit = g_spin_limit.load(std::memory_order_relaxed);
  a.ws_ml = reinterpret_cast<float*>(ws + g.ml_off);
  a.ws_o = reinterpret_cast<float*>(ws + g.o_off);
  if (g.total > 0xffffffffULL) return QKV_ERR_UNSUPPORTED;   // 32-bit buffer offsets
  a.ws_ml_bytes = (uint32_t)(g.o_off - g.ml_off);
  a.ws_o_bytes = (uint32_t)(g.total - g.o_off);
  return launch_status(qkv::launch_tq3_attn(a, 0, out, stream));
}

int qkv_decode_workspace_status(const void* workspace, hipStream_t stream) {
  if (!workspace) return QKV_ERR_NULL;
  if (!aligned(workspace, 256)) return QKV_ERR_ALIGN;
  if (hipStreamSynchronize(stream) != hipSuccess) return QKV_ERR_DEVICE;
  int word = 0;
  if (hipMemcpy(&word, static_cast<const char*>(workspace) + 4 * qkv::kWsErrorWord, sizeof(word),
                hipMemcpyDeviceToHost) != hipSuccess)
    return QKV_ERR_DEVICE;
  return word == 0 ? QKV_OK : QKV_ERR_TIMEOUT;
}

int qkv_decode_workspace_status_async(const void* workspace, int* status, hipStream_t stream) {
  if (!workspace || !status) return QKV_ERR_NULL;
  if (!aligned(workspace, 256) || !aligned(status, 4)) return QKV_ERR_ALIGN;
  return launch_status(qkv::launch_ws_status(workspace, status, QKV_OK, QKV_ERR_TIMEOUT, stream));
}

int qkv_decode_workspace_reset(void* workspace, size_t bytes, hipStream_t stream) {
  if (!workspace) return QKV_ERR_NULL;
  if (!aligned(workspace, 256) || bytes % 4) return QKV_ERR_ALIGN;
  if (bytes == 0) return QKV_OK;
  return launch_status(qkv::launch_fill_zero(workspace, bytes, stream));
}

// The allocation-free scratch of `device` (made current for the lookup; the
// caller's device is restored): looked up, and zero-filled on `stream` when
// `clear` or on the device's first use.
static int noalloc_scratch_on(int device, bool clear, hipStream_t stream, void** ptr) {
  if (device < 0 || device >= 64) return QKV_ERR_INVALID;
  int n = 0, cur = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || device >= n) return QKV_ERR_DEVICE;
  if (hipGetDevice(&cur) != hipSuccess) return QKV_ERR_DEVICE;
  if (hipSetDevice(device) != hipSuccess) return QKV_ERR_DEVICE;
  const bool ok = qkv::noalloc_scratch(device, clear, stream, ptr) == hipSuccess;
  if (hipSetDevice(cur) != hipSuccess || !ok) return QKV_ERR_DEVICE;
  return QKV_OK;
}

int qkv_decode_noalloc_status(int device, hipStream_t stream) {
  void* ptr = nullptr;
  const int st = noalloc_scratch_on(device, false, stream, &ptr);
  if (st) return st;
  return qkv_decode_workspace_status(ptr, stream);
}

int qkv_decode_noalloc_status_async(int device, int* status, hipStream_t stream) {
  if (!status) return QKV_ERR_NULL;
  if (!aligned(status, 4)) return QKV_ERR_ALIGN;
  void* ptr = nullptr;
  const int st = noalloc_scratch_on(device, false, stream, &ptr);
  if (st) return st;
  // launched with `device` current (the stream is one of its streams)
  int cur = 0;
  if (hipGetDevice(&cur) != hipSuccess || hipSetDevice(device) != hipSuccess) return QKV_ERR_DEVICE;
  const int rc = launch_status(qkv::launch_ws_status(ptr, status, QKV_OK, QKV_ERR_TIMEOUT, stream));
  if (hipSetDevice(cur) != hipSuccess) return QKV_ERR_DEVICE;
  return rc;
}

int qkv_decode_noalloc_reset(int device, hipStream_t stream) {
  void* ptr = nullptr;
  return noalloc_scratch_on(device, true, stream, &ptr);
}

int qkv_debug_set_merge_spin_limit(int limit) {
  g_spin_limit.store(limit < 0 ? qkv::kMergeSpinLimit : limit, std::memory_order_relaxed);
  return QKV_OK;
}

size_t qkv_prefill_attn_tq3_workspace_bytes(int num_q, int num_kv, int n_tok, int start_pos) {
  if (num_q <= 0 || num_kv <= 0 || n_tok <= 0 || start_pos < 0) return 0;
  return qkv::prefill_geom(num_q, num_kv, n_tok, start_pos).total;
}

int qkv_prefill_attn_tq3(const uint16_t* q, const qkv_block_tq3* k_cache,
                         const qkv_block_tq3* v_cache, const uint16_t* k_chunk,
                         const uint16_t* v_chunk, uint16_t* out, int num_q, int num_kv,
                         int head_dim, int start_pos, int n_tok, float scale, void* workspace,
                         size_t workspace_bytes, hipStream_t stream) {
  if (head_dim != 256) return QKV_ERR_UNSUPPORTED;
  if (num_kv <= 0 || num_q <= 0 || num_q % num_kv != 0 || n_tok < 1 || start_pos < 0)
    return QKV_ERR_INVALID;
  const int gqa = num_q / num_kv;
  if (gqa != 4 && gqa != 6) return QKV_ERR_UNSUPPORTED;
  if (!q || !out) return QKV_ERR_NULL;
  if ((k_chunk == nullptr) != (v_chunk == nullptr)) return QKV_ERR_NULL;
  const bool from_cache = k_chunk == nullptr;   // verify: the chunk's rows are in the cache
  if ((start_pos > 0 || from_cache) && (!k_cache || !v_cache)) return QKV_ERR_NULL;
  if (!aligned(q, 16) || !aligned(k_chunk, 16) || !aligned(v_chunk, 16) || !aligned(out, 16) ||
      !aligned(k_cache, 8) || !aligned(v_cache, 8))
    return QKV_ERR_ALIGN;
  const qkv::PrefillGeom g = qkv::prefill_geom(num_q, num_kv, n_tok, start_pos);
  if (!workspace || workspace_bytes < g.total) return QKV_ERR_WORKSPACE;
  if (!aligned(workspace, 256)) return QKV_ERR_ALIGN;
  const uint64_t qbytes = (uint64_t)n_tok * num_q * 256 * 2;
  if (qbytes > 0x7fffffffULL) return QKV_ERR_UNSUPPORTED;   // 32-bit query offsets
  if ((int64_t)start_pos + n_tok > (int64_t)INT32_MAX - 128) return QKV_ERR_INVALID;
  char* ws = static_cast<char*>(workspace);
  qkv::PrefillArgs a{};
  a.k_cache = reinterpret_cast<const uint32_t*>(k_cache);
  a.v_cache = reinterpret_cast<const uint32_t*>(v_cache);
  a.kx = reinterpret_cast<uint16_t*>(ws + g.kx_off);
  a.vt = reinterpret_cast<uint16_t*>(ws + g.vt_off);
  a.part_ml = reinterpret_cast<float*>(ws + g.ml_off);
  a.part_o = reinterpret_cast<float*>(ws + g.o_off);
  a.num_q = num_q;
  a.num_kv = num_kv;
  a.start_pos = start_pos;
  a.n_tok = n_tok;
  a.hist = from_cache ? start_pos + n_tok : start_pos;
  a.h_pad = (a.hist + 63) / 64 * 64;
  a.n_pad = from_cache ? 0 : g.n_pad;   // no chunk rows to stage
  a.n_split = g.n_split;
  a.from_cache = from_cache ? 1 : 0;
  a.scale_log2 = scale * qkv::kLog2e;
  return launch_status(qkv::launch_prefill_tq3(a, gqa, q, k_chunk, v_chunk, out, stream));
}

}  // extern "C"
