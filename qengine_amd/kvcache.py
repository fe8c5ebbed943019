"""Host-side API over libqkv.so for torch device tensors.

Mirrors the reference's append and attention launches (src/model.cuh call
sites) with torch tensors as the device-memory container.  Every function
calls the gfx950 HIP kernels through the C ABI; there is no CPU path.

Cache tensors are uint8 tensors whose last dimension is the block size
(52 bytes per TQ3 block, 36 bytes per Q8 block); fp16 tensors are
torch.float16.  Calls are ordered on the current torch stream.
"""
from __future__ import annotations

import torch

from ._lib import bench_lib, check, lib

TQ3_BLOCK_BYTES = 52
Q8_BLOCK_BYTES = 36


def _stream(stream=None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


# fp16 arguments: torch.float16, or 16-bit integer tensors holding fp16 bit
# patterns (the C ABI takes uint16_t)
FP16 = (torch.float16, torch.uint16, torch.int16)


def _need(t, nbytes: int, what: str, dtype=None) -> None:
    """Raise ValueError (before any launch) when `t` is not of `dtype` or
    holds fewer than `nbytes` bytes: the kernels trust the sizes implied by
    the shape arguments, so an undersized buffer would be read or written
    out of bounds on the device."""
    if t is None:
        raise ValueError(f"{what} is required")
    allowed = dtype if isinstance(dtype, tuple) else (dtype,)
    if dtype is not None and t.dtype not in allowed:
        raise ValueError(f"{what} must be {' or '.join(str(d) for d in allowed)}, got {t.dtype}")
    have = t.numel() * t.element_size()
    if have < nbytes:
        raise ValueError(f"{what} holds {have} bytes, the call needs {int(nbytes)}")


def _dev_ptr(t: torch.Tensor, what: str) -> int:
    if not t.is_cuda:
        raise ValueError(f"{what} must be a device tensor")
    if not t.is_contiguous():
        raise ValueError(f"{what} must be contiguous")
    return t.data_ptr()


def tq3_blocks(n_blocks: int, device) -> torch.Tensor:
    """Zero-initialised TQ3 block storage [n_blocks, 52] (model.cuh:1914-1920)."""
    return torch.zeros((n_blocks, TQ3_BLOCK_BYTES), dtype=torch.uint8, device=device)


def q8_blocks(n_blocks: int, device) -> torch.Tensor:
    return torch.zeros((n_blocks, Q8_BLOCK_BYTES), dtype=torch.uint8, device=device)


def tq3_init(device: int = 0) -> None:
    check(lib().qkv_tq3_init(device), "qkv_tq3_init")


def tq3_append(x: torch.Tensor, out: torch.Tensor, stream=None) -> None:
    """turboquant.cuh:112-165.  x: fp16 [..., 128*k]; out: uint8 blocks [n, 52]."""
    assert x.dtype == torch.float16
    n = x.numel() // 128
    assert x.numel() == n * 128 and out.numel() >= n * TQ3_BLOCK_BYTES
    check(lib().qkv_tq3_append(_dev_ptr(x, "x"), _dev_ptr(out, "out"), n, _stream(stream)),
          "qkv_tq3_append")


def tq3_append_kv(k: torch.Tensor, v: torch.Tensor, k_out: torch.Tensor, v_out: torch.Tensor,
                  stream=None) -> None:
    assert k.dtype == torch.float16 and v.dtype == torch.float16 and k.numel() == v.numel()
    n = k.numel() // 128
    check(lib().qkv_tq3_append_kv(_dev_ptr(k, "k"), _dev_ptr(v, "v"), _dev_ptr(k_out, "k_out"),
                                  _dev_ptr(v_out, "v_out"), n, _stream(stream)),
          "qkv_tq3_append_kv")


def tq3_dequant(blocks: torch.Tensor, out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """turboquant.cuh:169-200.  Returns fp16 [n_blocks*128]."""
    n = blocks.numel() // TQ3_BLOCK_BYTES
    if out is None:
        out = torch.empty(n * 128, dtype=torch.float16, device=blocks.device)
    check(lib().qkv_tq3_dequant(_dev_ptr(blocks, "blocks"), _dev_ptr(out, "out"), n,
                                _stream(stream)), "qkv_tq3_dequant")
    return out


def q8_append(x: torch.Tensor, out: torch.Tensor, stream=None) -> None:
    """attention.cuh:2587-2609.  x: fp16 [..., 32*k]; out: uint8 blocks [n, 36]."""
    assert x.dtype == torch.float16
    n = x.numel() // 32
    assert x.numel() == n * 32 and out.numel() >= n * Q8_BLOCK_BYTES
    check(lib().qkv_q8_append(_dev_ptr(x, "x"), _dev_ptr(out, "out"), n, _stream(stream)),
          "qkv_q8_append")


def q8_append_kv(k: torch.Tensor, v: torch.Tensor, k_out: torch.Tensor, v_out: torch.Tensor,
                 stream=None) -> None:
    """K and V in one launch (the two quantize_kv_q8_0_kern launches of
    model.cuh:2316-2333)."""
    assert k.dtype == torch.float16 and v.dtype == torch.float16 and k.numel() == v.numel()
    n = k.numel() // 32
    assert k.numel() == n * 32
    assert k_out.numel() >= n * Q8_BLOCK_BYTES and v_out.numel() >= n * Q8_BLOCK_BYTES
    check(lib().qkv_q8_append_kv(_dev_ptr(k, "k"), _dev_ptr(v, "v"), _dev_ptr(k_out, "k_out"),
                                 _dev_ptr(v_out, "v_out"), n, _stream(stream)),
          "qkv_q8_append_kv")


def q8_dequant(blocks: torch.Tensor, out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """attention.cuh:2614-2626."""
    n = blocks.numel() // Q8_BLOCK_BYTES
    if out is None:
        out = torch.empty(n * 32, dtype=torch.float16, device=blocks.device)
    check(lib().qkv_q8_dequant(_dev_ptr(blocks, "blocks"), _dev_ptr(out, "out"), n,
                               _stream(stream)), "qkv_q8_dequant")
    return out


def kv_move_tokens(k: torch.Tensor, v: torch.Tensor, moves, *, k_row_bytes: int,
                   v_row_bytes: int, slot_row0: int = 0, slot_rows: int | None = None,
                   stream=None) -> None:
    """kv_move_token (model.cuh:7430-7471) for a list of (from_pos, to_pos)
    moves of one layer, applied in list order, in one launch."""
    import ctypes
    moves = list(moves)
    if slot_rows is None:
        slot_rows = k.numel() // k_row_bytes - slot_row0
    flat = (ctypes.c_int32 * max(1, 2 * len(moves)))(*[int(x) for m in moves for x in m])
    check(lib().qkv_kv_move_tokens(_dev_ptr(k, "k"), _dev_ptr(v, "v"), k_row_bytes, v_row_bytes,
                                   slot_row0, slot_rows, ctypes.cast(flat, ctypes.c_void_p),
                                   len(moves), _stream(stream)), "qkv_kv_move_tokens")


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------

def _pool_rows(k_pool, v_pool, k_row_bytes, v_row_bytes):
    rows = k_pool.numel() * k_pool.element_size() // k_row_bytes
    if v_pool is not None:
        rows = min(rows, v_pool.numel() * v_pool.element_size() // v_row_bytes)
    return rows


def _flat_sizes(k_flat, v_flat, v_pool, n_rows, k_row_bytes, v_row_bytes, block_table,
                block_tokens) -> None:
    """The flat buffers hold n_rows rows and the table covers them."""
    _need(k_flat, n_rows * k_row_bytes, "k_flat")
    if v_pool is not None or v_flat is not None:
        _need(v_flat, n_rows * v_row_bytes, "v_flat")
    if block_tokens > 0:
        _need(block_table, -(-n_rows // block_tokens) * 4, "block_table", torch.int32)


def kv_gather_rows(k_pool, v_pool, k_flat, v_flat, block_table, *, n_rows, block_tokens,
                   k_row_bytes, v_row_bytes=0, stream=None) -> None:
    """Slot snapshot over a paged pool: logical rows 0 .. n_rows-1 of the slot
    whose block-table row is `block_table` (int32 device tensor) into the flat
    buffers [n_rows][row_bytes] (model.cuh:3394-3417 for the contiguous
    layout).  v_pool / v_flat may be None (keys only)."""
    _flat_sizes(k_flat, v_flat, v_pool, n_rows, k_row_bytes, v_row_bytes, block_table, block_tokens)
    pool_rows = _pool_rows(k_pool, v_pool, k_row_bytes, v_row_bytes)
    check(lib().qkv_kv_gather_rows(
        _dev_ptr(k_pool, "k_pool"), _opt_ptr(v_pool), _dev_ptr(k_flat, "k_flat"),
        _opt_ptr(v_flat), k_row_bytes, v_row_bytes, pool_rows,
        _i32(block_table, "block_table"), block_table.numel(),
        block_tokens, n_rows, _stream(stream)), "qkv_kv_gather_rows")


def kv_scatter_rows(k_pool, v_pool, k_flat, v_flat, block_table, *, n_rows, block_tokens,
                    k_row_bytes, v_row_bytes=0, stream=None) -> None:
    """Slot restore over a paged pool: the inverse of kv_gather_rows
    (model.cuh:3314-3335 for the contiguous layout)."""
    _flat_sizes(k_flat, v_flat, v_pool, n_rows, k_row_bytes, v_row_bytes, block_table, block_tokens)
    pool_rows = _pool_rows(k_pool, v_pool, k_row_bytes, v_row_bytes)
    check(lib().qkv_kv_scatter_rows(
        _dev_ptr(k_pool, "k_pool"), _opt_ptr(v_pool), _dev_ptr(k_flat, "k_flat"),
        _opt_ptr(v_flat), k_row_bytes, v_row_bytes, pool_rows,
        _i32(block_table, "block_table"), block_table.numel(),
        block_tokens, n_rows, _stream(stream)), "qkv_kv_scatter_rows")


def dfk2_dequant(q, scales, out, *, kv_dim, stream=None) -> None:
    """dfki2_dequant_kernel (model.cuh:149-159): int8 plane rows with
    group-128 fp16 scales to fp16."""
    check(lib().qkv_dfk2_dequant(_dev_ptr(q, "q"), _dev_ptr(scales, "scales"),
                                 _dev_ptr(out, "out"), q.numel(), kv_dim, _stream(stream)),
          "qkv_dfk2_dequant")


def tq3_append_dfk2(q, scales, out, stream=None) -> None:
    """KV-inject re-quantization into TQ3 (model.cuh:3189-3192 + 3218-3226 in
    one launch): block i from q[128 i ..] with scale scales[i]."""
    check(lib().qkv_tq3_append_dfk2(_dev_ptr(q, "q"), _dev_ptr(scales, "scales"),
                                    _dev_ptr(out, "out"), q.numel() // 128, _stream(stream)),
          "qkv_tq3_append_dfk2")


def q8_append_dfk2(q, scales, out, stream=None) -> None:
    """KV-inject re-quantization into Q8_0 (model.cuh:3189-3192 + 3227-3233):
    32-element block i with scale scales[i // 4]."""
    check(lib().qkv_q8_append_dfk2(_dev_ptr(q, "q"), _dev_ptr(scales, "scales"),
                                   _dev_ptr(out, "out"), q.numel() // 32, _stream(stream)),
          "qkv_q8_append_dfk2")


def hbm_read_bench(buf, sink, stream=None) -> None:
    """One streaming read of the whole tensor `buf` (bandwidth measurement;
    libqkv_bench.so, not the product library)."""
    check(bench_lib().qkv_hbm_read_bench(_dev_ptr(buf, "buf"), buf.numel() * buf.element_size(),
                                   _dev_ptr(sink, "sink"), _stream(stream)), "qkv_hbm_read_bench")


def mfma_rate_bench(workgroups, iters, sink, stream=None) -> None:
    """One launch of the MFMA-rate loop (workgroups x 8 waves x 16 * iters
    32x32x16 fp16 MFMAs on data-like operands; libqkv_bench.so)."""
    check(bench_lib().qkv_mfma_rate_bench(int(workgroups), int(iters), _dev_ptr(sink, "sink"),
                                          _stream(stream)), "qkv_mfma_rate_bench")


def _opt_ptr(t):
    return 0 if t is None else _dev_ptr(t, "tensor")


def attn_split_tq3(q, k, v, part_m, part_l, part_o, *, num_q, num_kv, start_pos, sub_n,
                   sub_n_max, active_end_max, scale, k_splits, sink_tok=0, window_tok=0,
                   tree_mask=None, head_dim=256, stream=None) -> None:
    """attention.cuh:1905-2177: unnormalised split partials, reference layout."""
    check(lib().qkv_attn_split_tq3(
        _dev_ptr(q, "q"), _dev_ptr(k, "k"), _dev_ptr(v, "v"), _dev_ptr(part_m, "part_m"),
        _dev_ptr(part_l, "part_l"), _dev_ptr(part_o, "part_o"), num_q, num_kv, head_dim,
        start_pos, sub_n, sub_n_max, active_end_max, float(scale), k_splits, sink_tok,
        window_tok, _opt_ptr(tree_mask), _stream(stream)), "qkv_attn_split_tq3")


def attn_split_q8(q, k, v, part_m, part_l, part_o, *, num_q, num_kv, start_pos, sub_n,
                  sub_n_max, active_end_max, scale, k_splits, head_dim=256, stream=None) -> None:
    """attention.cuh:2633-2801: unnormalised split partials over the Q8_0 cache."""
    check(lib().qkv_attn_split_q8(
        _dev_ptr(q, "q"), _dev_ptr(k, "k"), _dev_ptr(v, "v"), _dev_ptr(part_m, "part_m"),
        _dev_ptr(part_l, "part_l"), _dev_ptr(part_o, "part_o"), num_q, num_kv, head_dim,
        start_pos, sub_n, sub_n_max, active_end_max, float(scale), k_splits, _stream(stream)),
        "qkv_attn_split_q8")


def attn_split_merge(part_m, part_l, part_o, out, *, num_q, num_kv, sub_n, sub_n_max, k_splits,
                     head_dim=256, stream=None) -> None:
    """attention.cuh:1837-1891."""
    check(lib().qkv_attn_split_merge(
        _dev_ptr(part_m, "part_m"), _dev_ptr(part_l, "part_l"), _dev_ptr(part_o, "part_o"),
        _dev_ptr(out, "out"), num_q, num_kv, head_dim, sub_n, sub_n_max, k_splits,
        _stream(stream)), "qkv_attn_split_merge")


def tq3_kpool_update(k_cache, k_pool, k_pool_max, *, num_kv, total_kv, blk_lo, block_size_n=64,
                     head_dim=256, stream=None) -> None:
    """Block signatures of the TQ3 keys (attention.cuh:2445-2533): pools are
    fp16 tensors [num_kv][n_blocks_stride][256]; blocks blk_lo ..
    ceil(total_kv / block_size_n) - 1 are rebuilt."""
    check(lib().qkv_tq3_kpool_update(
        _dev_ptr(k_cache, "k_cache"), _dev_ptr(k_pool, "k_pool"), _dev_ptr(k_pool_max, "k_pool_max"),
        num_kv, head_dim, total_kv, blk_lo, k_pool.shape[1], block_size_n, _stream(stream)),
        "qkv_tq3_kpool_update")


def block_index_ms(q, k_pool, k_pool_max, block_index, *, num_q, num_kv, sub_n, start_pos,
                   top_k, n_blocks, block_size_n=64, beta=0.5, head_dim=256, workspace=None,
                   stream=None) -> None:
    """Top-k block selection (sparse_attn/sparse_index.cuh:214-330) into the
    int32 tensor block_index [num_kv][sub_n_max][top_k]; the block scores pass
    through `workspace` (allocated here when None)."""
    if workspace is None:
        n = int(lib().qkv_block_index_ms_workspace_bytes(num_kv, sub_n, n_blocks))
        workspace = torch.empty(max(n, 256), dtype=torch.uint8, device=block_index.device)
    check(lib().qkv_block_index_ms(
        _dev_ptr(q, "q"), _dev_ptr(k_pool, "k_pool"), _dev_ptr(k_pool_max, "k_pool_max"),
        _i32(block_index, "block_index"), num_q, num_kv, head_dim, sub_n, block_index.shape[1],
        start_pos, top_k, block_size_n, n_blocks, k_pool.shape[1], float(beta),
        _dev_ptr(workspace, "workspace"), workspace.numel() * workspace.element_size(),
        _stream(stream)), "qkv_block_index_ms")


def attn_block_sparse_split_tq3(q, k, v, block_index, part_m, part_l, part_o, *, num_q, num_kv,
                                start_pos, sub_n, sub_n_max, scale, top_k, k_splits,
                                block_size_n=64, tree_mask=None, head_dim=256,
                                stream=None) -> None:
    """attention.cuh:2193-2433: split partials over each query's selected blocks."""
    check(lib().qkv_attn_block_sparse_split_tq3(
        _dev_ptr(q, "q"), _dev_ptr(k, "k"), _dev_ptr(v, "v"), _i32(block_index, "block_index"),
        _dev_ptr(part_m, "part_m"), _dev_ptr(part_l, "part_l"), _dev_ptr(part_o, "part_o"),
        num_q, num_kv, head_dim, start_pos, sub_n, sub_n_max, float(scale), top_k, block_size_n,
        k_splits, _opt_ptr(tree_mask), _stream(stream)), "qkv_attn_block_sparse_split_tq3")


# bytes per token row and kv head of one cache (head_dim 256): TQ3 two 52-byte
# blocks, Q8_0 eight 36-byte blocks
TQ3_ROW = 2 * TQ3_BLOCK_BYTES
Q8_ROW = 8 * Q8_BLOCK_BYTES


def _attn_sizes(q, k, v, out, num_q, num_kv, n_keys, sub_n, head_dim, k_row, v_row) -> None:
    """q / out hold sub_n x num_q fp16 rows; k / v hold n_keys token rows."""
    _need(q, sub_n * num_q * head_dim * 2, "q", FP16)
    _need(out, sub_n * num_q * head_dim * 2, "out", FP16)
    _need(k, n_keys * num_kv * k_row, "k")
    _need(v, n_keys * num_kv * v_row, "v")


def decode_attn_tq3_workspace_bytes(num_q, num_kv, sub_n, n_keys) -> int:
    return int(lib().qkv_decode_attn_tq3_workspace_bytes(num_q, num_kv, sub_n, n_keys))


def decode_attn_tq3_workspace(num_q, num_kv, sub_n, n_keys, device) -> torch.Tensor:
    """Zero-filled workspace for decode_attn_tq3 (the kernel keeps it zeroed)."""
    n = decode_attn_tq3_workspace_bytes(num_q, num_kv, sub_n, n_keys)
    return torch.zeros(n, dtype=torch.uint8, device=device)


def decode_attn_tq3(q, k, v, out, workspace, *, num_q, num_kv, start_pos, sub_n, scale,
                    sink_tok=0, window_tok=0, tree_mask=None, head_dim=256, stream=None) -> None:
    """Fast path: split-K decode with the merge inside the same launch."""
    _attn_sizes(q, k, v, out, num_q, num_kv, start_pos + sub_n, sub_n, head_dim, TQ3_ROW, TQ3_ROW)
    check(lib().qkv_decode_attn_tq3(
        _dev_ptr(q, "q"), _dev_ptr(k, "k"), _dev_ptr(v, "v"), _dev_ptr(out, "out"), num_q,
        num_kv, head_dim, start_pos, sub_n, float(scale), sink_tok, window_tok,
        _opt_ptr(tree_mask), _dev_ptr(workspace, "workspace"),
        workspace.numel() * workspace.element_size(), _stream(stream)), "qkv_decode_attn_tq3")


def decode_attn_tq3_append(q, k_new, v_new, k, v, out, workspace, *, num_q, num_kv, start_pos,
                           sub_n, scale, sink_tok=0, window_tok=0, tree_mask=None, head_dim=256,
                           stream=None) -> None:
    """decode_attn_tq3 of a block of sub_n new tokens whose K / V rows (fp16
    [sub_n][num_kv][256]) are appended in the same call: encoded into rows
    start_pos .. start_pos + sub_n - 1 of k / v (one launch when the call has
    more than 16 query-head columns).  k and v must hold those rows."""
    _attn_sizes(q, k, v, out, num_q, num_kv, start_pos + sub_n, sub_n, head_dim, TQ3_ROW, TQ3_ROW)
    _need(k_new, sub_n * num_kv * head_dim * 2, "k_new", FP16)
    _need(v_new, sub_n * num_kv * head_dim * 2, "v_new", FP16)
    check(lib().qkv_decode_attn_tq3_append(
        _dev_ptr(q, "q"), _dev_ptr(k_new, "k_new"), _dev_ptr(v_new, "v_new"), _dev_ptr(k, "k"),
        _dev_ptr(v, "v"), _dev_ptr(out, "out"), num_q, num_kv, head_dim, start_pos, sub_n,
        float(scale), sink_tok, window_tok, _opt_ptr(tree_mask), _dev_ptr(workspace, "workspace"),
        workspace.numel() * workspace.element_size(), _stream(stream)), "qkv_decode_attn_tq3_append")


def decode_attn_tq3_noalloc(q, k, v, out, *, num_q, num_kv, start_pos, sub_n, scale,
                            sink_tok=0, window_tok=0, tree_mask=None, head_dim=256,
                            stream=None) -> None:
    """decode_attn_tq3 without a workspace argument: the library's fixed
    per-GPU scratch serves as the workspace (no allocation in the call)."""
    _attn_sizes(q, k, v, out, num_q, num_kv, start_pos + sub_n, sub_n, head_dim, TQ3_ROW, TQ3_ROW)
    check(lib().qkv_decode_attn_tq3_noalloc(
        _dev_ptr(q, "q"), _dev_ptr(k, "k"), _dev_ptr(v, "v"), _dev_ptr(out, "out"), num_q,
        num_kv, head_dim, start_pos, sub_n, float(scale), sink_tok, window_tok,
        _opt_ptr(tree_mask), _stream(stream)), "qkv_decode_attn_tq3_noalloc")


def decode_attn_q8_workspace(num_q, num_kv, sub_n, n_keys, device) -> torch.Tensor:
    """Zero-filled workspace for decode_attn_q8."""
    n = int(lib().qkv_decode_attn_q8_workspace_bytes(num_q, num_kv, sub_n, n_keys))
    return torch.zeros(n, dtype=torch.uint8, device=device)


def decode_attn_q8(q, k, v, out, workspace, *, num_q, num_kv, start_pos, sub_n, scale,
                   head_dim=256, stream=None) -> None:
    """Fast path over the Q8_0 cache: split-K decode with the merge inside the
    same launch."""
    _attn_sizes(q, k, v, out, num_q, num_kv, start_pos + sub_n, sub_n, head_dim, Q8_ROW, Q8_ROW)
    check(lib().qkv_decode_attn_q8(
        _dev_ptr(q, "q"), _dev_ptr(k, "k"), _dev_ptr(v, "v"), _dev_ptr(out, "out"), num_q,
        num_kv, head_dim, start_pos, sub_n, float(scale), _dev_ptr(workspace, "workspace"),
        workspace.numel() * workspace.element_size(), _stream(stream)), "qkv_decode_attn_q8")


def decode_attn_q8_append(q, k_new, v_new, k, v, out, workspace, *, num_q, num_kv, start_pos,
                          scale, head_dim=256, stream=None) -> None:
    """One launch for a decode step over the Q8_0 cache: k_new / v_new (fp16
    [num_kv][256]) are quantized into row start_pos of k / v and attended as
    key start_pos by the one query q (keys 0..start_pos).  k and v must hold
    row start_pos (the kernel writes it)."""
    _attn_sizes(q, k, v, out, num_q, num_kv, start_pos + 1, 1, head_dim, Q8_ROW, Q8_ROW)
    _need(k_new, num_kv * head_dim * 2, "k_new", FP16)
    _need(v_new, num_kv * head_dim * 2, "v_new", FP16)
    check(lib().qkv_decode_attn_q8_append(
        _dev_ptr(q, "q"), _dev_ptr(k_new, "k_new"), _dev_ptr(v_new, "v_new"), _dev_ptr(k, "k"),
        _dev_ptr(v, "v"), _dev_ptr(out, "out"), num_q, num_kv, head_dim, start_pos, float(scale),
        _dev_ptr(workspace, "workspace"), workspace.numel() * workspace.element_size(),
        _stream(stream)), "qkv_decode_attn_q8_append")


def decode_attn_q8k_tq3v_workspace(num_q, num_kv, sub_n, n_keys, device) -> torch.Tensor:
    """Zero-filled workspace for decode_attn_q8k_tq3v."""
    n = int(lib().qkv_decode_attn_q8k_tq3v_workspace_bytes(num_q, num_kv, sub_n, n_keys))
    return torch.zeros(n, dtype=torch.uint8, device=device)


def decode_attn_q8k_tq3v(q, k, v, out, workspace, *, num_q, num_kv, start_pos, sub_n, scale,
                         head_dim=256, stream=None) -> None:
    """V-only TurboQuant (reference TQ_KEYS_Q8 mode): keys in Q8_0 blocks, values
    in TQ3 blocks; one fused decode launch with the merge inside it."""
    _attn_sizes(q, k, v, out, num_q, num_kv, start_pos + sub_n, sub_n, head_dim, Q8_ROW, TQ3_ROW)
    check(lib().qkv_decode_attn_q8k_tq3v(
        _dev_ptr(q, "q"), _dev_ptr(k, "k"), _dev_ptr(v, "v"), _dev_ptr(out, "out"), num_q,
        num_kv, head_dim, start_pos, sub_n, float(scale), _dev_ptr(workspace, "workspace"),
        workspace.numel() * workspace.element_size(), _stream(stream)), "qkv_decode_attn_q8k_tq3v")


def decode_workspace_status(workspace, stream=None) -> int:
    """Synchronises the stream and returns QKV_OK (0) or QKV_ERR_TIMEOUT (-8): an
    in-kernel merge on this workspace ran out of polls and its rows were NaN."""
    return int(lib().qkv_decode_workspace_status(_dev_ptr(workspace, "workspace"),
                                                 _stream(stream)))


def decode_workspace_status_async(workspace, status, stream=None) -> None:
    """Enqueue the health check without synchronising: once the stream gets
    there, status[0] (an int32 device tensor) holds QKV_OK (0) or
    QKV_ERR_TIMEOUT (-8).  Capturable in a HIP graph."""
    _need(status, 4, "status", dtype=(torch.int32,))
    check(lib().qkv_decode_workspace_status_async(_dev_ptr(workspace, "workspace"),
                                                  _dev_ptr(status, "status"), _stream(stream)),
          "qkv_decode_workspace_status_async")


def decode_workspace_reset(workspace, stream=None) -> None:
    """Zero-fill a fast-path decode workspace (clears a sticky merge error)."""
    check(lib().qkv_decode_workspace_reset(_dev_ptr(workspace, "workspace"),
                                           workspace.numel() * workspace.element_size(),
                                           _stream(stream)), "qkv_decode_workspace_reset")


def decode_noalloc_status(device: int = 0, stream=None) -> int:
    """decode_workspace_status for the allocation-free decode's scratch of
    `device`: synchronises the stream, returns QKV_OK (0) or QKV_ERR_TIMEOUT (-8)."""
    return int(lib().qkv_decode_noalloc_status(int(device), _stream(stream)))


def decode_noalloc_status_async(status, device: int = 0, stream=None) -> None:
    """decode_workspace_status_async for the allocation-free decode's scratch
    of `device`."""
    _need(status, 4, "status", dtype=(torch.int32,))
    check(lib().qkv_decode_noalloc_status_async(int(device), _dev_ptr(status, "status"),
                                                _stream(stream)), "qkv_decode_noalloc_status_async")


def decode_noalloc_reset(device: int = 0, stream=None) -> None:
    """Zero-fill the allocation-free decode's scratch of `device` (clears a
    sticky merge error)."""
    check(lib().qkv_decode_noalloc_reset(int(device), _stream(stream)), "qkv_decode_noalloc_reset")


def debug_set_merge_spin_limit(limit: int) -> None:
    """Test hook: merger poll limit of later fast-path launches (negative = default)."""
    check(lib().qkv_debug_set_merge_spin_limit(int(limit)), "qkv_debug_set_merge_spin_limit")


# ---------------------------------------------------------------------------
# paged caches (per-slot int32 block tables)
# ---------------------------------------------------------------------------

def _i32(t, what):
    if t.dtype != torch.int32:
        raise ValueError(f"{what} must be int32")
    return _dev_ptr(t, what)


def tq3_append_kv_paged(k, v, k_pool, v_pool, block_tables, positions, *, block_tokens,
                        head_dim=256, stream=None) -> None:
    """Paged append: k, v fp16 [n_slots][n_tok][num_kv][256]; token t of slot s
    goes to position positions[s] + t through block_tables [n_slots][max_blocks]."""
    assert k.dtype == torch.float16 and v.dtype == torch.float16 and k.shape == v.shape
    n_slots, n_tok, num_kv = k.shape[0], k.shape[1], k.shape[2]
    pool_rows = k_pool.numel() // (TQ3_BLOCK_BYTES * num_kv * head_dim // 128)
    check(lib().qkv_tq3_append_kv_paged(
        _dev_ptr(k, "k"), _dev_ptr(v, "v"), _dev_ptr(k_pool, "k_pool"), _dev_ptr(v_pool, "v_pool"),
        n_slots, n_tok, num_kv, head_dim, _i32(block_tables, "block_tables"),
        block_tables.shape[1], block_tokens, pool_rows, _i32(positions, "positions"),
        _stream(stream)), "qkv_tq3_append_kv_paged")


def decode_attn_tq3_paged_workspace(num_q, num_kv, n_slots, max_ctx, device) -> torch.Tensor:
    n = int(lib().qkv_decode_attn_tq3_paged_workspace_bytes(num_q, num_kv, n_slots, max_ctx))
    return torch.zeros(n, dtype=torch.uint8, device=device)


def decode_attn_tq3_paged(q, k_pool, v_pool, out, workspace, block_tables, ctx_lens, *, num_q,
                          num_kv, max_ctx, block_tokens, scale, head_dim=256,
                          stream=None) -> None:
    """One decode query per slot over per-slot block tables (ragged contexts)."""
    pool_rows = k_pool.numel() // (TQ3_BLOCK_BYTES * num_kv * head_dim // 128)
    check(lib().qkv_decode_attn_tq3_paged(
        _dev_ptr(q, "q"), _dev_ptr(k_pool, "k_pool"), _dev_ptr(v_pool, "v_pool"),
        _dev_ptr(out, "out"), num_q, num_kv, head_dim, q.shape[0],
        _i32(block_tables, "block_tables"), block_tables.shape[1], block_tokens, pool_rows,
        _i32(ctx_lens, "ctx_lens"), max_ctx, float(scale), _dev_ptr(workspace, "workspace"),
        workspace.numel() * workspace.element_size(), _stream(stream)),
        "qkv_decode_attn_tq3_paged")


# ---------------------------------------------------------------------------
# chunked prefill over the TQ3 cache
# ---------------------------------------------------------------------------

def prefill_attn_tq3_workspace(num_q, num_kv, n_tok, start_pos, device) -> torch.Tensor:
    n = int(lib().qkv_prefill_attn_tq3_workspace_bytes(num_q, num_kv, n_tok, start_pos))
    return torch.empty(n, dtype=torch.uint8, device=device)


def prefill_attn_tq3(q, k_cache, v_cache, k_chunk, v_chunk, out, workspace, *, num_q, num_kv,
                     start_pos, scale, head_dim=256, stream=None) -> None:
    """Causal attention of a chunk (q [n_tok][num_q][256]) over the cache
    history rows 0..start_pos-1 (TQ3) and the chunk's own fp16 k/v; with
    k_chunk = v_chunk = None (verify) every key comes from the cache rows
    0..start_pos+n_tok-1."""
    n_tok = q.shape[0]
    from_cache = k_chunk is None
    kc = _dev_ptr(k_cache, "k_cache") if (start_pos > 0 or from_cache) else 0
    vc = _dev_ptr(v_cache, "v_cache") if (start_pos > 0 or from_cache) else 0
    check(lib().qkv_prefill_attn_tq3(
        _dev_ptr(q, "q"), kc, vc, _opt_ptr(k_chunk), _opt_ptr(v_chunk),
        _dev_ptr(out, "out"), num_q, num_kv, head_dim, start_pos, n_tok, float(scale),
        _dev_ptr(workspace, "workspace"), workspace.numel() * workspace.element_size(),
        _stream(stream)), "qkv_prefill_attn_tq3")
