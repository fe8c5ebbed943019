#!/usr/bin/env python3
"""Benchmark of the compressed KV-cache hot path on one MI355X.

Workload: 3-bit TQ3 KV split-K flash decode, 8 attention
layers, 32768-token context, 16 query heads / 4 kv heads, head_dim 256.
Each layer's cache is built on the GPU by the append kernel from seeded
N(0,1) fp16 K/V with 2% outlier channels (x8).  Three independent 8-layer
cache sets (654 MB) are rotated so the 256 MB Infinity Cache cannot serve
them.  A step = one decode token: decode attention over all 8 layers.

Prints one JSON line (value = microseconds per token, lower is better) with:
  roofline      HBM roofline of the attention kernel: algorithmic bytes per
                launch / its average duration (HIP events on the launch stream
                around the timed region, which holds only these launches),
                against 8 TB/s; traffic = HBM bytes per launch from rocprofv3
                counters (profiles/traffic.json); launch_read_floor = one
                launch of a plain read kernel over the same bytes (back to
                back, rotating buffers), the single-launch floor on this box
  step_stats    per-step median / p10 / p90 over the timed steps (an event
                pair around every step)
  hbm_read_peak measured streaming-read bandwidth (qkv_hbm_read_bench over a
                1 GiB buffer); every fraction is also given against it
  append        TQ3 append (K+V) throughput of the cache build
  append_q8     Q8_0 append (K+V) throughput over the same inputs
  config1       (CPU leg) the CPU-plumbing config: TQ3 roundtrip MSE, code
                histogram, codes checked against the oracle, and the elements
                within one fp32 ulp of a decision boundary
  cpu_baseline  the CPU oracle (C port of the reference arithmetic, OpenMP) on
                bounded samples, at all usable cores and at one thread: one
                decode token over the 8 layers (the reported value) and the
                TQ3 encode of one layer's K and V
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = ("3-bit KV decode-attn µs/token + HBM GB/s (% peak) at 32K ctx; "
          "append Mtok/s")
HBM_PEAK_GBS = 8000.0
NUM_Q, NUM_KV, HD, CTX, LAYERS, SETS = 16, 4, 256, 32768, 8, 3
BLOCKS_PER_TOKEN = NUM_KV * HD // 128              # 8 TQ3 blocks per token for K (and V)
# algorithmic bytes per layer and query token: K+V blocks + Q + O
ATTN_BYTES = CTX * 2 * BLOCKS_PER_TOKEN * 52 + NUM_Q * HD * 2 * 2
APPEND_BYTES_PER_TOKEN = 2 * NUM_KV * HD * 2 + 2 * BLOCKS_PER_TOKEN * 52   # 4928
Q8_BLOCKS_PER_TOKEN = NUM_KV * HD // 32                                      # 32 Q8_0 blocks (K or V)
APPEND_Q8_BYTES_PER_TOKEN = 2 * NUM_KV * HD * 2 + 2 * Q8_BLOCKS_PER_TOKEN * 36   # 6400
CPU_REPS = 5
APPEND_REPS = 5


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the configs 2, 4 and 5 measurements")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 256 MiB device copy (reference for HBM byte counters)")
    return ap.parse_args()


def outlier_kv(torch, gen, n_tok, dev):
    """fp16 [n_tok][NUM_KV][HD] ~ N(0,1) with round(0.02*HD)=5 fixed channels
    per head scaled x8 (the same channels for every token)."""
    x = torch.randn(n_tok, NUM_KV, HD, generator=gen, device=dev)
    n_out = round(0.02 * HD)
    for h in range(NUM_KV):
        ch = torch.randperm(HD, generator=gen, device=dev)[:n_out]
        x[:, h, ch] *= 8.0
    return x.to(torch.float16)


def _time(torch, stream, fn, reps):
    """Mean ms of fn() over reps calls, events on the launch stream."""
    fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for i in range(reps):
        fn(i)
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


def secondary(torch, kvcache, dev, stream):
    """BASELINE configs 2, 4 and 5 on synthetic inputs of their stated shapes
    (seeded N(0,1) fp16, encoded on the GPU).  Rates use algorithmic bytes
    (packed cache read + q/o) or FLOPs as stated per entry."""
    import numpy as np
    out = {}
    gen = torch.Generator(device=dev).manual_seed(7)
    rnd = lambda *shape: torch.randn(*shape, generator=gen, device=dev).to(torch.float16)
    scale = 1.0 / 16

    # ---- config 2: Q8_0 cache of 4096 tokens, append 1 token, split decode +
    # merge (reference K_SPLITS 8, sub_n_max 16); 8 layers x 4 sets rotated ----
    ctx, layers, sets = 4096, 8, 4
    blocks_tok = NUM_KV * HD // 32
    caches = []
    for _ in range(sets * layers):
        kb = kvcache.q8_blocks((ctx + 1) * blocks_tok, dev)
        vb = kvcache.q8_blocks((ctx + 1) * blocks_tok, dev)
        kvcache.q8_append(rnd(ctx, NUM_KV, HD), kb[: ctx * blocks_tok])
        kvcache.q8_append(rnd(ctx, NUM_KV, HD), vb[: ctx * blocks_tok])
        caches.append((kb, vb))
    knew, vnew, q = rnd(1, NUM_KV, HD), rnd(1, NUM_KV, HD), rnd(1, NUM_Q, HD)
    pm = torch.empty(NUM_Q, 16, 8, device=dev)
    pl = torch.empty(NUM_Q, 16, 8, device=dev)
    po = torch.empty(NUM_Q, 16, 8, HD, device=dev)
    o = torch.empty(1, NUM_Q, HD, dtype=torch.float16, device=dev)

    def q8_layer_split(i=0):
        kb, vb = caches[i % len(caches)]
        kvcache.q8_append(knew, kb[ctx * blocks_tok:])
        kvcache.q8_append(vnew, vb[ctx * blocks_tok:])
        kvcache.attn_split_q8(q, kb, vb, pm, pl, po, num_q=NUM_Q, num_kv=NUM_KV, start_pos=ctx,
                              sub_n=1, sub_n_max=16, active_end_max=ctx + 1, scale=scale,
                              k_splits=8)
        kvcache.attn_split_merge(pm, pl, po, o, num_q=NUM_Q, num_kv=NUM_KV, sub_n=1,
                                 sub_n_max=16, k_splits=8)
    ws8 = kvcache.decode_attn_q8_workspace(NUM_Q, NUM_KV, 1, ctx + 1, dev)

    def q8_layer(i=0):
        kb, vb = caches[i % len(caches)]
        kvcache.q8_append_kv(knew, vnew, kb[ctx * blocks_tok:], vb[ctx * blocks_tok:])
        kvcache.decode_attn_q8(q, kb, vb, o, ws8, num_q=NUM_Q, num_kv=NUM_KV, start_pos=ctx,
                               sub_n=1, scale=scale)
    ms_split = _time(torch, stream, q8_layer_split, 200)
    ms_eager = _time(torch, stream, q8_layer, 200)
    # the same layers launched from HIP graphs (one graph per cache set: 8
    # layers x 2 launches), replayed back to back: two kernels of ~2 and ~13 us
    # per layer are launch-bound when each call also pays the Python host path
    graphs = []
    for s_ in range(sets):
        for l_ in range(layers):
            q8_layer(s_ * layers + l_)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for l_ in range(layers):
                q8_layer(s_ * layers + l_)
        graphs.append(gr)
    ms = _time(torch, stream, lambda i=0: graphs[i % sets].replay(), 50) / layers
    del graphs

    # the same step as one fused launch per layer (append inside the decode)
    def q8_layer_fused(i=0):
        kb, vb = caches[i % len(caches)]
        kvcache.decode_attn_q8_append(q, knew, vnew, kb, vb, o, ws8, num_q=NUM_Q, num_kv=NUM_KV,
                                      start_pos=ctx, scale=scale)
    graphs = []
    for s_ in range(sets):
        for l_ in range(layers):
            q8_layer_fused(s_ * layers + l_)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for l_ in range(layers):
                q8_layer_fused(s_ * layers + l_)
        graphs.append(gr)
    ms_fused = _time(torch, stream, lambda i=0: graphs[i % sets].replay(), 50) / layers
    del graphs
    q8_bytes = 2 * (ctx + 1) * blocks_tok * 36 + NUM_Q * HD * 2 * 2
    out["config2_q8_decode"] = {
        "us_per_layer": round(ms * 1e3, 3),
        "bytes_per_layer": q8_bytes, "gbps": round(q8_bytes / (ms * 1e-3) / 1e9, 1),
        "frac": round(q8_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "eager_us_per_layer": round(ms_eager * 1e3, 3),
        "split_api_us_per_layer": round(ms_split * 1e3, 3),
        "fused_us_per_layer": round(ms_fused * 1e3, 3),
        "fused_frac": round(q8_bytes / (ms_fused * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "note": "fused_us_per_layer: the same step through qkv_decode_attn_q8_append (the "
                "append inside the decode launch: 1 launch per layer), HIP graphs as above; "
                "per layer: Q8 append of the new token's K and V and single-launch decode over "
                "4097 keys (2 launches), launched from HIP graphs (8 layers per graph, 4 cache "
                "sets); eager_us_per_layer: the same calls launched one by one from Python; "
                "split_api_us_per_layer: the same through the reference "
                "split layout (2 appends, split-K decode K_SPLITS 8, merge: 4 launches); 8 layers "
                "x 4 cache sets rotated"}
    del caches

    # ---- config 4: 8 slots, 24 q / 4 kv heads, 256-token blocks, ctx ~ U[1K, 64K],
    # slots 0-3 share a 4096-token prefix; a step appends 1 token per slot
    # (paged) and decodes all 8 slots; two pools rotated ----
    rng = np.random.default_rng(4)
    n_slots, nq4, bt_tok = 8, 24, 256
    ctx_s = rng.integers(1024, 65537, size=n_slots)
    ctx_s[:4] = np.maximum(ctx_s[:4], 4096 + 1)
    new_s = ctx_s + 1
    max_ctx = int(new_s.max())
    max_blocks = (max_ctx + bt_tok - 1) // bt_tok
    shared = 4096 // bt_tok
    tables = np.zeros((n_slots, max_blocks), np.int32)
    nxt = shared
    for s_ in range(n_slots):
        nb = (int(new_s[s_]) + bt_tok - 1) // bt_tok
        for b in range(nb):
            if s_ < 4 and b < shared:
                tables[s_, b] = b
            else:
                tables[s_, b] = nxt
                nxt += 1
    pool_rows = nxt * bt_tok
    pools = []
    for _ in range(2):
        kp = kvcache.tq3_blocks(pool_rows * 8, dev)
        vp = kvcache.tq3_blocks(pool_rows * 8, dev)
        for r0 in range(0, pool_rows, 65536):
            n = min(65536, pool_rows - r0)
            kvcache.tq3_append_kv(rnd(n, NUM_KV, HD), rnd(n, NUM_KV, HD),
                                  kp[r0 * 8:(r0 + n) * 8], vp[r0 * 8:(r0 + n) * 8])
        pools.append((kp, vp))
    bt_d = torch.from_numpy(tables).to(dev)
    pos_d = torch.from_numpy(ctx_s.astype(np.int32)).to(dev)
    len_d = torch.from_numpy(new_s.astype(np.int32)).to(dev)
    k4, v4, q4 = rnd(n_slots, 1, NUM_KV, HD), rnd(n_slots, 1, NUM_KV, HD), rnd(n_slots, nq4, HD)
    o4 = torch.empty(n_slots, nq4, HD, dtype=torch.float16, device=dev)
    ws4 = kvcache.decode_attn_tq3_paged_workspace(nq4, NUM_KV, n_slots, max_ctx, dev)

    def step4(i=0):
        kp, vp = pools[i % 2]
        kvcache.tq3_append_kv_paged(k4, v4, kp, vp, bt_d, pos_d, block_tokens=bt_tok)
        kvcache.decode_attn_tq3_paged(q4, kp, vp, o4, ws4, bt_d, len_d, num_q=nq4, num_kv=NUM_KV,
                                      max_ctx=max_ctx, block_tokens=bt_tok, scale=scale)
    ms = _time(torch, stream, step4, 100)
    logical = int(new_s.sum()) * 2 * BLOCKS_PER_TOKEN * 52 + n_slots * nq4 * HD * 2 * 2
    physical = logical - 3 * 4096 * 2 * BLOCKS_PER_TOKEN * 52
    out["config4_paged_step"] = {
        "us_per_step": round(ms * 1e3, 3), "ctx": [int(c) for c in new_s],
        "bytes_logical": logical, "bytes_physical": physical,
        "gbps_logical": round(logical / (ms * 1e-3) / 1e9, 1),
        "frac_logical": round(logical / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "note": "one layer: paged append of 1 token per slot + paged decode of 8 slots "
                "(2 launches); physical bytes count the shared prefix once"}
    del pools

    # ---- config 3's decode step with its append: one layer, the new token's K
    # and V encoded into row 32768, then the query over keys 0..32768 ----
    ctx3 = 32768
    k3 = kvcache.tq3_blocks((ctx3 + 1) * BLOCKS_PER_TOKEN, dev)
    v3 = kvcache.tq3_blocks((ctx3 + 1) * BLOCKS_PER_TOKEN, dev)
    kvcache.tq3_append_kv(rnd(ctx3, NUM_KV, HD), rnd(ctx3, NUM_KV, HD), k3[: ctx3 * BLOCKS_PER_TOKEN],
                          v3[: ctx3 * BLOCKS_PER_TOKEN])
    kn3, vn3, q3 = rnd(1, NUM_KV, HD), rnd(1, NUM_KV, HD), rnd(1, NUM_Q, HD)
    o3 = torch.empty(1, NUM_Q, HD, dtype=torch.float16, device=dev)
    ws3 = kvcache.decode_attn_tq3_workspace(NUM_Q, NUM_KV, 1, ctx3 + 1, dev)

    def step_two_calls(i=0):
        kvcache.tq3_append_kv(kn3, vn3, k3[ctx3 * BLOCKS_PER_TOKEN:], v3[ctx3 * BLOCKS_PER_TOKEN:])
        kvcache.decode_attn_tq3(q3, k3, v3, o3, ws3, num_q=NUM_Q, num_kv=NUM_KV, start_pos=ctx3,
                                sub_n=1, scale=scale)

    def step_one_call(i=0):
        kvcache.decode_attn_tq3_append(q3, kn3, vn3, k3, v3, o3, ws3, num_q=NUM_Q, num_kv=NUM_KV,
                                       start_pos=ctx3, sub_n=1, scale=scale)
    ms_two3 = _time(torch, stream, step_two_calls, 200)
    ms_one3 = _time(torch, stream, step_one_call, 200)
    out["config3_decode_step"] = {
        "one_call_us": round(ms_one3 * 1e3, 3), "two_call_us": round(ms_two3 * 1e3, 3),
        "note": "one layer of a decode step at 32K context: the new token's K and V appended "
                "(row 32768) and the query attended over keys 0..32768, called one by one from "
                "Python; one_call_us: qkv_decode_attn_tq3_append (one launch: the wave whose "
                "tile holds the new key encodes it); two_call_us: qkv_tq3_append_kv, then "
                "qkv_decode_attn_tq3"}
    del k3, v3

    # ---- config 5: one slot, 16 q / 4 kv, 131072-token history ----
    hist, chunk = 131072, 2048
    kb = kvcache.tq3_blocks((hist + chunk) * 8, dev)
    vb = kvcache.tq3_blocks((hist + chunk) * 8, dev)
    for r0 in range(0, hist, 65536):
        kvcache.tq3_append_kv(rnd(65536, NUM_KV, HD), rnd(65536, NUM_KV, HD),
                              kb[r0 * 8:(r0 + 65536) * 8], vb[r0 * 8:(r0 + 65536) * 8])
    qc, kc, vc = rnd(chunk, NUM_Q, HD), rnd(chunk, NUM_KV, HD), rnd(chunk, NUM_KV, HD)
    oc = torch.empty(chunk, NUM_Q, HD, dtype=torch.float16, device=dev)
    wsp = kvcache.prefill_attn_tq3_workspace(NUM_Q, NUM_KV, chunk, hist, dev)

    def prefill(i=0):
        kvcache.tq3_append_kv(kc, vc, kb[hist * 8:], vb[hist * 8:])
        kvcache.prefill_attn_tq3(qc, kb, vb, kc, vc, oc, wsp, num_q=NUM_Q, num_kv=NUM_KV,
                                 start_pos=hist, scale=scale)
    ms = _time(torch, stream, prefill, 5)
    flop = sum(4 * NUM_Q * HD * (hist + t + 1) for t in range(chunk))
    mfma_pf = mfma_sustained(torch, kvcache, dev, stream)
    out["config5_prefill_chunk"] = {
        "ms_per_chunk": round(ms, 3), "tflops": round(flop / (ms * 1e-3) / 1e12, 1),
        "frac_mfma_fp16": round(flop / (ms * 1e-3) / 1e12 / 2500.0, 4),
        "mfma_sustained_pflops": round(mfma_pf, 3),
        "frac_of_sustained_mfma": round(flop / (ms * 1e-3) / 1e15 / mfma_pf, 4),
        "note": "append of the 2048-token chunk + causal attention of the chunk over 131072 "
                "history keys (TQ3) and its own 2048 fp16 keys; FLOPs 4*num_q*hd per "
                "(query, visible key); mfma_sustained_pflops: qkv_mfma_rate_bench, a register-only "
                "loop of the same MFMA on random fp16 operands (the rate the part sustains on "
                "data-like operands; 2.5 PFLOP/s nominal)"}

    nv = 16
    qv, kv_, vv = rnd(nv, NUM_Q, HD), rnd(nv, NUM_KV, HD), rnd(nv, NUM_KV, HD)
    ov = torch.empty(nv, NUM_Q, HD, dtype=torch.float16, device=dev)
    wsv = kvcache.decode_attn_tq3_workspace(NUM_Q, NUM_KV, nv, hist + nv, dev)
    wsp16 = kvcache.prefill_attn_tq3_workspace(NUM_Q, NUM_KV, nv, hist, dev)

    def append16():
        kvcache.tq3_append_kv(kv_, vv, kb[hist * 8:(hist + nv) * 8], vb[hist * 8:(hist + nv) * 8])

    def verify(i=0):
        append16()
        kvcache.decode_attn_tq3(qv, kb, vb, ov, wsv, num_q=NUM_Q, num_kv=NUM_KV, start_pos=hist,
                                sub_n=nv, scale=scale)

    def verify_prefill_path(i=0):
        append16()
        kvcache.prefill_attn_tq3(qv, kb, vb, None, None, ov, wsp16, num_q=NUM_Q, num_kv=NUM_KV,
                                 start_pos=hist, scale=scale)
    def verify_one_call(i=0):
        kvcache.decode_attn_tq3_append(qv, kv_, vv, kb, vb, ov, wsv, num_q=NUM_Q, num_kv=NUM_KV,
                                       start_pos=hist, sub_n=nv, scale=scale)
    ms_two = _time(torch, stream, verify, 50)
    ms = _time(torch, stream, verify_one_call, 50)
    ms_pf = _time(torch, stream, verify_prefill_path, 50)
    vbytes = (hist + nv) * 2 * BLOCKS_PER_TOKEN * 52 + nv * NUM_Q * HD * 2 * 2
    out["config5_verify16"] = {
        "us": round(ms * 1e3, 3), "bytes": vbytes,
        "gbps": round(vbytes / (ms * 1e-3) / 1e9, 1),
        "frac": round(vbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "two_call_us": round(ms_two * 1e3, 3),
        "prefill_path_us": round(ms_pf * 1e3, 3),
        "note": "append of the 16 verify tokens, then causal attention of the 16 queries over "
                "the TQ3 cache (131088 keys, the block's own keys read back quantized), in one "
                "call and one launch: qkv_decode_attn_tq3_append, whose decode kernel encodes "
                "the block's rows itself, writes them to the caches and decodes every tile once "
                "for all 64 query-head columns (caches and output bit-identical to the two "
                "calls); two_call_us: qkv_tq3_append_kv, then qkv_decode_attn_tq3 with sub_n 16; "
                "prefill_path_us: the same step through qkv_prefill_attn_tq3 in verify mode"}

    # ---- f2: block-sparse verify of the same 16 queries (DFLASH_VERIFY_BLOCKSPARSE
    # defaults: top_k = 10% of the blocks capped at 64, beta 0.5, K_SPLITS 8) ----
    n_all = hist + nv
    nb = (n_all + 63) // 64
    kp = torch.zeros((NUM_KV, nb + 64, HD), dtype=torch.float16, device=dev)
    kx = torch.zeros_like(kp)
    kvcache.tq3_kpool_update(kb, kp, kx, num_kv=NUM_KV, total_kv=hist, blk_lo=0)
    top_k = min(64, max(1, int(nb * 0.10)))
    bi = torch.zeros((NUM_KV, nv, top_k), dtype=torch.int32, device=dev)
    spm = torch.empty(NUM_Q, nv, 8, device=dev)
    spl = torch.empty(NUM_Q, nv, 8, device=dev)
    spo = torch.empty(NUM_Q, nv, 8, HD, device=dev)
    wsb = kvcache.lib().qkv_block_index_ms_workspace_bytes(NUM_KV, nv, nb)
    wsi = torch.empty(wsb, dtype=torch.uint8, device=dev)

    def sparse_verify(i=0):
        append16()
        kvcache.tq3_kpool_update(kb, kp, kx, num_kv=NUM_KV, total_kv=n_all,
                                 blk_lo=(hist - 1) // 64)
        kvcache.block_index_ms(qv, kp, kx, bi, num_q=NUM_Q, num_kv=NUM_KV, sub_n=nv,
                               start_pos=hist, top_k=top_k, n_blocks=nb, workspace=wsi)
        kvcache.attn_block_sparse_split_tq3(qv, kb, vb, bi, spm, spl, spo, num_q=NUM_Q,
                                            num_kv=NUM_KV, start_pos=hist, sub_n=nv, sub_n_max=nv,
                                            scale=scale, top_k=top_k, k_splits=8)
        kvcache.attn_split_merge(spm, spl, spo, ov, num_q=NUM_Q, num_kv=NUM_KV, sub_n=nv,
                                 sub_n_max=nv, k_splits=8)
    ms = _time(torch, stream, sparse_verify, 50)
    out["f2_sparse_verify16"] = {
        "us": round(ms * 1e3, 3), "top_k": top_k, "n_blocks": nb,
        "note": "append of the 16 verify tokens, incremental key-block signatures (the last "
                "two 64-row blocks), top-k block index (10% of 2049 blocks -> 64), block-sparse "
                "split attention (K_SPLITS 8) and merge: 5 launches over the 131088-key TQ3 "
                "cache of config 5"}
    del kp, kx

    # ---- V-only TurboQuant (keys Q8_0, values TQ3): one query over 32768 keys
    # of config 3's head shape; 8 layers x 2 cache sets rotated ----
    ctx, n_caches = 32768, 16
    caches = []
    for _ in range(n_caches):
        kb = kvcache.q8_blocks(ctx * NUM_KV * HD // 32, dev)
        vb = kvcache.tq3_blocks(ctx * NUM_KV * HD // 128, dev)
        kvcache.q8_append(rnd(ctx, NUM_KV, HD), kb)
        kvcache.tq3_append(rnd(ctx, NUM_KV, HD), vb)
        caches.append((kb, vb))
    q = rnd(1, NUM_Q, HD)
    o = torch.empty(1, NUM_Q, HD, dtype=torch.float16, device=dev)
    wsm = kvcache.decode_attn_q8k_tq3v_workspace(NUM_Q, NUM_KV, 1, ctx, dev)

    def mixed_layer(i=0):
        kb, vb = caches[i % n_caches]
        kvcache.decode_attn_q8k_tq3v(q, kb, vb, o, wsm, num_q=NUM_Q, num_kv=NUM_KV,
                                     start_pos=ctx - 1, sub_n=1, scale=scale)
    ms = _time(torch, stream, mixed_layer, 320)
    mbytes = ctx * NUM_KV * (8 * 36 + 2 * 52) + NUM_Q * HD * 2 * 2   # Q8_0 keys, TQ3 values
    out["f4_mixed_decode_32k"] = {
        "us_per_launch": round(ms * 1e3, 3), "bytes": mbytes,
        "gbps": round(mbytes / (ms * 1e-3) / 1e9, 1),
        "frac": round(mbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "note": "qkv_decode_attn_q8k_tq3v: one query (16 q / 4 kv heads, d 256) over 32768 keys, "
                "keys Q8_0 (288 B per kv head and token), values TQ3 (104 B); 16 caches rotated"}
    del caches
    return out


def mfma_sustained(torch, kvcache, dev, stream):
    """Sustained fp16 MFMA rate on data-like operands: qkv_mfma_rate_bench,
    256 workgroups x 8 waves x 16 * 8000 v_mfma_f32_32x32x16_f16 per wave
    (a few ms per launch), 1 warm-up + 3 timed launches."""
    sink = torch.zeros(1, dtype=torch.float32, device=dev)
    wgs, iters = 256, 8000
    kvcache.mfma_rate_bench(wgs, iters, sink)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record(stream)
    for _ in range(3):
        kvcache.mfma_rate_bench(wgs, iters, sink)
    b.record(stream)
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / 3
    return wgs * 8 * 16 * iters * 32768.0 / (ms * 1e-3) / 1e15


def hbm_read_peak(torch, kvcache, dev, stream):
    """Sustained streaming-read bandwidth: qkv_hbm_read_bench over a 1 GiB
    buffer (4x the Infinity Cache), 2 warm-up + 10 timed reads."""
    buf = torch.ones(1 << 30, dtype=torch.uint8, device=dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    for _ in range(2):
        kvcache.hbm_read_bench(buf, sink)
    reps = 10
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record(stream)
    for _ in range(reps):
        kvcache.hbm_read_bench(buf, sink)
    b.record(stream)
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / reps
    gbps = buf.numel() / (ms * 1e-3) / 1e9
    del buf
    return {"gbps": round(gbps, 1), "frac_of_nominal": round(gbps / HBM_PEAK_GBS, 4),
            "bytes": 1 << 30, "kernel": "stream_read_kernel (qkv_hbm_read_bench)"}


def launch_read_floor(torch, kvcache, dev, stream, nbytes):
    """Per-launch time of a kernel that only reads `nbytes` (qkv_hbm_read_bench)
    once per launch: 16 launches over 16 buffers (more than the Infinity Cache
    holds) captured in a HIP graph, so that host submission does not pace
    them, and the graph replayed back to back: what one launch that streams a
    decode layer's bytes costs on this device, launch included."""
    nbytes = (nbytes + 63) // 64 * 64
    bufs = [torch.ones(nbytes, dtype=torch.uint8, device=dev) for _ in range(16)]
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    for b in bufs:
        kvcache.hbm_read_bench(b, sink)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for b in bufs:
            kvcache.hbm_read_bench(b, sink)
    for _ in range(3):
        graph.replay()
    reps = 20
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record(stream)
    for _ in range(reps):
        graph.replay()
    b.record(stream)
    torch.cuda.synchronize()
    us = a.elapsed_time(b) / (reps * len(bufs)) * 1e3
    del graph, bufs
    return {"us_per_launch": round(us, 3), "bytes": nbytes,
            "gbps": round(nbytes / (us * 1e-6) / 1e9, 1),
            "kernel": "stream_read_short_kernel (qkv_hbm_read_bench), 16 buffers, HIP graph replay"}


def config1_report(torch, kvcache, dev):
    """BASELINE config 1 (seed 0): K and V [1024][4][256] fp16 ~ N(0,1) with 5
    fixed x8 outlier channels per head, TQ3-encoded on the GPU (append) and
    decoded (dequant).  Reports the roundtrip MSE, the relative MSE, the
    8-bin code histogram, whether the codes equal the oracle's, and how many
    elements sit within one fp32 ulp of a decision boundary (where the
    reference's rsqrtf(128) / contraction could move a code)."""
    import numpy as np
    from oracle import oracle as O
    rng = np.random.default_rng(0)
    planes = []
    for _ in range(2):
        x = rng.standard_normal((1024, NUM_KV, HD)).astype(np.float32)
        for h in range(NUM_KV):
            x[:, h, rng.choice(HD, 5, replace=False)] *= 8.0
        planes.append(x.astype(np.float16))
    codes_all, sq, ref_sq, equal, near, n_el = [], 0.0, 0.0, True, 0, 0
    bounds = O.tq3_bounds().astype(np.float32)
    for x in planes:
        n = x.size // 128
        blocks = kvcache.tq3_blocks(n, dev)
        kvcache.tq3_append(torch.from_numpy(x.reshape(-1)).to(dev), blocks)
        dec = kvcache.tq3_dequant(blocks).float().cpu().numpy().reshape(-1)
        got = blocks.cpu().numpy().view(O.BLOCK_TQ3).reshape(-1)
        exp, rot = O.tq3_encode_rotated(x)
        equal = equal and bool(np.array_equal(got.view(np.uint8), exp.view(np.uint8)))
        xf = x.astype(np.float64).reshape(-1)
        sq += float(((dec - xf) ** 2).sum())
        ref_sq += float((xf ** 2).sum())
        n_el += xf.size
        qs = got["qs"].reshape(n, 16, 3).astype(np.uint32)
        w = qs[..., 0] | (qs[..., 1] << 8) | (qs[..., 2] << 16)
        codes_all.append(((w[..., None] >> (3 * np.arange(8))) & 7).reshape(-1))
        lo = np.nextafter(rot, np.float32(-np.inf))
        hi = np.nextafter(rot, np.float32(np.inf))
        near += int(((lo[..., None] <= bounds) & (bounds <= hi[..., None])).any(-1).sum())
    hist = np.bincount(np.concatenate(codes_all), minlength=8)
    return {"elements": n_el, "mse": sq / n_el, "rel_mse": sq / ref_sq,
            "code_hist": [int(c) for c in hist],
            "code_frac": [round(float(c) / hist.sum(), 4) for c in hist],
            "codes_equal_oracle": equal, "near_boundary_1ulp": near,
            "literal_wht256_fp16_scale": config1_literal(planes),
            "note": "K and V of config 1 (2 x 8192 blocks of 128), GPU append + dequant; "
                    "near_boundary_1ulp: rotated values whose one-ulp neighbourhood holds a "
                    "decision bound (oracle rotation)"}


def config1_literal(planes):
    """Config 1's wording taken literally, on the same K and V: one 256-point
    orthonormal WHT per head vector (random signs: the TQ3 128-entry sign
    vector repeated), the 8 Lloyd-Max levels for coordinates of a unit vector
    in 256 dimensions (the TQ3 levels, which are for 128, times sqrt(1/2)),
    one fp16 scale (the vector's norm) per 256-element block.  No reference
    kernel uses this format (the reference packs two 128-blocks with fp32
    norms, as above); numpy on the host, reported for the config's wording."""
    import numpy as np
    from scipy.linalg import hadamard
    from oracle import oracle as O
    h = hadamard(256).astype(np.float64) / 16.0
    sign = np.tile(np.where(O.tq3_signs() > 0, 1.0, -1.0), 2)
    cen = O.tq3_centroids().astype(np.float64) * np.sqrt(0.5)
    bnd = (cen[1:] + cen[:-1]) / 2
    sq = ref = 0.0
    n_el = 0
    codes = []
    for x in planes:
        v = x.astype(np.float64).reshape(-1, 256)
        norm = np.sqrt((v * v).sum(1))
        scale = norm.astype(np.float16).astype(np.float64)
        safe = np.where(norm > 0, norm, 1.0)
        y = (v / safe[:, None] * sign) @ h.T
        idx = np.searchsorted(bnd, y)
        rec = ((cen[idx] @ h) * sign) * scale[:, None]
        sq += float(((rec - v) ** 2).sum())
        ref += float((v * v).sum())
        n_el += v.size
        codes.append(idx.reshape(-1))
    hist = np.bincount(np.concatenate(codes), minlength=8)
    return {"mse": sq / n_el, "rel_mse": sq / ref, "code_hist": [int(c) for c in hist],
            "bytes_per_vector": 256 * 3 // 8 + 2}


def cpu_baselines(torch, caches, q, scale):
    """The oracle (C, -O3, OpenMP) on the GPU box's host: one decode token over
    the 8 layers of cache set 0 (split-K 32 + merge) and the TQ3 encode of one
    layer's 32768-token K and V, each at all usable cores and at one thread."""
    import numpy as np
    from oracle import oracle as O
    nproc = os.cpu_count()
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else nproc
    omp = os.environ.get("OMP_NUM_THREADS")
    cores = max(1, min(affinity, int(omp) if omp and omp.isdigit() else affinity))
    host = [(caches[0][l][0].cpu().numpy().view(O.BLOCK_TQ3).reshape(-1),
             caches[0][l][1].cpu().numpy().view(O.BLOCK_TQ3).reshape(-1),
             q[l].cpu().numpy().view(np.uint16)) for l in range(LAYERS)]

    def decode(threads, layers):
        t = time.perf_counter()
        for kb, vb, qh in host[:layers]:
            pm, pl, po = O.attn_split(O.KV_TQ3, qh, kb, vb, num_q=NUM_Q, num_kv=NUM_KV, hd=HD,
                                      start_pos=CTX - 1, sub_n=1, sub_n_max=1, active_end_max=CTX,
                                      scale=scale, k_splits=32, nthreads=threads)
            O.attn_split_merge(pm, pl, po, num_q=NUM_Q, num_kv=NUM_KV, hd=HD, sub_n=1,
                               sub_n_max=1, k_splits=32)
        return (time.perf_counter() - t) * LAYERS / layers

    dec_all = min(decode(cores, LAYERS) for _ in range(CPU_REPS)) * 1e6
    dec_one = decode(1, 2) * 1e6            # two layers at one thread, scaled to eight
    gen = torch.Generator().manual_seed(11)
    xk = torch.randn(CTX, NUM_KV, HD, generator=gen).to(torch.float16).numpy()
    xv = torch.randn(CTX, NUM_KV, HD, generator=gen).to(torch.float16).numpy()

    def encode(threads):
        t = time.perf_counter()
        O.tq3_encode(xk, nthreads=threads)
        O.tq3_encode(xv, nthreads=threads)
        return time.perf_counter() - t

    enc_all = min(encode(cores) for _ in range(3))
    enc_one = encode(1)
    return {"value": round(dec_all, 1), "unit": "us/token", "cores": cores, "kind": "port",
            "sample": f"1 decode token x 8 layers at 32768 ctx ({CPU_REPS} reps, best), oracle C "
                      "port of the reference split-K decode (32 splits) + merge, OpenMP over "
                      "(kv head, split)",
            "gbps": round(ATTN_BYTES * LAYERS / (dec_all * 1e-6) / 1e9, 3),
            "one_thread_us_per_token": round(dec_one, 1),
            "one_thread_sample": "2 of the 8 layers at one thread, scaled to 8",
            "nproc": nproc, "affinity_cores": affinity, "omp_num_threads": omp,
            "encode": {"unit": "M token-layers/s (K+V of one token in one layer)",
                       "all_cores": round(CTX / enc_all / 1e6, 3),
                       "one_thread": round(CTX / enc_one / 1e6, 3),
                       "sample": "TQ3 encode (oracle C port of tq3_quantize_kernel) of one "
                                 "layer's K and V, 32768 tokens x 4 kv heads x 256"}}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(this path has no multi-GPU component)", file=sys.stderr)
        return 2
    import torch
    from qengine_amd import kvcache

    dev = torch.device("cuda:0")
    if args.copy_calibration:
        a = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": a.numel()}))
        return 0

    kvcache.tq3_init(0)
    gen = torch.Generator(device=dev).manual_seed(3)
    stream = torch.cuda.current_stream()

    # ---- cache build with the append kernel (untimed; it also warms the GPU) ----
    caches, keep_src = [], None
    for s in range(SETS):
        src = [(outlier_kv(torch, gen, CTX, dev), outlier_kv(torch, gen, CTX, dev))
               for _ in range(LAYERS)]
        layers = [(kvcache.tq3_blocks(CTX * BLOCKS_PER_TOKEN, dev),
                   kvcache.tq3_blocks(CTX * BLOCKS_PER_TOKEN, dev)) for _ in range(LAYERS)]
        for (k16, v16), (kb, vb) in zip(src, layers):
            kvcache.tq3_append_kv(k16, v16, kb, vb)
        caches.append(layers)
        if s == 0:
            keep_src = src
        del src
    torch.cuda.synchronize()

    # ---- append throughput: APPEND_REPS passes re-encoding set 0's 8 layers
    # (K+V, one launch per layer) into its own caches, which leaves the bytes
    # unchanged; events on the launch stream around the back-to-back launches ----
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(APPEND_REPS):
        for (k16, v16), (kb, vb) in zip(keep_src, caches[0]):
            kvcache.tq3_append_kv(k16, v16, kb, vb)
    e1.record(stream)
    torch.cuda.synchronize()
    append_s = e0.elapsed_time(e1) * 1e-3
    append_tok_layers = APPEND_REPS * LAYERS * CTX
    # ---- Q8_0 append throughput: the same fp16 K/V of set 0's 8 layers
    # encoded into a Q8_0 cache pair (K+V in one launch per layer; 6400 B per
    # token-layer: 4096 read, 2304 written) ----
    q8k = kvcache.q8_blocks(CTX * Q8_BLOCKS_PER_TOKEN, dev)
    q8v = kvcache.q8_blocks(CTX * Q8_BLOCKS_PER_TOKEN, dev)
    for k16, v16 in keep_src:
        kvcache.q8_append_kv(k16, v16, q8k, q8v)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(APPEND_REPS):
        for k16, v16 in keep_src:
            kvcache.q8_append_kv(k16, v16, q8k, q8v)
    e1.record(stream)
    torch.cuda.synchronize()
    append_q8_s = e0.elapsed_time(e1) * 1e-3
    del keep_src, q8k, q8v
    q = [torch.randn(1, NUM_Q, HD, generator=gen, device=dev).to(torch.float16)
         for _ in range(LAYERS)]
    out = torch.empty(1, NUM_Q, HD, dtype=torch.float16, device=dev)
    ws = kvcache.decode_attn_tq3_workspace(NUM_Q, NUM_KV, 1, CTX, dev)
    scale = 1.0 / (HD ** 0.5)

    def layer(si, l):
        kb, vb = caches[si][l]
        kvcache.decode_attn_tq3(q[l], kb, vb, out, ws, num_q=NUM_Q, num_kv=NUM_KV,
                                start_pos=CTX - 1, sub_n=1, scale=scale)

    def step(i):
        si = i % SETS
        for l in range(LAYERS):
            layer(si, l)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # ---- timed region: K steps, an event between consecutive steps ----
    evs_step = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    torch.cuda.synchronize()
    evs_step[0].record(stream)
    for i in range(args.steps):
        step(i)
        evs_step[i + 1].record(stream)
    torch.cuda.synchronize()
    ms_per_step = evs_step[0].elapsed_time(evs_step[-1]) / args.steps
    us_per_token = ms_per_step * 1e3
    step_us = sorted(evs_step[i].elapsed_time(evs_step[i + 1]) * 1e3 for i in range(args.steps))
    pct = lambda f: step_us[min(len(step_us) - 1, int(f * (len(step_us) - 1) + 0.5))]

    # ---- roofline: the timed region holds only attention launches (LAYERS per
    # step, back to back on `stream`), so its events give the kernel's average
    # launch duration directly ----
    launch_ms = ms_per_step / LAYERS
    achieved = ATTN_BYTES / (launch_ms * 1e-3) / 1e9
    # isolated launches (an event pair around each), for reference
    n_launch = min(args.steps, 40) * LAYERS
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(n_launch)]
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(evs):
        a.record(stream)
        layer((i // LAYERS) % SETS, i % LAYERS)
        b.record(stream)
    torch.cuda.synchronize()
    durs = sorted(a.elapsed_time(b) for a, b in evs)

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("attn_tq3_32k_bytes_per_launch")

    read_peak = hbm_read_peak(torch, kvcache, dev, stream)
    read_floor = launch_read_floor(torch, kvcache, dev, stream, ATTN_BYTES)
    # CPU leg (the oracle as baseline and checker): CPU baselines, and config 1
    # -- the reference's CPU-runnable roundtrip case -- checked against it
    cpu = cfg1 = None
    if not args.no_cpu_baseline:
        cpu = cpu_baselines(torch, caches, q, scale)
        cfg1 = config1_report(torch, kvcache, dev)

    sec = None if args.no_secondary else secondary(torch, kvcache, dev, stream)

    line = {
        "metric": METRIC,
        "value": round(us_per_token, 3),
        "unit": "us/token",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: seeded N(0,1) fp16 K/V with 2% x8 outlier channels, TQ3-encoded on GPU",
        "config": {"workload": "tq3 split-K decode attention, config 3", "layers": LAYERS,
                   "ctx": CTX, "num_q": NUM_Q, "num_kv": NUM_KV, "head_dim": HD,
                   "cache_sets": SETS, "accumulate": "f32",
                   "bytes_per_layer": ATTN_BYTES},
        "hbm_gbps": round(ATTN_BYTES * LAYERS / (us_per_token * 1e-6) / 1e9, 1),
        "hbm_frac": round(ATTN_BYTES * LAYERS / (us_per_token * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "hbm_frac_of_measured_peak": round(ATTN_BYTES * LAYERS / (us_per_token * 1e-6) / 1e9
                                           / read_peak["gbps"], 4),
        "step_stats": {"unit": "us/token", "n": args.steps, "median": round(pct(0.5), 3),
                       "p10": round(pct(0.1), 3), "p90": round(pct(0.9), 3),
                       "min": round(step_us[0], 3), "max": round(step_us[-1], 3)},
        "hbm_read_peak": read_peak,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "kernel": "tq3_attn_kernel<0, false, false>",
                     "frac_of_measured_peak": round(achieved / read_peak["gbps"], 4),
                     "avg_launch_us": round(launch_ms * 1e3, 3),
                     "isolated_launch_median_us": round(durs[len(durs) // 2] * 1e3, 3),
                     "launch_read_floor": read_floor,
                     "frac_of_launch_read_floor": round(read_floor["us_per_launch"]
                                                        / (launch_ms * 1e3), 4)},
        "append": {"mtok_layers_per_s": round(append_tok_layers / append_s / 1e6, 1),
                   "gbps": round(append_tok_layers * APPEND_BYTES_PER_TOKEN / append_s / 1e9, 1),
                   "frac": round(append_tok_layers * APPEND_BYTES_PER_TOKEN / append_s / 1e9
                                 / HBM_PEAK_GBS, 4),
                   "frac_of_measured_peak": round(append_tok_layers * APPEND_BYTES_PER_TOKEN
                                                  / append_s / 1e9 / read_peak["gbps"], 4)},
        "append_q8": {"mtok_layers_per_s": round(append_tok_layers / append_q8_s / 1e6, 1),
                      "gbps": round(append_tok_layers * APPEND_Q8_BYTES_PER_TOKEN / append_q8_s / 1e9, 1),
                      "frac": round(append_tok_layers * APPEND_Q8_BYTES_PER_TOKEN / append_q8_s / 1e9
                                    / HBM_PEAK_GBS, 4),
                      "frac_of_measured_peak": round(append_tok_layers * APPEND_Q8_BYTES_PER_TOKEN
                                                     / append_q8_s / 1e9 / read_peak["gbps"], 4),
                      "us_per_launch": round(append_q8_s * 1e6 / (APPEND_REPS * LAYERS), 2),
                      "note": "qkv_q8_append_kv over 32768 tokens x 4 kv heads (K+V, one launch "
                              "per layer), 8 layers x %d passes; 6400 B per token-layer "
                              "(4096 fp16 read, 2304 Q8_0 written)" % APPEND_REPS},
        "config1": cfg1,
        "cpu_baseline": cpu,
        "secondary": sec,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
