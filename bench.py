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
                counters (profiles/traffic.json)
  append        TQ3 append (K+V) throughput of the cache build
  cpu_baseline  the CPU oracle (C port of the reference arithmetic, OpenMP)
                on a bounded sample: one decode token over the 8 layers
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
CPU_REPS = 5
APPEND_REPS = 5


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
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
    del keep_src
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

    # ---- timed region: K steps ----
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record(stream)
    for i in range(args.steps):
        step(i)
    t1.record(stream)
    torch.cuda.synchronize()
    ms_per_step = t0.elapsed_time(t1) / args.steps
    us_per_token = ms_per_step * 1e3

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

    # ---- CPU baseline: the oracle on one decode token over the 8 layers ----
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import oracle as O
        import numpy as np
        cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
        cores = max(1, min(cores, 16))
        host = [(caches[0][l][0].cpu().numpy().view(O.BLOCK_TQ3).reshape(-1),
                 caches[0][l][1].cpu().numpy().view(O.BLOCK_TQ3).reshape(-1),
                 q[l].cpu().numpy().view(np.uint16)) for l in range(LAYERS)]
        times = []
        for rep in range(CPU_REPS):
            t = time.perf_counter()
            for kb, vb, qh in host:
                pm, pl, po = O.attn_split(O.KV_TQ3, qh, kb, vb, num_q=NUM_Q, num_kv=NUM_KV,
                                          hd=HD, start_pos=CTX - 1, sub_n=1, sub_n_max=1,
                                          active_end_max=CTX, scale=scale, k_splits=32,
                                          nthreads=cores)
                O.attn_split_merge(pm, pl, po, num_q=NUM_Q, num_kv=NUM_KV, hd=HD, sub_n=1,
                                   sub_n_max=1, k_splits=32)
            times.append(time.perf_counter() - t)
        cpu_us = min(times) * 1e6
        cpu = {"value": round(cpu_us, 1), "unit": "us/token", "cores": cores, "kind": "port",
               "sample": f"1 decode token x 8 layers at 32768 ctx ({CPU_REPS} reps, best), oracle C "
                         "port of the reference split-K decode, OpenMP over (kv head, split)",
               "gbps": round(ATTN_BYTES * LAYERS / (cpu_us * 1e-6) / 1e9, 3)}

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
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "kernel": "tq3_attn_kernel<0>",
                     "avg_launch_us": round(launch_ms * 1e3, 3),
                     "isolated_launch_median_us": round(durs[len(durs) // 2] * 1e3, 3)},
        "append": {"mtok_layers_per_s": round(append_tok_layers / append_s / 1e6, 1),
                   "gbps": round(append_tok_layers * APPEND_BYTES_PER_TOKEN / append_s / 1e9, 1),
                   "frac": round(append_tok_layers * APPEND_BYTES_PER_TOKEN / append_s / 1e9
                                 / HBM_PEAK_GBS, 4)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
