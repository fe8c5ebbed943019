"""Per-phase timeline of the TQ3 fast-path decode launch (diagnostic).

Runs the decode attention of BASELINE config 3 (16 q / 4 kv heads, d=256,
32768 keys; other sizes by flag) through ``libqkv_trace.so``: the same
library as ``libqkv.so`` except that the decode kernel is compiled with
-DQKV_PHASE_TRACE, so that every wave records ``s_memrealtime`` (100 MHz, one
clock for the whole GPU) at its phase boundaries (``TracePhase`` in
``csrc/attn_tq3.hip``).  Launches run back to back on rotating caches (more
bytes than the Infinity Cache holds); the stamps of the last launch of each
burst are read back, and every phase is reported as medians / percentiles
over workgroups, in microseconds from the launch's first wave.

    python -m qengine_amd.phase_trace [--ctx 32768] [--bursts 20] [--md FILE]
"""
import argparse
import ctypes
import os
import sys

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
WAVES = 8
SLOTS = 16
PHASES = ["entry", "query", "setup", "scores", "softmax", "tiles", "merged", "published",
          "polled", "end", "merge barrier", "rows in", "folded", "setup work", "tile barrier"]
TICK_US = 0.01   # s_memrealtime runs at 100 MHz


def _stamps(L, n_wg):
    buf = np.zeros(n_wg * WAVES * SLOTS, dtype=np.uint64)
    rc = L.qkv_debug_phase_stamps(buf.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(buf.size))
    if rc != 0:
        raise RuntimeError(f"qkv_debug_phase_stamps failed ({rc})")
    return buf.reshape(n_wg, WAVES, SLOTS)


def _launch_sample(st):
    """One launch's stamps -> dict of per-workgroup phase times (us from its first wave)."""
    t = st[:, :, :len(PHASES)].astype(np.int64)
    live = t[:, :, 0] > 0
    t0 = t[:, :, 0][live].min()
    rel = np.where(t > 0, (t - t0) * TICK_US, np.nan)
    out = {}
    out["entry"] = np.nanmin(rel[:, :, 0], axis=1)                       # first wave of the workgroup
    out["query"] = np.nanmax(rel[:, :, 1], axis=1)
    out["setup work w0-3"] = np.nanmax(rel[:, :4, 13], axis=1)
    out["setup work w4-7"] = np.nanmax(rel[:, 4:, 13], axis=1)
    out["setup"] = np.nanmax(rel[:, :, 2], axis=1)
    for name, k in (("scores", 3), ("softmax", 4), ("tiles", 5)):
        out[name + " w0-3"] = np.nanmax(rel[:, :4, k], axis=1)
        out[name + " w4-7"] = np.nanmax(rel[:, 4:, k], axis=1)
    out["tile barrier"] = np.nanmax(rel[:, :, 14], axis=1)
    out["merge barrier"] = np.nanmax(rel[:, :, 10], axis=1)
    out["merged"] = np.nanmax(rel[:, :, 6], axis=1)
    out["published"] = np.nanmax(rel[:, :, 7], axis=1)
    pol = rel[:, 0, 8]
    merger = ~np.isnan(pol)
    out["polled (mergers)"] = pol[merger]
    out["rows in (mergers)"] = rel[:, 0, 11][merger]
    out["folded (mergers)"] = rel[:, 0, 12][merger]
    end = np.nanmax(rel[:, :, 9], axis=1)
    out["end (mergers)"] = end[merger]
    out["end (others)"] = end[~merger]
    xcd = st[:, 0, 15].astype(np.int64)
    out["_xcd_start"] = {int(x): float(np.nanmin(out["entry"][xcd == x])) for x in np.unique(xcd)}
    out["_launch_end"] = float(np.nanmax(end))
    return out


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--ctx", type=int, default=32768)
    ap.add_argument("--num-q", type=int, default=16)
    ap.add_argument("--num-kv", type=int, default=4)
    ap.add_argument("--sets", type=int, default=24, help="cache sets rotated over (default 24: 654 MB at 32K)")
    ap.add_argument("--burst", type=int, default=24, help="back-to-back launches per sample")
    ap.add_argument("--bursts", type=int, default=20, help="samples (the last launch of each burst)")
    ap.add_argument("--md", default=None, help="also write the table to this markdown file")
    args = ap.parse_args(argv)

    import torch
    sys.path.insert(0, os.path.dirname(_HERE))
    from qengine_amd import _lib
    _lib.LIB_PATH = os.path.join(_HERE, "libqkv_trace.so")
    from qengine_amd import kvcache

    L = _lib.lib()
    if not hasattr(L, "qkv_debug_phase_stamps"):
        raise SystemExit("libqkv_trace.so has no phase stamps: build it (make -C qengine_amd/csrc)")
    L.qkv_debug_phase_stamps.restype = ctypes.c_int
    L.qkv_debug_phase_stamps.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    L.qkv_debug_phase_clear.restype = ctypes.c_int

    dev = torch.device("cuda:0")
    kvcache.tq3_init(0)
    ctx, nq, nkv = args.ctx, args.num_q, args.num_kv
    g = torch.Generator(device=dev).manual_seed(11)
    caches = []
    for _ in range(args.sets):
        k16 = torch.randn(ctx, nkv, 256, generator=g, device=dev).half()
        v16 = torch.randn(ctx, nkv, 256, generator=g, device=dev).half()
        kb, vb = kvcache.tq3_blocks(ctx * nkv * 2, dev), kvcache.tq3_blocks(ctx * nkv * 2, dev)
        kvcache.tq3_append_kv(k16, v16, kb, vb)
        caches.append((kb, vb))
    del k16, v16
    q = torch.randn(1, nq, 256, generator=g, device=dev).half()
    out = torch.empty(1, nq, 256, dtype=torch.float16, device=dev)
    ws = kvcache.decode_attn_tq3_workspace(nq, nkv, 1, ctx, dev)

    def step(i):
        kb, vb = caches[i % len(caches)]
        kvcache.decode_attn_tq3(q, kb, vb, out, ws, num_q=nq, num_kv=nkv, start_pos=ctx - 1, sub_n=1,
                                scale=1 / 16)

    for i in range(2 * args.burst):
        step(i)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(10 * args.burst):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    us_launch = e0.elapsed_time(e1) / (10 * args.burst) * 1e3

    samples = []
    n_wg_max = 4096
    for b in range(args.bursts):
        if L.qkv_debug_phase_clear() != 0:
            raise RuntimeError("qkv_debug_phase_clear failed")
        for i in range(args.burst):
            step(b * args.burst + i)
        torch.cuda.synchronize()
        st = _stamps(L, n_wg_max)
        n_wg = int((st[:, 0, 0] > 0).sum())
        samples.append(_launch_sample(st[:n_wg]))

    keys = [k for k in samples[0] if not k.startswith("_")]
    lines = [f"Decode phase timeline: {ctx} keys, {nq} q / {nkv} kv heads, d=256, one query; "
             f"{len(samples)} launches (the last of each burst of {args.burst} back-to-back launches "
             f"over {args.sets} rotating cache sets); trace build {us_launch:.2f} us/launch (events).",
             "",
             "Times in us from the launch's first wave; per workgroup (the latest of its waves, except "
             "`entry`: its first), then median / p10 / p90 / max over workgroups, each the median over "
             "launches.",
             "",
             "| phase | median | p10 | p90 | max |",
             "|---|---|---|---|---|"]
    for k in keys:
        stats = np.array([[np.median(s[k]), np.percentile(s[k], 10), np.percentile(s[k], 90), np.max(s[k])]
                          for s in samples if len(s[k])])
        med = np.median(stats, axis=0)
        lines.append(f"| {k} | {med[0]:.2f} | {med[1]:.2f} | {med[2]:.2f} | {med[3]:.2f} |")
    xcds = sorted(samples[0]["_xcd_start"])
    xs = np.array([[s["_xcd_start"].get(x, np.nan) for x in xcds] for s in samples])
    lines += ["", "First wave per XCD (us from the launch's first wave, median over launches): " +
              ", ".join(f"XCD {x}: {v:.2f}" for x, v in zip(xcds, np.nanmedian(xs, axis=0))),
              "", f"Last wave done: {np.median([s['_launch_end'] for s in samples]):.2f} us "
              "after the first wave started (median over launches)."]
    text = "\n".join(lines)
    print(text)
    if args.md:
        with open(args.md, "w") as f:
            f.write(text + "\n")


if __name__ == "__main__":
    main()
