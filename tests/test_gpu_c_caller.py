"""The C ABI from compiled C and C++ callers (tests/c_caller/qkv_caller.c,
built by tests/c_caller/Makefile as C11 and as C++17, linked against the
in-tree libqkv.so).

Each binary issues one TQ3 decode step the way the reference launches it
(model.cuh:2316-2333 appends of the new token's K then V at row start_pos;
model.cuh:2472-2491 split-K decode over the slot base, sub_n 1, sub_n_max 16,
K_SPLITS 8, merged in place over the query buffer) plus the single-launch
fast path.  The caches and both outputs must equal, bit for bit, the same
calls made through the Python binding (same kernels, same inputs), the
outputs of the two binaries must be identical, and the outputs are checked
against the oracle (split + merge within 2e-3 per row of the reference-order
restatement; the fast path to its own bar)."""
import os
import subprocess

import numpy as np
import pytest

from oracle import oracle as O
from tests._data import assert_tq3_attn, check_rel, kv_f16, q_f16

pytestmark = pytest.mark.gpu
HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c_caller")
BINS = ["qkv_caller_c", "qkv_caller_cxx"]
TOL = 2e-3


def _run(binary, tmp_path, n_ctx, num_q, num_kv, k16, v16, q):
    path = os.path.join(HERE, binary)
    if not os.path.exists(path):
        pytest.fail(f"{path} is not built (run __graft_entry__.build())")
    fin, fout = tmp_path / f"{binary}.in", tmp_path / f"{binary}.out"
    with open(fin, "wb") as f:
        f.write(np.array([n_ctx, num_q, num_kv], np.int32).tobytes())
        f.write(k16.tobytes() + v16.tobytes() + q.tobytes())
    print(f"running {binary} n_ctx={n_ctx} num_q={num_q} num_kv={num_kv}", flush=True)
    r = subprocess.run([path, str(fin), str(fout)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, (binary, r.returncode, r.stdout, r.stderr)
    raw = np.fromfile(fout, dtype=np.uint8)
    qb = num_q * 256 * 2
    cb = (n_ctx + 1) * num_kv * 2 * 52
    assert raw.size == 2 * qb + 2 * cb
    merged = raw[:qb].view(np.float16).reshape(num_q, 256)
    fast = raw[qb:2 * qb].view(np.float16).reshape(num_q, 256)
    return merged, fast, raw[2 * qb:2 * qb + cb], raw[2 * qb + cb:]


def _python_path(dev, n_ctx, num_q, num_kv, k16, v16, q):
    import torch
    from qengine_amd import kvcache
    bpt = num_kv * 2
    kd = torch.from_numpy(k16.reshape(-1).view(np.uint16).copy()).to(dev).view(torch.float16)
    vd = torch.from_numpy(v16.reshape(-1).view(np.uint16).copy()).to(dev).view(torch.float16)
    kc = kvcache.tq3_blocks((n_ctx + 1) * bpt, dev)
    vc = kvcache.tq3_blocks((n_ctx + 1) * bpt, dev)
    row = num_kv * 256
    if n_ctx:
        kvcache.tq3_append(kd[:n_ctx * row], kc[:n_ctx * bpt])
        kvcache.tq3_append(vd[:n_ctx * row], vc[:n_ctx * bpt])
    kvcache.tq3_append(kd[n_ctx * row:], kc[n_ctx * bpt:])
    kvcache.tq3_append(vd[n_ctx * row:], vc[n_ctx * bpt:])
    qd = torch.from_numpy(q.reshape(1, num_q, 256)).to(dev)
    q_split = qd.clone()
    pm = torch.empty(num_q, 16, 8, device=dev)
    pl = torch.empty(num_q, 16, 8, device=dev)
    po = torch.empty(num_q, 16, 8, 256, device=dev)
    kvcache.attn_split_tq3(q_split, kc, vc, pm, pl, po, num_q=num_q, num_kv=num_kv,
                           start_pos=n_ctx, sub_n=1, sub_n_max=16, active_end_max=n_ctx + 1,
                           scale=1 / 16, k_splits=8)
    kvcache.attn_split_merge(pm, pl, po, q_split, num_q=num_q, num_kv=num_kv, sub_n=1,
                             sub_n_max=16, k_splits=8)
    out = torch.empty_like(qd)
    ws = kvcache.decode_attn_tq3_workspace(num_q, num_kv, 1, n_ctx + 1, dev)
    kvcache.decode_attn_tq3(qd, kc, vc, out, ws, num_q=num_q, num_kv=num_kv, start_pos=n_ctx,
                            sub_n=1, scale=1 / 16)
    torch.cuda.synchronize()
    return (q_split.cpu().numpy().reshape(num_q, 256), out.cpu().numpy().reshape(num_q, 256),
            kc.cpu().numpy().reshape(-1), vc.cpu().numpy().reshape(-1))


@pytest.mark.parametrize("n_ctx,num_q,num_kv,seed", [(4096, 16, 4, 81), (100, 24, 4, 82), (0, 8, 2, 83)])
def test_c_and_cxx_callers_match_python_path(dev, tmp_path, n_ctx, num_q, num_kv, seed):
    rng = np.random.default_rng(seed)
    k16 = kv_f16(rng, n_ctx + 1, num_kv, 256)
    v16 = kv_f16(rng, n_ctx + 1, num_kv, 256)
    q = q_f16(rng, 1, num_q, 256)
    res = [_run(b, tmp_path, n_ctx, num_q, num_kv, k16, v16, q) for b in BINS]
    py = _python_path(dev, n_ctx, num_q, num_kv, k16, v16, q)
    for b, r in zip(BINS, res):
        for name, got, exp in zip(("merged", "fast", "k cache", "v cache"), r, py):
            assert np.array_equal(got.view(np.uint8), exp.view(np.uint8)), (b, name)
    # the caches are the reference's encoding; the outputs follow the oracle
    kb, vb = O.tq3_encode(k16), O.tq3_encode(v16)
    assert np.array_equal(res[0][2], kb.view(np.uint8).reshape(-1))
    assert np.array_equal(res[0][3], vb.view(np.uint8).reshape(-1))
    pm, pl, po = O.attn_split(O.KV_TQ3, q, kb, vb, num_q=num_q, num_kv=num_kv, hd=256,
                              start_pos=n_ctx, sub_n=1, sub_n_max=16, active_end_max=n_ctx + 1,
                              scale=1 / 16, k_splits=8)
    ref = O.attn_split_merge(pm, pl, po, num_q=num_q, num_kv=num_kv, hd=256, sub_n=1, sub_n_max=16,
                             k_splits=8).view(np.float16).astype(np.float64).reshape(num_q, 256)
    check_rel(res[0][0].astype(np.float64), ref, TOL, what=("split+merge", n_ctx))
    exact = O.attn_exact_tq3(q, kb, vb, num_q=num_q, num_kv=num_kv, hd=256, start_pos=n_ctx,
                             sub_n=1, scale=1 / 16).reshape(num_q, 256)
    assert_tq3_attn(res[0][1].astype(np.float64), ref, exact, what=("fast", n_ctx))
