"""GPU parity of the V-only TurboQuant decode (keys Q8_0, values TQ3: the
reference's TQ_KEYS_Q8 mode, model.cuh:2574-2588) against the CPU oracle on
identical seeded inputs.  Bar: every (query, head) output row within 2e-3
relative error of the fp64 attention over the dequantized cache (max |diff| /
max |ref| per row); fp32 accumulation."""
import numpy as np
import pytest

from oracle import oracle as O
from tests._data import check_rel, kv_f16, q_f16

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _torch():
    import torch
    return torch


def _dev(a, dev):
    return _torch().from_numpy(np.ascontiguousarray(a)).to(dev)


def _case(seed, n, num_q, sub_n, num_kv=4):
    rng = np.random.default_rng(seed)
    kq = O.q8_encode(kv_f16(rng, n, num_kv, 256))
    vt = O.tq3_encode(kv_f16(rng, n, num_kv, 256))
    q = q_f16(rng, sub_n, num_q, 256)
    ref = O.attn_q8k_tq3v_f64(q, kq, vt, num_q=num_q, num_kv=num_kv, hd=256,
                              start_pos=n - sub_n, sub_n=sub_n, scale=1 / 16)
    return q, kq, vt, ref


def _decode(dev, q, kq, vt, ws, n, num_q, sub_n, num_kv=4):
    from qengine_amd import kvcache
    torch = _torch()
    out = torch.zeros((sub_n, num_q, 256), dtype=torch.float16, device=dev)
    print(f"mixed decode n={n} num_q={num_q} sub_n={sub_n}", flush=True)
    kvcache.decode_attn_q8k_tq3v(_dev(q.view(np.uint16), dev), _dev(kq.view(np.uint8), dev),
                                 _dev(vt.view(np.uint8), dev), out, ws, num_q=num_q,
                                 num_kv=num_kv, start_pos=n - sub_n, sub_n=sub_n, scale=1 / 16)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("n,num_q,sub_n", [
    (4097, 16, 1), (32768, 16, 1),
    (1, 16, 1), (31, 16, 1), (127, 16, 1), (129, 16, 1), (20000, 16, 1),
    (700, 24, 1),      # GQA 6
    (700, 8, 1),       # GQA 2
    (530, 16, 16),     # 16 causal queries
    (3000, 4, 1),      # GQA 1
    (3000, 32, 1),     # GQA 8 (staging rows 0 and 1)
    (4500, 16, 4),     # several causal queries over thousands of keys
    (3000, 32, 2),     # GQA 8, two queries
    (2000, 4, 3),      # GQA 1, three queries
])
def test_mixed_decode_vs_oracle(dev, n, num_q, sub_n):
    from qengine_amd import kvcache
    q, kq, vt, ref = _case(900 + n + num_q + sub_n, n, num_q, sub_n)
    ws = kvcache.decode_attn_q8k_tq3v_workspace(num_q, 4, sub_n, n, dev)
    check_rel(_decode(dev, q, kq, vt, ws, n, num_q, sub_n), ref, TOL)


def test_mixed_and_q8_share_a_workspace(dev):
    """Calls of both Q8-key decodes, of different lengths, in turn on one
    workspace (the mergers clear the tags they consumed)."""
    from qengine_amd import kvcache
    torch = _torch()
    ws = kvcache.decode_attn_q8k_tq3v_workspace(16, 4, 4, 8192, dev)
    for i, (n, sub_n) in enumerate([(8192, 1), (4097, 1), (1000, 4), (8192, 1), (300, 4)]):
        q, kq, vt, ref = _case(950 + i, n, 16, sub_n)
        check_rel(_decode(dev, q, kq, vt, ws, n, 16, sub_n), ref, TOL, what=(n, sub_n))
        rng = np.random.default_rng(960 + i)
        k16, v16 = kv_f16(rng, n, 4, 256), kv_f16(rng, n, 4, 256)
        kb, vb = O.q8_encode(k16), O.q8_encode(v16)
        out = torch.zeros((sub_n, 16, 256), dtype=torch.float16, device=dev)
        kvcache.decode_attn_q8(_dev(q.view(np.uint16), dev), _dev(kb.view(np.uint8), dev),
                               _dev(vb.view(np.uint8), dev), out, ws, num_q=16, num_kv=4,
                               start_pos=n - sub_n, sub_n=sub_n, scale=1 / 16)
        torch.cuda.synchronize()
        ref8 = O.attn_ref_f64(q, O.q8_decode(kb), O.q8_decode(vb), num_q=16, num_kv=4, hd=256,
                              start_pos=n - sub_n, sub_n=sub_n, scale=1 / 16)
        check_rel(out.cpu().numpy(), ref8, TOL, what=("q8", n, sub_n))
