"""Below 4096 cache rows the reference decodes through its legacy unfused path
(model.cuh:2544-2664): bulk fp16 dequantization, attn_score_kernel_h,
softmax_kernel, attn_value_kernel_h (attention.cuh:277-316, 531-575,
885-907), or with TQ_FUSED the fp32 TQ3 kernels (attention.cuh:400-483,
920-989).  This build serves every length with its fused decode kernels; here
they are checked against the oracle's restatement of that legacy path
(oracle.legacy_decode) at 1 .. 4095 rows.

Bars:
- TQ3 decode (fast path and split + merge): tests/_data.assert_tq3_attn
  against the default legacy path (fp16 scratch) and the exact fp64 attention,
  and every row within 2e-3 of the TQ_FUSED legacy path, whose fp32
  dequantization has no fp16 rounding;
- Q8 decode: every row within 2e-3 of the legacy path;
- Q8 keys + TQ3 values: every row within 2e-3 of the TQ_FUSED legacy path and
  assert_tq3_attn against the default one."""
import numpy as np
import pytest

from oracle import oracle as O
from tests._data import assert_tq3_attn, check_rel, kv_f16, q_f16

pytestmark = pytest.mark.gpu
TOL = 2e-3
HD, NKV = 256, 4
LENS = [1, 2, 63, 64, 65, 257, 1000, 2048, 4095]


def _dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _legacy(kk, vk, q, k, v, num_q, n, fused=False):
    return O.legacy_decode(kk, vk, q, k, v, num_q=num_q, num_kv=NKV, hd=HD, seq_len=n,
                           scale=1 / 16, tq_fused=fused).view(np.float16).reshape(1, num_q, HD)


@pytest.mark.parametrize("num_q", [16, 24])
@pytest.mark.parametrize("n", LENS)
def test_tq3_decode_vs_legacy(dev, n, num_q):
    import torch
    from qengine_amd import kvcache
    rng = np.random.default_rng(3000 + n + num_q)
    kb, vb = O.tq3_encode(kv_f16(rng, n, NKV, HD)), O.tq3_encode(kv_f16(rng, n, NKV, HD))
    q = q_f16(rng, 1, num_q, HD)
    print(f"tq3 legacy n={n} num_q={num_q}", flush=True)
    qd, kd, vd = _dev(q.view(np.uint16), dev), _dev(kb.view(np.uint8), dev), _dev(vb.view(np.uint8), dev)
    out = torch.zeros((1, num_q, HD), dtype=torch.float16, device=dev)
    ws = kvcache.decode_attn_tq3_workspace(num_q, NKV, 1, n, dev)
    kvcache.decode_attn_tq3(qd, kd, vd, out, ws, num_q=num_q, num_kv=NKV, start_pos=n - 1,
                            sub_n=1, scale=1 / 16)
    ks = 8
    pm = torch.zeros((num_q, 1, ks), dtype=torch.float32, device=dev)
    pl = torch.zeros_like(pm)
    po = torch.zeros((num_q, 1, ks, HD), dtype=torch.float32, device=dev)
    out2 = torch.zeros_like(out)
    kvcache.attn_split_tq3(qd, kd, vd, pm, pl, po, num_q=num_q, num_kv=NKV, start_pos=n - 1,
                           sub_n=1, sub_n_max=1, active_end_max=n, scale=1 / 16, k_splits=ks)
    kvcache.attn_split_merge(pm, pl, po, out2, num_q=num_q, num_kv=NKV, sub_n=1, sub_n_max=1,
                             k_splits=ks)
    torch.cuda.synchronize()
    legacy = _legacy(O.KV_TQ3, O.KV_TQ3, q, kb, vb, num_q, n)
    fused = _legacy(O.KV_TQ3, O.KV_TQ3, q, kb, vb, num_q, n, fused=True)
    exact = O.attn_exact_tq3(q, kb, vb, num_q=num_q, num_kv=NKV, hd=HD, start_pos=n - 1,
                             sub_n=1, scale=1 / 16)
    for got in (out.cpu().numpy(), out2.cpu().numpy()):
        assert np.all(np.isfinite(got))
        assert_tq3_attn(got, legacy, exact, what=n)
        check_rel(got, fused, TOL)


@pytest.mark.parametrize("n", LENS)
def test_q8_decode_vs_legacy(dev, n):
    import torch
    from qengine_amd import kvcache
    rng = np.random.default_rng(4000 + n)
    kb, vb = O.q8_encode(kv_f16(rng, n, NKV, HD)), O.q8_encode(kv_f16(rng, n, NKV, HD))
    q = q_f16(rng, 1, 16, HD)
    print(f"q8 legacy n={n}", flush=True)
    out = torch.zeros((1, 16, HD), dtype=torch.float16, device=dev)
    ws = kvcache.decode_attn_q8_workspace(16, NKV, 1, n, dev)
    kvcache.decode_attn_q8(_dev(q.view(np.uint16), dev), _dev(kb.view(np.uint8), dev),
                           _dev(vb.view(np.uint8), dev), out, ws, num_q=16, num_kv=NKV,
                           start_pos=n - 1, sub_n=1, scale=1 / 16)
    torch.cuda.synchronize()
    check_rel(out.cpu().numpy(), _legacy(O.KV_Q8, O.KV_Q8, q, kb, vb, 16, n), TOL)


@pytest.mark.parametrize("n", LENS)
def test_q8k_tq3v_decode_vs_legacy(dev, n):
    import torch
    from qengine_amd import kvcache
    rng = np.random.default_rng(5000 + n)
    kq, vt = O.q8_encode(kv_f16(rng, n, NKV, HD)), O.tq3_encode(kv_f16(rng, n, NKV, HD))
    q = q_f16(rng, 1, 16, HD)
    print(f"q8k/tq3v legacy n={n}", flush=True)
    out = torch.zeros((1, 16, HD), dtype=torch.float16, device=dev)
    ws = kvcache.decode_attn_q8k_tq3v_workspace(16, NKV, 1, n, dev)
    kvcache.decode_attn_q8k_tq3v(_dev(q.view(np.uint16), dev), _dev(kq.view(np.uint8), dev),
                                 _dev(vt.view(np.uint8), dev), out, ws, num_q=16, num_kv=NKV,
                                 start_pos=n - 1, sub_n=1, scale=1 / 16)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    fused = _legacy(O.KV_Q8, O.KV_TQ3, q, kq, vt, 16, n, fused=True)
    legacy = _legacy(O.KV_Q8, O.KV_TQ3, q, kq, vt, 16, n)
    exact = O.attn_q8k_tq3v_f64(q, kq, vt, num_q=16, num_kv=NKV, hd=HD, start_pos=n - 1, sub_n=1,
                                scale=1 / 16)
    check_rel(got, fused, TOL)
    assert_tq3_attn(got, legacy, exact, what=n)
