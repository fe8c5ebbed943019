"""The streaming-read kernel behind bench.py's HBM read peak and single-launch
read floor (qkv_hbm_read_bench)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n4,at", [(1024 * 37 + 8, -1), (1024 * 37 + 8, 1024 * 20 + 3),
                                   (4096 * 1024 + 64, -1)])
def test_hbm_read_bench_reads_every_piece(dev, n4, at):
    """qkv_hbm_read_bench (the bench's read peak and single-launch floor) loads
    every 16-byte piece: a buffer that is zero except one piece holding the
    sink value makes exactly that piece's thread write the sink, also in the
    unrolled loop's tail."""
    import torch
    from qengine_amd import kvcache
    buf = torch.zeros(n4 * 4, dtype=torch.int32, device=dev)
    buf[(at % n4) * 4] = int(np.array(0x9E3779B9, dtype=np.uint32).view(np.int32))
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    kvcache.hbm_read_bench(buf.view(torch.uint8), sink)
    torch.cuda.synchronize()
    assert int(sink.cpu().numpy().view(np.uint32)[0]) == 0x9E3779B9
    sink.zero_()
    buf.zero_()
    kvcache.hbm_read_bench(buf.view(torch.uint8), sink)
    torch.cuda.synchronize()
    assert int(sink.cpu()[0]) == 0
