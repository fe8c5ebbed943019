"""GPU parity of qkv_kv_move_tokens against the reference's per-token copies
(kv_move_token, model.cuh:7430-7471; oracle.move_token_rows applies them in
list order).  Rows are opaque bytes, so the bar is bit-exact: random TQ3
(8 x 52 B per token) and Q8_0 (32 x 36 B) rows, moves that run in parallel
and lists whose moves depend on each other (run in order), no-op moves, a
slot offset, and the empty list."""
import zlib

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


ROW_BYTES = {"tq3": 8 * 52, "q8": 32 * 36}

CASES = [
    ("disjoint", [(10, 0), (11, 1), (12, 2), (40, 3)]),                # parallel
    ("accept_tree", [(5, 2), (9, 3), (12, 4), (13, 5)]),              # 5 read after written
    ("chain", [(3, 0), (0, 6), (6, 1)]),                              # each reads the last one
    ("same_dest", [(7, 2), (8, 2)]),                                  # the later write wins
    ("noop_mixed", [(4, 4), (20, 21), (21, 21)]),
    ("many", [(63 - i, i) for i in range(32)]),
]


@pytest.mark.parametrize("fmt", ["tq3", "q8"])
@pytest.mark.parametrize("name,moves", CASES, ids=[c[0] for c in CASES])
def test_kv_move_tokens_matches_sequential_copies(dev, fmt, name, moves):
    from qengine_amd import kvcache
    torch = _torch()
    rb = ROW_BYTES[fmt]
    rows, slot0 = 96, 16                      # a slot of 64 rows starting at row 16
    rng = np.random.default_rng(zlib.crc32(f"{fmt}/{name}".encode()))
    k = rng.integers(0, 256, (rows, rb), dtype=np.uint8)
    v = rng.integers(0, 256, (rows, rb), dtype=np.uint8)
    kd, vd = torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev)
    kvcache.kv_move_tokens(kd, vd, moves, k_row_bytes=rb, v_row_bytes=rb, slot_row0=slot0,
                           slot_rows=64)
    torch.cuda.synchronize()
    assert np.array_equal(kd.cpu().numpy(), O.move_token_rows(k, moves, slot0))
    assert np.array_equal(vd.cpu().numpy(), O.move_token_rows(v, moves, slot0))


def test_kv_move_tokens_mixed_row_sizes_and_empty(dev):
    """K and V rows of different sizes (a Q8_0 key row and a TQ3 value row);
    an empty list changes nothing."""
    from qengine_amd import kvcache
    torch = _torch()
    rng = np.random.default_rng(7)
    k = rng.integers(0, 256, (32, ROW_BYTES["q8"]), dtype=np.uint8)
    v = rng.integers(0, 256, (32, ROW_BYTES["tq3"]), dtype=np.uint8)
    kd, vd = torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev)
    moves = [(30, 1), (1, 2)]
    kvcache.kv_move_tokens(kd, vd, moves, k_row_bytes=ROW_BYTES["q8"],
                           v_row_bytes=ROW_BYTES["tq3"])
    kvcache.kv_move_tokens(kd, vd, [], k_row_bytes=ROW_BYTES["q8"], v_row_bytes=ROW_BYTES["tq3"])
    torch.cuda.synchronize()
    assert np.array_equal(kd.cpu().numpy(), O.move_token_rows(k, moves))
    assert np.array_equal(vd.cpu().numpy(), O.move_token_rows(v, moves))
