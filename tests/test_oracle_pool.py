"""Pins the oracle's BlockPool/PageTable restatement.

Known answers: src/main.cpp:298-408 (Phase 3: [0,2] [1] [3,4,5], 6 blocks,
full reclaim) and src/main.cpp:73-156 (Phase 4: pages [0,2]).  Random traces
are compared op for op with the reference's own classes (oracle/_ref).
"""
import numpy as np
import pytest

import oracle
from oracle import OP_ALLOC_SEQ as A, OP_APPEND as P, OP_FREE_SEQ as F
from oracle import ST_EXISTS, ST_OK, ST_OOM, ST_UNKNOWN


def _trace(total, bs, ops, max_seqs=8, max_blocks_out=16, ref=False):
    return oracle.pool_trace(total, bs, ops, max_seqs, max_blocks_out, use_reference=ref)


def test_phase3_fragmentation_known_answer():
    ops = [(A, 1), (A, 2)] + [(P, 1)] * 20 + [(P, 2)] * 5 + [(A, 3)] + [(P, 3)] * 35
    res, lens, blocks, drain = _trace(100, 16, ops)
    assert (res[:, 0] == ST_OK).all()
    assert list(lens[1:4]) == [20, 5, 35]
    assert list(blocks[1][:3]) == [0, 2, -1]
    assert list(blocks[2][:2]) == [1, -1]
    assert list(blocks[3][:4]) == [3, 4, 5, -1]
    assert len(drain) == 100 - 6                      # 6 blocks in use
    ops_free = ops + [(F, 1), (F, 2), (F, 3)]
    _, lens2, _, drain2 = _trace(100, 16, ops_free)
    assert len(drain2) == 100 and (lens2[1:4] == -1).all()


def test_phase4_pages_known_answer():
    ops = [(A, 1), (A, 2)] + [(P, 1)] * 5
    _, lens, blocks, _ = _trace(8, 4, ops)
    assert lens[1] == 5 and list(blocks[1][:3]) == [0, 2, -1]


def test_lifo_reuse_order_and_lazy_blocks():
    # N tokens use max(1, ceil(N/bs)) blocks; freeing returns blocks in table
    # order, so the last block of the freed sequence is handed out first.
    ops = [(A, 0)] + [(P, 0)] * 33 + [(F, 0), (A, 1), (P, 1), (A, 2)]
    res, lens, blocks, drain = _trace(10, 16, ops)
    assert list(res[:, 1][:1]) == [0]
    assert [b for b in res[1:34, 1] if b >= 0] == [1, 2]  # blocks at tokens 17 and 33
    assert list(blocks[1][:2]) == [2, -1] and list(blocks[2][:1]) == [1]
    assert list(drain[:3]) == [0, 3, 4]


def test_error_statuses():
    ops = [(A, 0), (A, 0), (P, 5), (F, 6), (A, 1), (A, 2), (P, 0)]
    res, lens, _, _ = _trace(2, 4, ops)
    assert list(res[:, 0]) == [ST_OK, ST_EXISTS, ST_UNKNOWN, ST_UNKNOWN, ST_OK, ST_OOM, ST_OK]
    # Exhaust: the 5th token of sequence 0 needs a block the pool no longer has.
    ops2 = ops + [(P, 0)] * 4
    res2, lens2, _, _ = _trace(2, 4, ops2)
    assert res2[-1, 0] == ST_OOM and lens2[0] == 4   # length unchanged on OOM


def _random_trace(rng, n_ops, max_seqs):
    ops = []
    for _ in range(n_ops):
        r = rng.random()
        s = int(rng.integers(0, max_seqs))
        ops.append((A if r < 0.15 else F if r < 0.25 else P, s))
    return ops


@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built (needs the StrataKV sources)")
@pytest.mark.parametrize("seed", range(40))
def test_random_traces_match_reference(seed):
    rng = np.random.default_rng(seed)
    total = int(rng.integers(1, 40))
    bs = int(rng.integers(1, 9))
    ops = _random_trace(rng, 400, 6)
    mine = _trace(total, bs, ops, max_seqs=6, max_blocks_out=64)
    theirs = _trace(total, bs, ops, max_seqs=6, max_blocks_out=64, ref=True)
    for a, b in zip(mine, theirs):
        np.testing.assert_array_equal(a, b)
