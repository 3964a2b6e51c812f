"""KV append on the GPU: bit-exact against the oracle's scatter.

Both sides start from the same poisoned pools (0xFFFF, a NaN pattern), so an
element written to a wrong place, or not written, shows up as a mismatch
anywhere in the pool.
"""
import numpy as np
import pytest

import oracle
from kvcase import make_tables

pytestmark = pytest.mark.gpu

POISON = 0xFFFF


def _run(skv, k_new, v_new, total_blocks, bs, Hkv, hd, tables, positions, tokens_per_seq,
         offsets=None):
    B = tables.shape[0]
    k_pool = np.full((total_blocks, bs, Hkv, hd), POISON, np.uint16)
    v_pool = k_pool.copy()
    dk = skv.DeviceBuffer.from_numpy(k_pool)
    dv = skv.DeviceBuffer.from_numpy(v_pool)
    dkn = skv.DeviceBuffer.from_numpy(k_new)
    dvn = skv.DeviceBuffer.from_numpy(v_new)
    dt = skv.DeviceBuffer.from_numpy(tables)
    dp = skv.DeviceBuffer.from_numpy(np.asarray(positions, np.int32))
    do = None if offsets is None else skv.DeviceBuffer.from_numpy(np.asarray(offsets, np.int32))
    src = skv.DTYPE_FP32 if k_new.dtype == np.float32 else skv.DTYPE_BF16
    skv.kv_append(dkn, dvn, src, dk, dv, total_blocks, dt, tables.shape[1], dp, B, tokens_per_seq,
                  Hkv, hd, bs, token_offsets=do)
    skv.synchronize()
    got_k = dk.download(np.uint16, k_pool.shape)
    got_v = dv.download(np.uint16, v_pool.shape)
    oracle.kv_append(k_new, v_new, k_pool, v_pool, tables, positions, B, tokens_per_seq, Hkv, hd,
                     bs, offsets=offsets)
    return got_k, got_v, k_pool, v_pool


def _bits_equal(got, ref, what):
    diff = np.flatnonzero(got.reshape(-1) != ref.reshape(-1))
    assert diff.size == 0, f"{what}: {diff.size} elements differ, first at flat index {diff[0]}"


@pytest.mark.parametrize("geom", [(4, 64), (8, 128), (2, 96), (3, 20)], ids=["tl", "l3", "hd96", "odd"])
@pytest.mark.parametrize("src", ["bf16", "fp32"])
def test_decode_append_one_token_per_sequence(gpu, geom, src):
    Hkv, hd = geom
    bs = 16
    rng = np.random.default_rng(hd)
    lens = rng.integers(1, 300, size=24)
    total = int(sum(-(-int(L) // bs) for L in lens)) + 5
    tables = make_tables(lens, bs, total, "random", rng)
    positions = (lens - 1).astype(np.int32)  # write the last slot of each context
    if src == "bf16":
        k_new = rng.integers(0, 0x10000, size=(24, Hkv * hd), dtype=np.uint16)
        v_new = rng.integers(0, 0x10000, size=(24, Hkv * hd), dtype=np.uint16)
    else:
        k_new = rng.standard_normal((24, Hkv * hd), dtype=np.float32)
        v_new = rng.standard_normal((24, Hkv * hd), dtype=np.float32)
    gk, gv, rk, rv = _run(gpu, k_new, v_new, total, bs, Hkv, hd, tables, positions, 1)
    _bits_equal(gk, rk, "K")
    _bits_equal(gv, rv, "V")


def test_fp32_rounding_edge_patterns(gpu):
    """Ties, carries into the exponent, infinities and NaN payloads follow the
    reference's set_value rule bit for bit."""
    Hkv, hd, bs = 8, 128, 16
    uppers = np.array([0x0000, 0x0001, 0x3F80, 0x3F81, 0x7F7F, 0x7F80, 0x7FC0, 0x8000, 0xFF7F,
                       0xFFFF, 0x007F, 0x4049], np.uint32)
    lowers = np.array([0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF], np.uint32)
    bits = (uppers[:, None] << 16 | lowers[None, :]).reshape(-1)
    row = np.resize(bits, Hkv * hd).astype(np.uint32).view(np.float32)
    k_new = np.stack([row, row[::-1].copy()]).astype(np.float32)
    v_new = k_new[::-1].copy()
    tables = np.array([[3, 1], [0, 2]], np.int32)
    gk, gv, rk, rv = _run(gpu, k_new, v_new, 4, bs, Hkv, hd, tables, [17, 5], 1)
    _bits_equal(gk, rk, "K")
    _bits_equal(gv, rv, "V")


def test_chunk_append_prefill_blocks(gpu):
    """Config-5-shaped chunk append: 4 sequences x 2048 tokens, Hkv 8, hd 128,
    into non-monotone tables (reused blocks)."""
    Hkv, hd, bs, T = 8, 128, 16, 2048
    rng = np.random.default_rng(5)
    total = 4 * (T // bs) + 64
    tables = make_tables([T] * 4, bs, total, "random", rng)
    k_new = rng.integers(0, 0x10000, size=(4 * T, Hkv * hd), dtype=np.uint16)
    v_new = rng.integers(0, 0x10000, size=(4 * T, Hkv * hd), dtype=np.uint16)
    gk, gv, rk, rv = _run(gpu, k_new, v_new, total, bs, Hkv, hd, tables, [0, 0, 0, 0], T)
    _bits_equal(gk, rk, "K")
    _bits_equal(gv, rv, "V")


def test_ragged_offsets_and_mid_block_start(gpu):
    Hkv, hd, bs = 4, 64, 16
    rng = np.random.default_rng(8)
    counts = np.array([5, 0, 40, 16, 1], np.int32)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    starts = np.array([3, 10, 15, 32, 0], np.int32)
    lens = starts + counts
    total = 40
    tables = make_tables(np.maximum(lens, 1), bs, total, "random", rng)
    rows = int(offsets[-1])
    k_new = rng.integers(0, 0x10000, size=(rows, Hkv * hd), dtype=np.uint16)
    v_new = rng.integers(0, 0x10000, size=(rows, Hkv * hd), dtype=np.uint16)
    gk, gv, rk, rv = _run(gpu, k_new, v_new, total, bs, Hkv, hd, tables, starts, int(counts.max()),
                          offsets=offsets)
    _bits_equal(gk, rk, "K")
    _bits_equal(gv, rv, "V")


def test_positions_outside_table_are_not_written(gpu):
    Hkv, hd, bs = 4, 64, 16
    tables = np.array([[2, -1], [7, 1]], np.int32)   # -1: no block for page 1
    rng = np.random.default_rng(3)
    k_new = rng.integers(0, 0x10000, size=(2 * 20, Hkv * hd), dtype=np.uint16)
    v_new = k_new.copy()
    gk, gv, rk, rv = _run(gpu, k_new, v_new, 8, bs, Hkv, hd, tables, [0, 10], 20)
    _bits_equal(gk, rk, "K")
    _bits_equal(gv, rv, "V")


@pytest.mark.parametrize("seed", range(16))
def test_random_ragged_appends(gpu, seed):
    """Seeded random cases: kv geometry (odd head dims included), batch, each
    sequence's start position and token count (ragged offsets, some empty),
    bf16 or fp32 source, and tables with entries outside the pool."""
    rng = np.random.default_rng(700 + seed)
    Hkv, hd = [(4, 64), (8, 128), (2, 96), (3, 20), (1, 128), (8, 64)][rng.integers(0, 6)]
    bs = 16
    B = int(rng.integers(1, 9))
    counts = rng.choice([0, 1, 2, 15, 16, 17, 40, 100], B).astype(np.int32)
    starts = rng.choice([0, 1, 15, 16, 17, 100, 255], B).astype(np.int32)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    lens = np.maximum(starts + counts, 1)
    total = sum(-(-int(L) // bs) for L in lens) + 9
    tables = make_tables(lens, bs, total, "random", rng, extra_cols=int(rng.integers(0, 3)))
    for _ in range(int(rng.integers(0, 4))):    # entries outside the pool: those rows are skipped
        tables[rng.integers(0, B), rng.integers(0, tables.shape[1])] = int(rng.choice([-1, total, total + 5]))
    rows = max(int(offsets[-1]), 1)
    if rng.random() < 0.5:
        k_new = rng.standard_normal((rows, Hkv * hd), dtype=np.float32)
        v_new = rng.standard_normal((rows, Hkv * hd), dtype=np.float32)
    else:
        k_new = rng.integers(0, 0x10000, size=(rows, Hkv * hd), dtype=np.uint16)
        v_new = rng.integers(0, 0x10000, size=(rows, Hkv * hd), dtype=np.uint16)
    gk, gv, rk, rv = _run(gpu, k_new, v_new, total, bs, Hkv, hd, tables, starts, int(max(counts.max(), 1)),
                          offsets=offsets)
    _bits_equal(gk, rk, f"seed {seed} K")
    _bits_equal(gv, rv, f"seed {seed} V")
