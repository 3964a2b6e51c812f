"""Pins the oracle's KV append (src/models/transformer_block.cpp:484-509).

Checked against a numpy fancy-index scatter written from the layout formula
element = ((block * bs + slot) * Hkv + h) * hd + d, on poisoned pools, so every
written element lands at its index and nothing else changes.
"""
import numpy as np

import oracle
from kvcase import make_tables


def _numpy_scatter(pool, rows, tables, positions, counts, offsets, bs):
    pool = pool.copy()
    flat = pool.reshape(-1, pool.shape[2] * pool.shape[3])     # [total*bs, Hkv*hd]
    for b, n in enumerate(counts):
        for j in range(n):
            pos = positions[b] + j
            page = pos // bs
            if page >= tables.shape[1] or tables[b, page] < 0 or tables[b, page] >= pool.shape[0]:
                continue
            flat[tables[b, page] * bs + pos % bs] = rows[offsets[b] + j]
    return pool


def test_scatter_matches_layout_formula_bf16_and_fp32():
    rng = np.random.default_rng(0)
    Hkv, hd, bs = 3, 8, 4
    counts = [5, 1, 9]
    positions = np.array([2, 7, 0], np.int32)
    lens = positions + np.array(counts)
    total = 20
    tables = make_tables(lens, bs, total, "random", rng)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    rows16 = rng.integers(0, 0x10000, size=(offsets[-1], Hkv * hd), dtype=np.uint16)
    rows32 = rng.standard_normal((offsets[-1], Hkv * hd), dtype=np.float32)
    for rows, expect_rows in ((rows16, rows16), (rows32, oracle.f32_to_bf16(rows32))):
        kp = np.full((total, bs, Hkv, hd), 0xFFFF, np.uint16)
        vp = kp.copy()
        oracle.kv_append(rows, rows, kp, vp, tables, positions, 3, max(counts), Hkv, hd, bs,
                         offsets=offsets)
        expect = _numpy_scatter(np.full_like(kp, 0xFFFF), expect_rows, tables, positions, counts,
                                offsets, bs)
        np.testing.assert_array_equal(kp, expect)
        np.testing.assert_array_equal(vp, expect)


def test_uniform_layout_equals_ragged_layout():
    rng = np.random.default_rng(1)
    Hkv, hd, bs, T = 2, 4, 4, 6
    tables = make_tables([T, T], bs, 6, "random", rng)
    rows = rng.integers(0, 0x10000, size=(2 * T, Hkv * hd), dtype=np.uint16)
    a = np.zeros((6, bs, Hkv, hd), np.uint16)
    b = a.copy()
    oracle.kv_append(rows, rows, a, a.copy(), tables, [0, 0], 2, T, Hkv, hd, bs)
    oracle.kv_append(rows, rows, b, b.copy(), tables, [0, 0], 2, T, Hkv, hd, bs,
                     offsets=np.array([0, T, 2 * T], np.int32))
    np.testing.assert_array_equal(a, b)
