"""Seeded random decode cases against the oracle: geometry, batch size, context
length distribution (uniform, log-normal, many empty or one-block sequences)
and table width (both sides of the 16-block short-table limit) drawn per seed,
so the stream-K split meets range boundaries at every kind of position: inside
a segment, among the empty slots it puts before a segment's blocks, on a
segment's first block, with empty sequences in between.  Each case also runs
as the fused append + decode and must equal the separate append then decode
bit for bit.

Tolerance: |gpu - ref| <= 2e-3 + 1e-2 * |ref| (the decode tests' bound).
"""
import numpy as np
import pytest

import oracle
from kvcase import assert_close, bf16_normal, make_tables

pytestmark = pytest.mark.gpu

GEOMS = [(32, 4, 64), (32, 8, 128), (64, 8, 128), (8, 2, 64), (16, 16, 64), (32, 32, 128), (8, 1, 128)]


def _lens(rng, B):
    kind = rng.integers(0, 4)
    if kind == 0:
        lens = rng.integers(1, 600, B)
    elif kind == 1:
        lens = np.clip(np.exp(rng.normal(np.log(300), 1.0, B)), 1, 5000).astype(np.int64)
    elif kind == 2:
        lens = rng.integers(0, 40, B)            # one to three blocks, many empty
    else:
        lens = rng.choice([0, 1, 15, 16, 17, 31, 32, 33, 255, 256, 257], B)
    lens[rng.random(B) < 0.1] = 0
    return lens.astype(np.int32)


def _case(seed):
    rng = np.random.default_rng(1000 + seed)
    Hq, Hkv, hd = GEOMS[rng.integers(0, len(GEOMS))]
    B = int(rng.choice([1, 2, 5, 17, 64, 130, 300]))
    lens = _lens(rng, B)
    block_bytes = 16 * Hkv * hd * 2
    while sum(-(-int(L) // 16) for L in lens if L > 0) * block_bytes > (48 << 20):   # keep each pool small
        lens //= 2
    need = [0 if L <= 0 else -(-int(L) // 16) for L in lens]
    extra = int(rng.choice([0, 1, 20]))
    total = sum(need) + 11
    tables = make_tables(lens, 16, total, "random", rng, extra_cols=extra)
    k_pool = bf16_normal(rng, (total, 16, Hkv, hd))
    v_pool = bf16_normal(rng, (total, 16, Hkv, hd))
    q = oracle.f32_to_bf16(rng.standard_normal((B, Hq, hd), dtype=np.float32))
    k_new = bf16_normal(rng, (B, Hkv, hd))
    v_new = bf16_normal(rng, (B, Hkv, hd))
    return dict(Hq=Hq, Hkv=Hkv, hd=hd, B=B, lens=lens, total=total, tables=tables, k_pool=k_pool,
                v_pool=v_pool, q=q, k_new=k_new, v_new=v_new, scale=1.0 / np.sqrt(hd))


def _run(skv, c, fused):
    D = skv.DeviceBuffer
    dk, dv = D.from_numpy(c["k_pool"]), D.from_numpy(c["v_pool"])
    dt, dl, dq = D.from_numpy(c["tables"]), D.from_numpy(c["lens"]), D.from_numpy(c["q"])
    dkn, dvn = D.from_numpy(c["k_new"]), D.from_numpy(c["v_new"])
    shape = (c["B"], c["Hq"], c["hd"])
    dout = D.from_numpy(np.full(shape, np.nan, np.float32))
    ws, wsb = skv.decode_workspace(c["B"], c["Hq"], c["Hkv"], c["hd"])
    mb = c["tables"].shape[1]
    args = (c["Hq"], c["Hkv"], c["hd"], 16, c["scale"], dout, ws, wsb)
    if fused:
        skv.paged_decode_append(dq, skv.DTYPE_BF16, dkn, dvn, skv.DTYPE_BF16, dk, dv, c["total"], dt, mb, dl,
                                c["B"], *args)
    else:
        dp = D.from_numpy((c["lens"] - 1).astype(np.int32))
        skv.kv_append(dkn, dvn, skv.DTYPE_BF16, dk, dv, c["total"], dt, mb, dp, c["B"], 1, c["Hkv"], c["hd"], 16)
        skv.paged_decode(dq, skv.DTYPE_BF16, dk, dv, c["total"], dt, mb, dl, c["B"], *args)
    skv.synchronize()
    return dout.download(np.float32, shape), dk.download(np.uint16, c["k_pool"].shape), \
        dv.download(np.uint16, c["v_pool"].shape)


@pytest.mark.parametrize("seed", range(64))
def test_random_decode_case(gpu, seed):
    c = _case(seed)
    what = (f"seed={seed} geom=({c['Hq']},{c['Hkv']},{c['hd']}) B={c['B']} table width={c['tables'].shape[1]} "
            f"lens {int(c['lens'].min())}..{int(c['lens'].max())}")
    out_f, k_f, v_f = _run(gpu, c, fused=True)
    out_s, k_s, v_s = _run(gpu, c, fused=False)
    assert np.array_equal(k_f, k_s) and np.array_equal(v_f, v_s), f"{what}: pools differ"
    assert np.array_equal(out_f.view(np.uint32), out_s.view(np.uint32)), f"{what}: fused != separate"
    k_ref, v_ref = c["k_pool"].copy(), c["v_pool"].copy()
    row = c["Hkv"] * c["hd"]
    oracle.kv_append(c["k_new"].reshape(c["B"], row), c["v_new"].reshape(c["B"], row), k_ref, v_ref, c["tables"],
                     c["lens"] - 1, c["B"], 1, c["Hkv"], c["hd"], 16)
    assert np.array_equal(k_f, k_ref) and np.array_equal(v_f, v_ref), f"{what}: pools vs oracle"
    ref = oracle.paged_decode(oracle.bf16_to_f32(c["q"]), k_ref, v_ref, c["tables"], c["lens"], c["Hkv"], 16,
                              c["scale"])
    assert_close(out_f, ref, what=what)
