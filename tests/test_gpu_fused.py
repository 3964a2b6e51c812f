"""Fused append + decode (skv_paged_decode_append, skv_paged_attention_decode_append).

Contract: one call equals skv_kv_append at positions context_lens - 1 followed
by skv_paged_decode, bit for bit (pools and outputs), including the positions
both skip.  Each case runs both ways on the GPU from the same starting pools,
and is also checked against the oracle: pools bit-exact against the oracle's
scatter, outputs within 2e-3 + 1e-2 |ref| of the oracle's fp32 loops over the
appended pools.
"""
import math

import numpy as np
import pytest

import oracle
from kvcase import assert_close, bf16_normal, make_tables

pytestmark = pytest.mark.gpu


def _case(Hq, Hkv, hd, bs, lens, kv_dtype, q_dtype, seed, max_blocks=None, bad_last=()):
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, np.int32)
    need = sum(max(0, -(-int(L) // bs)) for L in lens)
    total = need + 9
    tables = make_tables(lens, bs, total, "random", rng)
    if max_blocks is not None:
        tables = np.ascontiguousarray(tables[:, :max_blocks])
    for b in bad_last:  # last block outside the pool: append and block both skipped
        nb = -(-int(lens[b]) // bs)
        tables[b, nb - 1] = total + 3
    B = len(lens)
    k_pool = bf16_normal(rng, (total, bs, Hkv, hd))
    v_pool = bf16_normal(rng, (total, bs, Hkv, hd))
    if kv_dtype == "bf16":
        k_new = bf16_normal(rng, (B, Hkv, hd))
        v_new = bf16_normal(rng, (B, Hkv, hd))
    else:
        k_new = rng.standard_normal((B, Hkv, hd), dtype=np.float32)
        v_new = rng.standard_normal((B, Hkv, hd), dtype=np.float32)
    q32 = rng.standard_normal((B, Hq, hd), dtype=np.float32)
    q_dev = oracle.f32_to_bf16(q32) if q_dtype == "bf16" else q32
    q_ref = oracle.bf16_to_f32(q_dev) if q_dtype == "bf16" else q32
    return dict(Hq=Hq, Hkv=Hkv, hd=hd, bs=bs, lens=lens, total=total, tables=tables,
                k_pool=k_pool, v_pool=v_pool, k_new=k_new, v_new=v_new, q_dev=q_dev,
                q_ref=q_ref, kv_dtype=kv_dtype, q_dtype=q_dtype, scale=1.0 / math.sqrt(hd))


def _run(skv, c, fused, misalign=False):
    B = len(c["lens"])
    dk = skv.DeviceBuffer.from_numpy(c["k_pool"])
    dv = skv.DeviceBuffer.from_numpy(c["v_pool"])
    dt = skv.DeviceBuffer.from_numpy(c["tables"])
    dl = skv.DeviceBuffer.from_numpy(c["lens"])
    dq = skv.DeviceBuffer.from_numpy(c["q_dev"])
    kvd = skv.DTYPE_BF16 if c["kv_dtype"] == "bf16" else skv.DTYPE_FP32
    qd = skv.DTYPE_BF16 if c["q_dtype"] == "bf16" else skv.DTYPE_FP32
    shift = 2 if misalign else 0  # new rows 2 bytes past a 16-byte boundary
    raw_k = np.frombuffer(c["k_new"].tobytes(), np.uint8)
    raw_v = np.frombuffer(c["v_new"].tobytes(), np.uint8)
    dkn = skv.DeviceBuffer(raw_k.size + 16)
    dvn = skv.DeviceBuffer(raw_v.size + 16)
    dkn.upload(np.concatenate([np.zeros(shift, np.uint8), raw_k, np.zeros(16 - shift, np.uint8)]))
    dvn.upload(np.concatenate([np.zeros(shift, np.uint8), raw_v, np.zeros(16 - shift, np.uint8)]))
    kn_ptr, vn_ptr = dkn.ptr + shift, dvn.ptr + shift
    out_shape = (B, c["Hq"], c["hd"])
    dout = skv.DeviceBuffer(4 * int(np.prod(out_shape)))
    dout.upload(np.full(out_shape, np.nan, np.float32))
    ws, wsb = skv.decode_workspace(B, c["Hq"], c["Hkv"], c["hd"])
    mb = c["tables"].shape[1]
    if fused:
        skv.paged_decode_append(dq, qd, kn_ptr, vn_ptr, kvd, dk, dv, c["total"], dt, mb, dl, B,
                                c["Hq"], c["Hkv"], c["hd"], c["bs"], c["scale"], dout, ws, wsb)
    else:
        dp = skv.DeviceBuffer.from_numpy((c["lens"] - 1).astype(np.int32))
        skv.kv_append(kn_ptr, vn_ptr, kvd, dk, dv, c["total"], dt, mb, dp, B, 1, c["Hkv"], c["hd"],
                      c["bs"])
        skv.paged_decode(dq, qd, dk, dv, c["total"], dt, mb, dl, B, c["Hq"], c["Hkv"], c["hd"],
                         c["bs"], c["scale"], dout, ws, wsb)
    skv.synchronize()
    return (dout.download(np.float32, out_shape), dk.download(np.uint16, c["k_pool"].shape),
            dv.download(np.uint16, c["v_pool"].shape))


def _check(skv, c, what, misalign=False, no_oracle=()):
    """no_oracle: sequences with a block outside the pool or a context past the
    table, which the reference (and so the oracle's attention) rejects; for them
    only the pools and the fused == separate equality are checked."""
    out_f, k_f, v_f = _run(skv, c, fused=True, misalign=misalign)
    out_s, k_s, v_s = _run(skv, c, fused=False, misalign=misalign)
    assert np.array_equal(k_f, k_s) and np.array_equal(v_f, v_s), f"{what}: pools differ"
    assert np.array_equal(out_f.view(np.uint32), out_s.view(np.uint32)), f"{what}: outputs differ"
    # Oracle: the same scatter on the CPU, then the reference's loops.
    B = len(c["lens"])
    k_ref, v_ref = c["k_pool"].copy(), c["v_pool"].copy()
    row = c["Hkv"] * c["hd"]
    oracle.kv_append(c["k_new"].reshape(B, row), c["v_new"].reshape(B, row), k_ref, v_ref,
                     c["tables"], c["lens"] - 1, B, 1, c["Hkv"], c["hd"], c["bs"])
    assert np.array_equal(k_f, k_ref) and np.array_equal(v_f, v_ref), f"{what}: pools vs oracle"
    sel = np.array([b for b in range(B) if b not in no_oracle])
    ref = oracle.paged_decode(c["q_ref"][sel], k_ref, v_ref, c["tables"][sel], c["lens"][sel],
                              c["Hkv"], c["bs"], c["scale"])
    return assert_close(out_f[sel], ref, what=what)


@pytest.mark.parametrize("geom", [(32, 4, 64), (32, 8, 128), (64, 8, 128), (8, 2, 64), (8, 8, 64)],
                         ids=["tl", "l3", "l70", "g4_hkv2", "mha"])
@pytest.mark.parametrize("kv_dtype", ["bf16", "fp32"])
def test_fused_matches_append_then_decode(gpu, geom, kv_dtype):
    Hq, Hkv, hd = geom
    lens = [1, 2, 15, 16, 17, 31, 32, 33, 300, 1024, 2049, 4097]
    c = _case(Hq, Hkv, hd, 16, lens, kv_dtype, "bf16", seed=hd * 7 + Hq)
    _check(gpu, c, f"geom={geom} kv={kv_dtype}")


@pytest.mark.parametrize("q_dtype", ["bf16", "fp32"])
def test_fused_skipped_positions(gpu, q_dtype):
    """Zero/negative lengths, a last block outside the pool, and contexts longer
    than the table are skipped exactly as the separate append skips them."""
    lens = [0, 40, -3, 16, 200, 1, 999]
    c = _case(32, 8, 128, 16, lens, "bf16", q_dtype, seed=5, bad_last=(3,), max_blocks=40)
    # Sequence 6 needs 63 blocks but the table has 40: its position is past the table.
    _check(gpu, c, f"skips q={q_dtype}", no_oracle=(3, 6))


@pytest.mark.parametrize("geom", [(32, 4, 64), (32, 8, 128)], ids=["tl", "l3"])
def test_fused_short_tables(gpu, geom):
    """Short tables (one workgroup per kv head, blocks split over its
    wavefronts): the new row lands in whichever wavefront holds the last
    block; skipped positions as in the separate append."""
    Hq, Hkv, hd = geom
    cap_blocks = 12 if hd == 64 else 8
    lens = [1, 16, 17, 33, 48, 49, 16 * cap_blocks, 0, 40, 16 * cap_blocks + 5]
    c = _case(Hq, Hkv, hd, 16, lens, "fp32", "fp32", seed=hd + 1, bad_last=(8,), max_blocks=cap_blocks)
    # Sequence 9 needs one more block than the table has: its position is past the table.
    _check(gpu, c, f"short tables {geom}", no_oracle=(8, 9))


def test_fused_generic_path_and_misaligned_rows(gpu):
    """Shapes outside the MFMA kernel, and new rows not 16-byte aligned, take the
    append kernel before the decode; the result is the same contract."""
    c = _case(12, 4, 64, 8, [5, 70, 513, 9], "bf16", "bf16", seed=21)
    _check(gpu, c, "generic bs=8")
    c = _case(32, 8, 128, 16, [5, 70, 513, 9], "bf16", "bf16", seed=22)
    _check(gpu, c, "misaligned rows", misalign=True)


def test_fused_batch_above_one_launch(gpu):
    """More than 4,096 sequences run as consecutive launches; the new rows of
    every chunk are offset with it."""
    rng = np.random.default_rng(3)
    lens = rng.integers(1, 40, size=4100).astype(np.int32)
    c = _case(8, 4, 64, 16, lens, "fp32", "bf16", seed=23)
    _check(gpu, c, "B=4100")


@pytest.mark.parametrize("L", [1, 16, 17, 100, 4097])
def test_single_sequence_fused_entry(gpu, L):
    """skv_paged_attention_decode_append == skv_kv_append_token + skv_paged_attention_decode."""
    Hq, Hkv, hd, bs = 32, 4, 64, 16
    rng = np.random.default_rng(L)
    nb = -(-L // bs)
    total = nb + 4
    table = rng.permutation(total)[:nb].astype(np.int32)
    k_pool = bf16_normal(rng, (total, bs, Hkv, hd))
    v_pool = bf16_normal(rng, (total, bs, Hkv, hd))
    k_row = rng.standard_normal((Hkv, hd), dtype=np.float32)
    v_row = rng.standard_normal((Hkv, hd), dtype=np.float32)
    q = rng.standard_normal((Hq, hd), dtype=np.float32)
    scale = 1.0 / math.sqrt(hd)
    results = []
    for fused in (True, False):
        dk, dv = gpu.DeviceBuffer.from_numpy(k_pool), gpu.DeviceBuffer.from_numpy(v_pool)
        dt = gpu.DeviceBuffer.from_numpy(table)
        dq = gpu.DeviceBuffer.from_numpy(q)
        dkr, dvr = gpu.DeviceBuffer.from_numpy(k_row), gpu.DeviceBuffer.from_numpy(v_row)
        dout = gpu.DeviceBuffer(4 * Hq * hd)
        ws, wsb = gpu.single_decode_workspace(Hq, Hkv, hd)
        if fused:
            gpu.paged_attention_decode_append(dq, dkr, dvr, gpu.DTYPE_FP32, dk, dv, total, dt, dout,
                                              L, bs, Hq, Hkv, hd, scale, ws, wsb)
        else:
            gpu._check(gpu.lib().skv_kv_append_token(dkr.ptr, dvr.ptr, gpu.DTYPE_FP32, dk.ptr,
                                                     dv.ptr, total, dt.ptr, nb, L - 1, Hkv, hd, bs,
                                                     None))
            gpu.paged_attention_decode(dq, dk, dv, total, dt, dout, L, bs, Hq, Hkv, hd, scale, ws,
                                       wsb)
        gpu.synchronize()
        results.append((dout.download(np.float32, (Hq, hd)), dk.download(np.uint16, k_pool.shape),
                        dv.download(np.uint16, v_pool.shape)))
    (o1, k1, v1), (o2, k2, v2) = results
    assert np.array_equal(k1, k2) and np.array_equal(v1, v2)
    assert np.array_equal(o1.view(np.uint32), o2.view(np.uint32))
    k_ref, v_ref = k_pool.copy(), v_pool.copy()
    oracle.kv_append(k_row.reshape(1, -1), v_row.reshape(1, -1), k_ref, v_ref, table[None, :],
                     np.array([L - 1], np.int32), 1, 1, Hkv, hd, bs)
    ref = oracle.paged_decode(q[None], k_ref, v_ref, table[None, :], np.array([L], np.int32), Hkv,
                              bs, scale)
    assert_close(o1[None], ref, what=f"single fused L={L}")
