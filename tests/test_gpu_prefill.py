"""Chunked prefill attention on the GPU (skv_paged_prefill, through the C ABI)
against the oracle (oracle.paged_prefill: the reference's per-token causal
loops of src/layers/attention.cpp:263-337, pinned in test_oracle_prefill.py
against the reference's own chunked PagedAttention::forward).

Tolerance: |gpu - ref| <= 2e-3 + 1e-2 * |ref| (fp32 accumulation on the GPU,
bf16 K/V; P.V on the matrix cores in fp16, V above the fp16 range recomputed
in fp32).
Outputs start as NaN so a missing store fails; unused slots of the last block
hold NaN so a key past the chunk that leaked into P.V fails too.
"""
import math

import numpy as np
import pytest

import oracle
from kvcase import assert_close, bf16_normal, make_tables

pytestmark = pytest.mark.gpu

NAN_BF16 = 0x7FC0


def _case(Hq, Hkv, hd, bs, ctx, chunk, q_dtype="bf16", seed=0, layout="random"):
    rng = np.random.default_rng(seed)
    lens = np.asarray(ctx, np.int32)
    chunk = np.asarray(chunk, np.int64)
    offsets = np.concatenate([[0], np.cumsum(chunk)]).astype(np.int32)
    total = sum(-(-int(L) // bs) for L in lens) + 5
    tables = make_tables(lens, bs, total, layout, rng)
    kp = bf16_normal(rng, (total, bs, Hkv, hd))
    vp = bf16_normal(rng, (total, bs, Hkv, hd))
    for b, L in enumerate(lens):  # poison the slots past each context
        nb = -(-int(L) // bs)
        if nb and L % bs:
            kp[tables[b, nb - 1], L % bs:] = NAN_BF16
            vp[tables[b, nb - 1], L % bs:] = NAN_BF16
    N = int(offsets[-1])
    q32 = rng.standard_normal((N, Hq, hd), dtype=np.float32)
    q_dev = oracle.f32_to_bf16(q32) if q_dtype == "bf16" else q32
    q_ref = oracle.bf16_to_f32(q_dev) if q_dtype == "bf16" else q32
    return dict(Hq=Hq, Hkv=Hkv, hd=hd, bs=bs, lens=lens, offsets=offsets, total=total,
                tables=tables, kp=kp, vp=vp, q_dev=q_dev, q_ref=q_ref, q_dtype=q_dtype, N=N,
                scale=1.0 / math.sqrt(hd))


def _gpu(skv, c):
    d = {k: skv.DeviceBuffer.from_numpy(c[k]) for k in ("kp", "vp", "tables", "offsets", "lens", "q_dev")}
    shape = (c["N"], c["Hq"], c["hd"])
    out = skv.DeviceBuffer(4 * max(1, int(np.prod(shape))))
    out.upload(np.full(shape, np.nan, np.float32))
    qd = skv.DTYPE_BF16 if c["q_dtype"] == "bf16" else skv.DTYPE_FP32
    skv.paged_prefill(d["q_dev"], qd, d["kp"], d["vp"], c["total"], d["tables"], c["tables"].shape[1],
                      d["offsets"], d["lens"], len(c["lens"]), c["N"], c["Hq"], c["Hkv"], c["hd"],
                      c["bs"], c["scale"], out)
    skv.synchronize()
    return out.download(np.float32, shape)


def _ref(c, precision="f32"):
    return oracle.paged_prefill(c["q_ref"], c["kp"], c["vp"], c["tables"], c["offsets"], c["lens"],
                                c["Hkv"], c["bs"], c["scale"], precision=precision, threads=8)


CHUNKS = ([1, 5, 17, 64, 100, 33, 7, 16],        # chunk tokens
          [1, 5, 40, 64, 333, 2049, 7, 300])     # contexts (>= chunk)


@pytest.mark.parametrize("geom", [(32, 4, 64), (32, 8, 128), (64, 8, 128), (8, 8, 64), (16, 1, 128),
                                  (8, 4, 128)],
                         ids=["tl", "l3", "l70", "mha", "g16", "g2"])
@pytest.mark.parametrize("q_dtype", ["bf16", "fp32"])
def test_prefill_matches_oracle(gpu, geom, q_dtype):
    Hq, Hkv, hd = geom
    c = _case(Hq, Hkv, hd, 16, CHUNKS[1], CHUNKS[0], q_dtype, seed=hd + Hq)
    got = _gpu(gpu, c)
    assert_close(got, _ref(c), what=f"prefill {geom} q={q_dtype}")
    assert_close(got, _ref(c, "f64"), what=f"prefill {geom} q={q_dtype} vs f64")


@pytest.mark.parametrize("geom,bs", [((12, 4, 64), 8), ((8, 2, 96), 16), ((6, 3, 40), 5)],
                         ids=["bs8", "hd96", "odd"])
def test_prefill_generic_shapes(gpu, geom, bs):
    Hq, Hkv, hd = geom
    c = _case(Hq, Hkv, hd, bs, [9, 70, 200], [9, 30, 3], seed=bs + hd)
    assert_close(_gpu(gpu, c), _ref(c), what=f"generic prefill {geom} bs={bs}")


def test_prefill_last_token_matches_decode(gpu):
    """The last row of each chunk sees the whole context: the decode kernel's
    result for that sequence (different kernels, same tolerance)."""
    c = _case(32, 8, 128, 16, [50, 600, 1024], [20, 64, 3], seed=9)
    got = _gpu(gpu, c)
    B = len(c["lens"])
    last = c["offsets"][1:] - 1
    q_last = c["q_dev"][last]
    dq, dk, dv = (gpu.DeviceBuffer.from_numpy(a) for a in (q_last, c["kp"], c["vp"]))
    dt, dl = gpu.DeviceBuffer.from_numpy(c["tables"]), gpu.DeviceBuffer.from_numpy(c["lens"])
    dout = gpu.DeviceBuffer(4 * B * 32 * 128)
    ws, wsb = gpu.decode_workspace(B, 32, 8, 128)
    gpu.paged_decode(dq, gpu.DTYPE_BF16, dk, dv, c["total"], dt, c["tables"].shape[1], dl, B, 32, 8,
                     128, 16, c["scale"], dout, ws, wsb)
    gpu.synchronize()
    dec = dout.download(np.float32, (B, 32, 128))
    assert_close(got[last], dec, what="last chunk row vs decode")


def test_prefill_long_chunk_sampled(gpu):
    """A cfg5-shaped chunk: 2,048 new tokens after 2,048 + 9 earlier ones, L70
    geometry, non-monotone table; 24 rows checked against the oracle."""
    c = _case(64, 8, 128, 16, [4105, 2048], [2048, 2048], seed=5, layout="random")
    got = _gpu(gpu, c)
    assert np.isfinite(got).all()
    rng = np.random.default_rng(1)
    rows = sorted(set(rng.choice(c["N"], size=20, replace=False).tolist()) | {0, 2047, 2048, 4095})
    seqs, pos = oracle.prefill_positions(c["offsets"], c["lens"])
    ref = oracle.paged_decode(c["q_ref"][rows], c["kp"], c["vp"], c["tables"][seqs[rows]],
                              (pos[rows] + 1).astype(np.int32), 8, 16, c["scale"], threads=8)
    assert_close(got[rows], ref, what="long chunk rows")


@pytest.mark.parametrize("geom", [(32, 4, 64), (64, 8, 128)], ids=["tl", "l70"])
@pytest.mark.parametrize("q_dtype", ["bf16", "fp32"])
def test_prefill_v_beyond_fp16_range(gpu, geom, q_dtype):
    """V elements the matrix-core P.V cannot take as fp16 (finite bf16 values
    above 65504) in a few keys: the tiles that read them are recomputed in
    fp32, the others keep the fp16 P.V.  65280, the largest bf16 value within
    the fp16 range, takes the fp16 path exactly."""
    Hq, Hkv, hd = geom
    c = _case(Hq, Hkv, hd, 16, CHUNKS[1], CHUNKS[0], q_dtype, seed=hd + 7)
    big = oracle.f32_to_bf16(np.array([1.0e6, -3.0e5, 65280.0, 7.0e4], np.float32))
    assert oracle.bf16_to_f32(big)[2] == 65280.0
    tables = c["tables"]
    # (sequence, key, kv head, dim, value): keys inside each sequence's context
    for b, key, h, d, v in ((5, 3, 0, 1, big[0]), (5, 1500, Hkv - 1, hd - 1, big[1]), (4, 320, 1, 5, big[2]),
                            (6, 6, 0, 0, big[3])):
        assert key < c["lens"][b]
        c["vp"][tables[b, key // 16], key % 16, h, d] = v
    got = _gpu(gpu, c)
    assert_close(got, _ref(c), what=f"prefill with large V {geom} q={q_dtype}")
    assert_close(got, _ref(c, "f64"), what=f"prefill with large V {geom} q={q_dtype} vs f64")


def _ref_skipping_invalid_blocks(c):
    """float64 causal attention over exactly the keys whose block id lies in
    the pool (the kernels skip absent and out-of-pool table entries; the
    oracle, like the reference, refuses them)."""
    seqs, pos = oracle.prefill_positions(c["offsets"], c["lens"])
    G = c["Hq"] // c["Hkv"]
    kp = oracle.bf16_to_f32(c["kp"]).astype(np.float64)
    vp = oracle.bf16_to_f32(c["vp"]).astype(np.float64)
    out = np.zeros((c["N"], c["Hq"], c["hd"]))
    for n in range(c["N"]):
        keys = np.arange(pos[n] + 1)
        blk = c["tables"][seqs[n], keys // c["bs"]].astype(np.int64)
        ok = (blk >= 0) & (blk < c["total"])
        keys, blk = keys[ok], blk[ok]
        for h in range(c["Hq"]):
            kvh = h // G
            K = kp[blk, keys % c["bs"], kvh]
            V = vp[blk, keys % c["bs"], kvh]
            s = K @ c["q_ref"][n, h].astype(np.float64) * c["scale"]
            w = np.exp(s - s.max())
            out[n, h] = (w / w.sum()) @ V
    return out


@pytest.mark.parametrize("geom", [(32, 4, 64), (64, 8, 128)], ids=["tl", "l70"])
def test_prefill_skips_absent_and_out_of_pool_blocks(gpu, geom):
    """Table entries inside a context that are absent (-1) or outside the pool
    are skipped: at the start of a 64-key step (the step's existing keys are
    then not a prefix), at its end, and a sequence's first block."""
    Hq, Hkv, hd = geom
    c = _case(Hq, Hkv, hd, 16, [40, 333, 200], [17, 64, 30], seed=hd + 23)
    # The brute force is the oracle where the oracle applies (no invalid ids).
    assert_close(_ref_skipping_invalid_blocks(c), _ref(c), what="brute force vs oracle")
    t = c["tables"]
    t[1, 4] = -1                     # keys 64..79: the first block of step 1
    t[1, 11] = c["total"] + 7        # keys 176..191: the last block of step 2
    t[1, 16] = -1                    # keys 256..271 (the chunk's diagonal steps)
    t[2, 0] = -1                     # the sequence's first block
    got = _gpu(gpu, c)
    assert_close(got, _ref_skipping_invalid_blocks(c), what=f"prefill with invalid blocks {geom}")
