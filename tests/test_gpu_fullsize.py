"""Parity at BASELINE.json's full sizes (configs 2-5), on device-generated data.

The pools are generated on the GPU (counter-hash N(0,1) bf16) with the same
tables bench.py times.  After one bench step (append of one token per sequence
at its last slot, then decode):
* the step is the fused call bench.py times (append at lens - 1, then decode);
  every output is finite, and a plain decode of the appended pools afterwards
  gives identical bits;
* the appended rows hold exactly the new K/V bits;
* sequences are checked against the oracle -- every sequence of cfg2 and cfg3, a
  seeded sample of 8 plus the shortest and longest of cfg4, 6 of the 32 long
  sequences and all 4 new ones of cfg5: their blocks are gathered on the GPU
  into a compact pool, read back, and the oracle's fp32 loops run over them
  (tolerance 2e-3 + 1e-2|ref|).
"""
import math
import sys

import numpy as np
import pytest

import oracle
from kvcase import assert_close

pytestmark = pytest.mark.gpu


def _bench():
    import bench  # repository root is on sys.path (conftest)

    return bench


def _step(skv, w, seed):
    """Device state for one bench step of workload w; returns buffers and out."""
    B, Hq, Hkv, hd, bs, total = w["B"], w["Hq"], w["Hkv"], w["hd"], w["bs"], w["total"]
    n = total * bs * Hkv * hd
    d = dict(k=skv.DeviceBuffer(n * 2), v=skv.DeviceBuffer(n * 2),
             q=skv.DeviceBuffer(B * Hq * hd * 2), kn=skv.DeviceBuffer(B * Hkv * hd * 2),
             vn=skv.DeviceBuffer(B * Hkv * hd * 2))
    skv.fill_normal_bf16(d["k"], n, seed)
    skv.fill_normal_bf16(d["v"], n, seed + 1)
    skv.fill_normal_bf16(d["q"], B * Hq * hd, seed + 2)
    skv.fill_normal_bf16(d["kn"], B * Hkv * hd, seed + 3)
    skv.fill_normal_bf16(d["vn"], B * Hkv * hd, seed + 4)
    d["t"] = skv.DeviceBuffer.from_numpy(w["tables"])
    d["l"] = skv.DeviceBuffer.from_numpy(w["lens"])
    d["p"] = skv.DeviceBuffer.from_numpy(w["lens"] - 1)
    d["ws"], wsb = skv.decode_workspace(B, Hq, Hkv, hd)
    mb = w["tables"].shape[1]

    def decode(fused=False):
        """fused: the bench step (skv_paged_decode_append: append the new rows
        at lens - 1, then attend); otherwise a plain decode of the pools."""
        out = skv.DeviceBuffer(B * Hq * hd * 4)
        if fused:
            skv.paged_decode_append(d["q"], skv.DTYPE_BF16, d["kn"], d["vn"], skv.DTYPE_BF16,
                                    d["k"], d["v"], total, d["t"], mb, d["l"], B, Hq, Hkv, hd, bs,
                                    1.0 / math.sqrt(hd), out, d["ws"], wsb)
        else:
            skv.paged_decode(d["q"], skv.DTYPE_BF16, d["k"], d["v"], total, d["t"], mb, d["l"], B,
                             Hq, Hkv, hd, bs, 1.0 / math.sqrt(hd), out, d["ws"], wsb)
        skv.synchronize()
        return out.download(np.float32, (B, Hq, hd))

    return d, decode


def _gather(skv, pool, total, table_row, nb, block_elems, shape):
    tbl = skv.DeviceBuffer.from_numpy(np.ascontiguousarray(table_row[:nb], np.int32))
    dst = skv.DeviceBuffer(nb * block_elems * 2)
    skv.gather_blocks(pool, total, tbl, nb, block_elems, dst)
    skv.synchronize()
    return dst.download(np.uint16, (nb,) + shape)


@pytest.mark.parametrize("cfg,n_sample", [(2, 1), (3, 64), (4, 8)])
def test_full_size_config(gpu, cfg, n_sample):
    bench = _bench()
    w = bench.workload(cfg)
    B, Hq, Hkv, hd, bs, total = w["B"], w["Hq"], w["Hkv"], w["hd"], w["bs"], w["total"]
    print(f"cfg{cfg}: B={B} contexts {int(w['lens'].min())}..{int(w['lens'].max())}", flush=True)
    d, decode = _step(gpu, w, seed=0x5EED0000 + 17 * cfg)
    out = decode(fused=True)
    assert np.isfinite(out).all()
    # A plain decode of the appended pools gives the same bits: the fused
    # append stored exactly the rows it attended to, and the kernel is
    # deterministic.
    assert np.array_equal(out, decode()), "fused step and plain decode differ"

    rng = np.random.default_rng(cfg)
    lens = w["lens"]
    pick = set(rng.choice(B, size=min(n_sample, B), replace=False).tolist())
    pick |= {int(np.argmin(lens)), int(np.argmax(lens))}
    q = d["q"].download(np.uint16, (B, Hq, hd))
    kn = d["kn"].download(np.uint16, (B, Hkv, hd))
    vn = d["vn"].download(np.uint16, (B, Hkv, hd))
    for b in sorted(pick):
        L = int(lens[b])
        nb = -(-L // bs)
        kp = _gather(gpu, d["k"], total, w["tables"][b], nb, bs * Hkv * hd, (bs, Hkv, hd))
        vp = _gather(gpu, d["v"], total, w["tables"][b], nb, bs * Hkv * hd, (bs, Hkv, hd))
        # The appended row sits at the last slot, bit for bit.
        assert np.array_equal(kp[(L - 1) // bs, (L - 1) % bs], kn[b]), f"K append seq {b}"
        assert np.array_equal(vp[(L - 1) // bs, (L - 1) % bs], vn[b]), f"V append seq {b}"
        ref = oracle.paged_decode(oracle.bf16_to_f32(q[b:b + 1]), kp, vp,
                                  np.arange(nb, dtype=np.int32)[None, :], np.array([L], np.int32),
                                  Hkv, bs, 1.0 / math.sqrt(hd), threads=8)
        err = assert_close(out[b:b + 1], ref, what=f"cfg{cfg} seq {b} (L={L})")
        print(f"  seq {b:3d} L={L:6d} max abs err {err:.2e}", flush=True)


def test_full_size_churn_config5(gpu):
    """cfg5 after one churn step: 4 new sequences' 2,048-token prefill chunks
    land bit-exact in LIFO-reused (non-monotone) blocks; decode over the 32
    long (131,072) and 4 new sequences matches the oracle on a sample."""
    bench = _bench()
    w = bench.churn_workload(1)
    B, Hq, Hkv, hd, bs, total = w["B"], w["Hq"], w["Hkv"], w["hd"], w["bs"], w["total"]
    nl, nn, chunk = bench.CHURN_LONG, bench.CHURN_NEW, bench.CHURN_CHUNK
    row = Hkv * hd
    mb = w["tables"].shape[1]
    t_new = w["tables"][nl:]
    assert any(np.any(np.diff(r[: chunk // bs]) < 0) for r in t_new), "churn tables are monotone"
    d, decode = _step(gpu, dict(w, lens=w["lens"]), seed=0x5EED0055)
    # The prefill chunks at positions 0..2,047 of the new sequences first, then
    # the fused step appends one decode token per sequence at lens - 1 (the
    # churn rows' position 2,048) and decodes, as in bench.py.
    ck = gpu.DeviceBuffer(nn * chunk * row * 2)
    cv = gpu.DeviceBuffer(nn * chunk * row * 2)
    gpu.fill_normal_bf16(ck, nn * chunk * row, 77)
    gpu.fill_normal_bf16(cv, nn * chunk * row, 78)
    zero = gpu.DeviceBuffer.from_numpy(np.zeros(nn, np.int32))
    gpu.kv_append(ck, cv, gpu.DTYPE_BF16, d["k"], d["v"], total, d["t"].ptr + nl * mb * 4, mb, zero,
                  nn, chunk, Hkv, hd, bs)
    out = decode(fused=True)
    assert np.isfinite(out).all()
    q = d["q"].download(np.uint16, (B, Hq, hd))
    kc = ck.download(np.uint16, (nn, chunk // bs, bs, Hkv, hd))
    vc = cv.download(np.uint16, (nn, chunk // bs, bs, Hkv, hd))
    rng = np.random.default_rng(5)
    pick = sorted(set(rng.choice(nl, size=6, replace=False).tolist()) | set(range(nl, B)))
    for b in pick:
        L = int(w["lens"][b])
        nb = -(-L // bs)
        kp = _gather(gpu, d["k"], total, w["tables"][b], nb, bs * row, (bs, Hkv, hd))
        vp = _gather(gpu, d["v"], total, w["tables"][b], nb, bs * row, (bs, Hkv, hd))
        if b >= nl:
            j = b - nl
            assert np.array_equal(kp[: chunk // bs], kc[j]), f"chunk K of new sequence {j}"
            assert np.array_equal(vp[: chunk // bs], vc[j]), f"chunk V of new sequence {j}"
        ref = oracle.paged_decode(oracle.bf16_to_f32(q[b:b + 1]), kp, vp,
                                  np.arange(nb, dtype=np.int32)[None, :], np.array([L], np.int32),
                                  Hkv, bs, 1.0 / math.sqrt(hd), threads=8)
        err = assert_close(out[b:b + 1], ref, what=f"cfg5 seq {b} (L={L})")
        print(f"  seq {b:3d} L={L:6d} max abs err {err:.2e}", flush=True)
