"""Attention with o_proj + residual folded into one launch
(skv_paged_decode_append_oproj).

Contract: the context, the projected output and the pools are bit-identical
to skv_paged_decode_append (fp32 q and new rows, one sequence) followed by
skv_linear_residual_f32 on the same inputs; the context is also checked
against the oracle's attention over the oracle's appended pools (2e-3 +
1e-2 |ref|, the decode tests' bound).  Shapes outside the folded kernels
return SKV_ERR_UNSUPPORTED and leave every output untouched.
"""
import math

import numpy as np
import pytest

import oracle
from kvcase import assert_close, bf16_normal, make_tables

pytestmark = pytest.mark.gpu

BS = 16


def _case(Hq, Hkv, hd, H, L, mb, seed, with_bias, pad=0):
    rng = np.random.default_rng(seed)
    total = 40
    tables = make_tables([L], BS, total, "random", rng, extra_cols=16)[:, :mb].copy()
    K = Hq * hd
    w = oracle.f32_to_bf16((0.05 * rng.standard_normal((H, K + pad))).astype(np.float32))
    return dict(Hq=Hq, Hkv=Hkv, hd=hd, H=H, K=K, L=L, mb=mb, total=total, tables=tables,
                k_pool=bf16_normal(rng, (total, BS, Hkv, hd)), v_pool=bf16_normal(rng, (total, BS, Hkv, hd)),
                q=rng.standard_normal((1, Hq, hd), dtype=np.float32),
                k_new=rng.standard_normal((1, Hkv, hd), dtype=np.float32),
                v_new=rng.standard_normal((1, Hkv, hd), dtype=np.float32),
                w=w, stride_n=K + pad,
                bias=rng.standard_normal(H).astype(np.float32) if with_bias else None,
                res=rng.standard_normal(H).astype(np.float32), scale=1.0 / math.sqrt(hd))


def _run(skv, c, folded, alias=False, expect=0):
    D, lib = skv.DeviceBuffer, skv.lib()
    dk, dv = D.from_numpy(c["k_pool"]), D.from_numpy(c["v_pool"])
    dt = D.from_numpy(c["tables"])
    dl = D.from_numpy(np.array([c["L"]], np.int32))
    dq, dkn, dvn = D.from_numpy(c["q"]), D.from_numpy(c["k_new"]), D.from_numpy(c["v_new"])
    dw = D.from_numpy(c["w"])
    db = D.from_numpy(c["bias"]) if c["bias"] is not None else None
    dres = D.from_numpy(c["res"])
    ctx = D.from_numpy(np.full(c["K"], np.nan, np.float32))
    out = dres if alias else D.from_numpy(np.full(c["H"], np.nan, np.float32))
    bias_ptr = db.ptr if db is not None else None
    if folded:
        rc = lib.skv_paged_decode_append_oproj(
            dq.ptr, dkn.ptr, dvn.ptr, dk.ptr, dv.ptr, c["total"], dt.ptr, c["mb"], dl.ptr, c["Hq"], c["Hkv"],
            c["hd"], BS, c["scale"], dw.ptr, skv.DTYPE_BF16, 1, c["stride_n"], bias_ptr, dres.ptr, c["H"],
            ctx.ptr, out.ptr, None)
        assert rc == expect, rc
    else:
        ws, wsb = skv.decode_workspace(1, c["Hq"], c["Hkv"], c["hd"])
        skv.paged_decode_append(dq, skv.DTYPE_FP32, dkn, dvn, skv.DTYPE_FP32, dk, dv, c["total"], dt, c["mb"],
                                dl, 1, c["Hq"], c["Hkv"], c["hd"], BS, c["scale"], ctx, ws, wsb)
        skv._check(lib.skv_linear_residual_f32(ctx.ptr, dw.ptr, skv.DTYPE_BF16, 1, c["stride_n"], c["K"], c["H"],
                                               bias_ptr, dres.ptr, out.ptr, None))
    skv.synchronize()
    return (ctx.download(np.float32, (c["K"],)), out.download(np.float32, (c["H"],)),
            dk.download(np.uint16, c["k_pool"].shape), dv.download(np.uint16, c["v_pool"].shape))


GEOMS = {"tinyllama": (32, 4, 64, 2048), "small": (8, 2, 64, 512)}
LENS = [0, 1, 2, 15, 16, 17, 33, 100, 144, 160, 255, 256]


@pytest.mark.parametrize("with_bias", [False, True])
@pytest.mark.parametrize("geom", sorted(GEOMS))
def test_fold_matches_decode_then_oproj(gpu, geom, with_bias):
    Hq, Hkv, hd, H = GEOMS[geom]
    for i, L in enumerate(LENS):
        need = max(1, -(-L // BS))
        for mb in sorted({need, 16}):
            c = _case(Hq, Hkv, hd, H, L, mb, seed=100 * i + mb, with_bias=with_bias, pad=8 * (i % 2))
            what = f"{geom} L={L} mb={mb} bias={with_bias}"
            got, want = _run(gpu, c, True, alias=(i % 3 == 0)), _run(gpu, c, False, alias=(i % 3 == 0))
            for a, b, name in zip(got, want, ("context", "out", "k pool", "v pool")):
                assert np.array_equal(a.view(np.uint32 if a.dtype == np.float32 else np.uint16),
                                      b.view(np.uint32 if b.dtype == np.float32 else np.uint16)), f"{what}: {name}"
            if L == 0:
                assert not got[0].any(), what
                continue
            k_ref, v_ref = c["k_pool"].copy(), c["v_pool"].copy()
            oracle.kv_append(c["k_new"].reshape(1, -1), c["v_new"].reshape(1, -1), k_ref, v_ref, c["tables"],
                             np.array([L - 1], np.int32), 1, 1, Hkv, hd, BS)
            assert np.array_equal(got[2], k_ref) and np.array_equal(got[3], v_ref), f"{what}: pools vs oracle"
            ref = oracle.paged_decode(c["q"], k_ref, v_ref, c["tables"], np.array([L], np.int32), Hkv, BS,
                                      c["scale"])
            assert_close(got[0].reshape(1, Hq, hd), ref, what=what)


@pytest.mark.parametrize("change", ["table_17", "head_dim_128", "fp32_weights", "k_512_too_small", "hq16"])
def test_fold_unsupported_shapes_launch_nothing(gpu, change):
    Hq, Hkv, hd, H = GEOMS["tinyllama"]
    mb = 16
    if change == "table_17":
        mb = 17
    if change == "head_dim_128":
        Hq, Hkv, hd = 16, 4, 128
    if change == "k_512_too_small":
        Hq, Hkv, hd = 4, 2, 64     # in_dim 256
    if change == "hq16":
        Hq, Hkv = 16, 4           # 4 query heads per kv head over 4 kv heads: no instance
    c = _case(Hq, Hkv, hd, H, 100, mb, seed=3, with_bias=False)
    if change == "fp32_weights":
        D = gpu.DeviceBuffer
        rc = gpu.lib().skv_paged_decode_append_oproj(
            D.from_numpy(c["q"]).ptr, D.from_numpy(c["k_new"]).ptr, D.from_numpy(c["v_new"]).ptr,
            D.from_numpy(c["k_pool"]).ptr, D.from_numpy(c["v_pool"]).ptr, c["total"],
            D.from_numpy(c["tables"]).ptr, mb, D.from_numpy(np.array([100], np.int32)).ptr, Hq, Hkv, hd, BS,
            c["scale"], D.from_numpy(np.zeros((H, c["K"]), np.float32)).ptr, gpu.DTYPE_FP32, 1, c["K"], None,
            D.from_numpy(c["res"]).ptr, H, D(4 * c["K"]).ptr, D(4 * H).ptr, None)
        assert rc == gpu.SKV_ERR_UNSUPPORTED
        return
    ctx, out, kp, vp = _run(gpu, c, True, expect=gpu.SKV_ERR_UNSUPPORTED)
    assert np.isnan(ctx).all() and np.isnan(out).all()
    assert np.array_equal(kp, c["k_pool"]) and np.array_equal(vp, c["v_pool"])
