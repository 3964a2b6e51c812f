"""The decoder-layer sub-steps around the paged-KV path (skv_layer_ops.hip),
through the C ABI, against float64 numpy restatements of the reference's
behaviour: linear.cpp:113-163 (Y = X W, W logical [in, out], output-major rows
behind a transpose view or GEMM-ready), gemm_cuda.cu:172-202 (RMSNorm),
attention.cpp:96-135 (split-half RoPE, float inverse frequency, double angle),
transformer_block.cpp:315-323 (SwiGLU), the residual add.

Tolerance for the fp32-accumulated dot products: |gpu - ref| <= 1e-5 * sum|x w|
+ 1e-6 (the accumulation order differs from the reference loop, the rounding
bound scales with the sum of absolute products)."""
import ctypes

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def _linear(skv, x, w_store, dtype, stride_k, stride_n, K, N, bias=None, offset=0):
    """w_store: the weight buffer exactly as laid out in device memory."""
    raw = np.frombuffer(w_store.tobytes(), np.uint8)
    dw = skv.DeviceBuffer(raw.size + 16)
    dw.upload(np.concatenate([np.zeros(offset, np.uint8), raw, np.zeros(16 - offset, np.uint8)]))
    dx = skv.DeviceBuffer.from_numpy(np.ascontiguousarray(x, np.float32))
    rows = x.shape[0]
    dy = skv.DeviceBuffer(rows * N * 4)
    dy.upload(np.full((rows, N), np.nan, np.float32))
    db = None if bias is None else skv.DeviceBuffer.from_numpy(bias.astype(np.float32))
    wd = skv.DTYPE_BF16 if dtype == "bf16" else skv.DTYPE_FP32
    skv._check(skv.lib().skv_linear_f32(dx.ptr, rows, dw.ptr + offset, wd, stride_k, stride_n, K, N,
                                         None if db is None else db.ptr, dy.ptr, None))
    skv.synchronize()
    return dy.download(np.float32, (rows, N))


@pytest.mark.parametrize("K,N,rows", [(2048, 300, 1), (5632, 64, 1), (1000, 37, 1), (37, 5, 2),
                                      (10000, 20, 1), (2048, 2048, 3)])
@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
@pytest.mark.parametrize("layout", ["rows", "rows_unaligned", "cols"])
def test_linear_matches_float64(gpu, K, N, rows, dtype, layout):
    rng = np.random.default_rng(K + N + rows)
    x = rng.standard_normal((rows, K)).astype(np.float32)
    w = (0.05 * rng.standard_normal((K, N))).astype(np.float32)   # logical [in, out]
    if dtype == "bf16":
        w_bits = oracle.f32_to_bf16(w)
        w = oracle.bf16_to_f32(w_bits)
    bias = rng.standard_normal(N).astype(np.float32) if N % 2 else None
    if layout.startswith("rows"):   # output-major [out][in] rows, transpose view
        store = np.ascontiguousarray((w_bits if dtype == "bf16" else w).T)
        sk, sn = 1, K
    else:                            # GEMM-ready [in][out]
        store = np.ascontiguousarray(w_bits if dtype == "bf16" else w)
        sk, sn = N, 1
    offset = (2 if dtype == "bf16" else 4) if layout == "rows_unaligned" else 0
    got = _linear(gpu, x, store, dtype, sk, sn, K, N, bias, offset)
    ref = x.astype(np.float64) @ w.astype(np.float64)
    if bias is not None:
        ref += bias
    bound = 1e-5 * (np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64)) + 1e-6
    err = np.abs(got - ref)
    assert np.isfinite(got).all()
    assert (err <= bound).all(), f"max err {err.max():.3e}, worst ratio {(err / bound).max():.2f}"


def test_rmsnorm_rope_swiglu_add(gpu):
    rng = np.random.default_rng(7)
    H, heads, hd, pos = 2048, 32, 64, 1234
    x = rng.standard_normal((2, H)).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    dx, dg = gpu.DeviceBuffer.from_numpy(x), gpu.DeviceBuffer.from_numpy(gamma)
    dy = gpu.DeviceBuffer(x.nbytes)
    gpu._check(gpu.lib().skv_rmsnorm_f32(dx.ptr, dy.ptr, dg.ptr, 2, H, 1e-5, None))
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd * xd).mean(axis=1, keepdims=True) + 1e-5) * gamma
    got = dy.download(np.float32, x.shape)
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-6)

    q = rng.standard_normal((heads, hd)).astype(np.float32)
    dq = gpu.DeviceBuffer.from_numpy(q)
    gpu._check(gpu.lib().skv_rope_f32(dq.ptr, heads, hd, pos, None))
    half = hd // 2
    inv = np.array([np.float32(10000.0 ** (-2.0 * i / hd)) for i in range(half)], np.float64)
    ang = pos * inv
    c, s = np.cos(ang), np.sin(ang)
    a, b = q[:, :half].astype(np.float64), q[:, half:].astype(np.float64)
    ref = np.concatenate([a * c - b * s, a * s + b * c], axis=1)
    got = dq.download(np.float32, q.shape)
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-5)

    g = (4 * rng.standard_normal(5632)).astype(np.float32)
    u = rng.standard_normal(5632).astype(np.float32)
    dgt, du = gpu.DeviceBuffer.from_numpy(g), gpu.DeviceBuffer.from_numpy(u)
    gpu._check(gpu.lib().skv_swiglu_f32(dgt.ptr, du.ptr, g.size, None))
    gd = g.astype(np.float64)
    ref = gd / (1 + np.exp(-gd)) * u
    assert np.allclose(dgt.download(np.float32, g.shape), ref, rtol=1e-5, atol=1e-6)

    t = rng.standard_normal(H).astype(np.float32)
    dt, ds = gpu.DeviceBuffer.from_numpy(t), gpu.DeviceBuffer.from_numpy(x[0])
    gpu._check(gpu.lib().skv_add_f32(dt.ptr, ds.ptr, H, None))
    assert np.array_equal(dt.download(np.float32, t.shape), t + x[0])


def _bf16_rows(rng, n, k, scale=0.05):
    return oracle.f32_to_bf16((scale * rng.standard_normal((n, k))).astype(np.float32))


@pytest.mark.parametrize("with_bias", [False, True])
@pytest.mark.parametrize("position", [-1, 0, 777])
def test_fused_projections_match_separate_kernels(gpu, with_bias, position):
    """skv_fused_qkv_f32, skv_fused_gate_up_swiglu_f32 and skv_linear_residual_f32
    give the same bits as rmsnorm + linear + rope / swiglu / add run separately."""
    rng = np.random.default_rng(11 + position)
    H, Hq, Hkv, hd, inter = 1024, 16, 4, 64, 2816
    lib, D = gpu.lib(), gpu.DeviceBuffer
    h = rng.standard_normal(H).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    W = {n: _bf16_rows(rng, o, i) for n, o, i in
         (("q", Hq * hd, H), ("k", Hkv * hd, H), ("v", Hkv * hd, H), ("o", H, Hq * hd),
          ("g", inter, H), ("u", inter, H), ("d", H, inter))}
    B = {n: (rng.standard_normal(w.shape[0]).astype(np.float32) if with_bias else None)
         for n, w in W.items()}
    dW = {n: D.from_numpy(w) for n, w in W.items()}
    dB = {n: (D.from_numpy(b) if b is not None else None) for n, b in B.items()}
    bp = lambda n: dB[n].ptr if dB[n] is not None else None
    dh, dg = D.from_numpy(h), D.from_numpy(gamma)

    def out(n):
        return D(4 * n)

    def lin(x, name, y):
        w = W[name]
        gpu._check(lib.skv_linear_f32(x.ptr, 1, dW[name].ptr, gpu.DTYPE_BF16, 1, w.shape[1], w.shape[1],
                                      w.shape[0], bp(name), y.ptr, None))

    # separate
    xn = out(H)
    gpu._check(lib.skv_rmsnorm_f32(dh.ptr, xn.ptr, dg.ptr, 1, H, 1e-5, None))
    qs, ks, vs = out(Hq * hd), out(Hkv * hd), out(Hkv * hd)
    lin(xn, "q", qs), lin(xn, "k", ks), lin(xn, "v", vs)
    if position >= 0:
        gpu._check(lib.skv_rope_f32(qs.ptr, Hq, hd, position, None))
        gpu._check(lib.skv_rope_f32(ks.ptr, Hkv, hd, position, None))
    # fused
    qf, kf, vf = out(Hq * hd), out(Hkv * hd), out(Hkv * hd)
    strides = (ctypes.c_int64 * 3)(H, H, H)
    gpu._check(lib.skv_fused_qkv_f32(dh.ptr, dg.ptr, ctypes.c_float(1e-5), dW["q"].ptr, dW["k"].ptr,
                                     dW["v"].ptr, gpu.DTYPE_BF16, 1, strides, bp("q"), bp("k"), bp("v"),
                                     H, Hq, Hkv, hd, position, qf.ptr, kf.ptr, vf.ptr, None))
    gpu.synchronize()
    for a, b, n in ((qs, qf, Hq * hd), (ks, kf, Hkv * hd), (vs, vf, Hkv * hd)):
        assert np.array_equal(a.download(np.uint32, (n,)), b.download(np.uint32, (n,)))

    # o_proj + residual
    ctx = D.from_numpy(rng.standard_normal(Hq * hd).astype(np.float32))
    hs = out(H)
    lin(ctx, "o", hs)
    gpu._check(lib.skv_add_f32(hs.ptr, dh.ptr, H, None))
    hf = out(H)
    gpu._check(lib.skv_linear_residual_f32(ctx.ptr, dW["o"].ptr, gpu.DTYPE_BF16, 1, Hq * hd, Hq * hd, H,
                                           bp("o"), dh.ptr, hf.ptr, None))
    # rmsnorm + gate/up + swiglu
    xn2, gs, us = out(H), out(inter), out(inter)
    gpu._check(lib.skv_rmsnorm_f32(hs.ptr, xn2.ptr, dg.ptr, 1, H, 1e-5, None))
    lin(xn2, "g", gs), lin(xn2, "u", us)
    gpu._check(lib.skv_swiglu_f32(gs.ptr, us.ptr, inter, None))
    af = out(inter)
    gpu._check(lib.skv_fused_gate_up_swiglu_f32(hs.ptr, dg.ptr, ctypes.c_float(1e-5), dW["g"].ptr,
                                                dW["u"].ptr, gpu.DTYPE_BF16, 1, H, H, bp("g"), bp("u"),
                                                H, inter, af.ptr, None))
    # down + residual
    ds_, yf = out(H), out(H)
    lin(gs, "d", ds_)
    gpu._check(lib.skv_add_f32(ds_.ptr, hs.ptr, H, None))
    gpu._check(lib.skv_linear_residual_f32(gs.ptr, dW["d"].ptr, gpu.DTYPE_BF16, 1, inter, inter, H,
                                           bp("d"), hs.ptr, yf.ptr, None))
    gpu.synchronize()
    for a, b, n in ((hs, hf, H), (gs, af, inter), (ds_, yf, H)):
        assert np.array_equal(a.download(np.uint32, (n,)), b.download(np.uint32, (n,)))


@pytest.mark.parametrize("with_bias", [False, True])
def test_fused_qkv_at_device_position(gpu, with_bias):
    """skv_fused_qkv_at_f32 (position read on the device, cos/sin from the
    skv_rope_cos_sin table) gives the bits of skv_fused_qkv_f32 at the same
    position; a position past the table is clamped to its last row."""
    rng = np.random.default_rng(5)
    H, Hq, Hkv, hd, P = 1024, 16, 4, 64, 300
    lib, D = gpu.lib(), gpu.DeviceBuffer
    h = rng.standard_normal(H).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    W = {n: _bf16_rows(rng, o, H) for n, o in (("q", Hq * hd), ("k", Hkv * hd), ("v", Hkv * hd))}
    dW = {n: D.from_numpy(w) for n, w in W.items()}
    dB = {n: (D.from_numpy(rng.standard_normal(W[n].shape[0]).astype(np.float32)) if with_bias else None)
          for n in W}
    bp = lambda n: dB[n].ptr if dB[n] is not None else None
    dh, dg = D.from_numpy(h), D.from_numpy(gamma)
    table = np.zeros((P, hd), np.float32)
    gpu._check(lib.skv_rope_cos_sin(hd, 0, P, table.ctypes.data))
    d_table = D.from_numpy(table)
    strides = (ctypes.c_int64 * 3)(H, H, H)
    for position, want_pos in ((0, 0), (1, 1), (17, 17), (299, 299), (450, 299)):
        pos_buf = D.from_numpy(np.array([position], np.int32))
        outs = {}
        for mode in ("host", "device"):
            q, k, v = D(4 * Hq * hd), D(4 * Hkv * hd), D(4 * Hkv * hd)
            if mode == "host":
                gpu._check(lib.skv_fused_qkv_f32(dh.ptr, dg.ptr, ctypes.c_float(1e-5), dW["q"].ptr, dW["k"].ptr,
                                                 dW["v"].ptr, gpu.DTYPE_BF16, 1, strides, bp("q"), bp("k"), bp("v"),
                                                 H, Hq, Hkv, hd, want_pos, q.ptr, k.ptr, v.ptr, None))
            else:
                gpu._check(lib.skv_fused_qkv_at_f32(dh.ptr, dg.ptr, ctypes.c_float(1e-5), dW["q"].ptr, dW["k"].ptr,
                                                    dW["v"].ptr, gpu.DTYPE_BF16, 1, strides, bp("q"), bp("k"),
                                                    bp("v"), H, Hq, Hkv, hd, pos_buf.ptr, d_table.ptr, P, q.ptr,
                                                    k.ptr, v.ptr, None))
            gpu.synchronize()
            outs[mode] = [b.download(np.uint32, (n,)) for b, n in ((q, Hq * hd), (k, Hkv * hd), (v, Hkv * hd))]
        for a, b in zip(outs["host"], outs["device"]):
            assert np.array_equal(a, b), position


def test_rope_cos_sin_table_rejects(gpu):
    buf = np.zeros(64, np.float32)
    with pytest.raises(gpu.SkvError):
        gpu._check(gpu.lib().skv_rope_cos_sin(63, 0, 1, buf.ctypes.data))    # odd head_dim
    with pytest.raises(gpu.SkvError):
        gpu._check(gpu.lib().skv_rope_cos_sin(64, 0, 0, buf.ctypes.data))    # no positions


def test_fused_projections_refuse_unsupported_layouts(gpu):
    """GEMM-ready (input-major) or misaligned weights: SKV_ERR_UNSUPPORTED, nothing written."""
    lib = gpu.lib()
    H = 256
    w = gpu.DeviceBuffer(H * H * 2 + 16)
    x = gpu.DeviceBuffer.from_numpy(np.ones(H, np.float32))
    y = gpu.DeviceBuffer.from_numpy(np.full(H, 7.0, np.float32))
    rc = lib.skv_linear_residual_f32(x.ptr, w.ptr, gpu.DTYPE_BF16, H, 1, H, H, None, x.ptr, y.ptr, None)
    assert rc == gpu.SKV_ERR_UNSUPPORTED
    rc = lib.skv_linear_residual_f32(x.ptr, w.ptr + 2, gpu.DTYPE_BF16, 1, H, H, H, None, x.ptr, y.ptr, None)
    assert rc == gpu.SKV_ERR_UNSUPPORTED
    gpu.synchronize()
    assert np.array_equal(y.download(np.float32, (H,)), np.full(H, 7.0, np.float32))


def _fused_calls(gpu, lib, dims, W, dW, bp, x_rows, position, rows_api):
    """Run the three fused projections over x_rows [n][H]: one call with
    rows_api, else one single-token call per row; returns host arrays."""
    H, Hq, Hkv, hd, inter = dims
    D = gpu.DeviceBuffer
    n = x_rows.shape[0]
    rng = np.random.default_rng(5)
    gamma = D.from_numpy((1 + 0.1 * rng.standard_normal(H)).astype(np.float32))
    ctx = rng.standard_normal((n, Hq * hd)).astype(np.float32)
    act_in = rng.standard_normal((n, inter)).astype(np.float32)
    res = rng.standard_normal((n, H)).astype(np.float32)
    dt = W["dtype"]
    strides = (ctypes.c_int64 * 3)(H, H, H)
    out = {k: D(4 * n * m) for k, m in (("q", Hq * hd), ("k", Hkv * hd), ("v", Hkv * hd), ("act", inter),
                                        ("o", H), ("d", H))}
    dx, dctx, dact, dres = D.from_numpy(x_rows), D.from_numpy(ctx), D.from_numpy(act_in), D.from_numpy(res)
    eps = ctypes.c_float(1e-5)
    if rows_api:
        scratch = D(4 * n * H)
        gpu._check(lib.skv_fused_qkv_rows_f32(dx.ptr, n, gamma.ptr, eps, dW["q"].ptr, dW["k"].ptr, dW["v"].ptr,
                                              dt, 1, strides, bp("q"), bp("k"), bp("v"), H, Hq, Hkv, hd,
                                              position, out["q"].ptr, out["k"].ptr, out["v"].ptr, scratch.ptr,
                                              None))
        gpu._check(lib.skv_fused_gate_up_swiglu_rows_f32(dx.ptr, n, gamma.ptr, eps, dW["g"].ptr, dW["u"].ptr, dt,
                                                         1, H, H, bp("g"), bp("u"), H, inter, out["act"].ptr,
                                                         scratch.ptr, None))
        gpu._check(lib.skv_linear_residual_rows_f32(dctx.ptr, n, dW["o"].ptr, dt, 1, Hq * hd, Hq * hd, H,
                                                    bp("o"), dres.ptr, out["o"].ptr, None))
        gpu._check(lib.skv_linear_residual_rows_f32(dact.ptr, n, dW["d"].ptr, dt, 1, inter, inter, H,
                                                    bp("d"), dres.ptr, out["d"].ptr, None))
    else:
        for r in range(n):
            off = lambda buf, dim: buf.ptr + 4 * r * dim
            pos = position + r if position >= 0 else -1
            gpu._check(lib.skv_fused_qkv_f32(off(dx, H), gamma.ptr, eps, dW["q"].ptr, dW["k"].ptr, dW["v"].ptr,
                                             dt, 1, strides, bp("q"), bp("k"), bp("v"), H, Hq, Hkv, hd, pos,
                                             off(out["q"], Hq * hd), off(out["k"], Hkv * hd),
                                             off(out["v"], Hkv * hd), None))
            gpu._check(lib.skv_fused_gate_up_swiglu_f32(off(dx, H), gamma.ptr, eps, dW["g"].ptr, dW["u"].ptr, dt,
                                                        1, H, H, bp("g"), bp("u"), H, inter,
                                                        off(out["act"], inter), None))
            gpu._check(lib.skv_linear_residual_f32(off(dctx, Hq * hd), dW["o"].ptr, dt, 1, Hq * hd, Hq * hd, H,
                                                   bp("o"), off(dres, H), off(out["o"], H), None))
            gpu._check(lib.skv_linear_residual_f32(off(dact, inter), dW["d"].ptr, dt, 1, inter, inter, H,
                                                   bp("d"), off(dres, H), off(out["d"], H), None))
    gpu.synchronize()
    sizes = {"q": Hq * hd, "k": Hkv * hd, "v": Hkv * hd, "act": inter, "o": H, "d": H}
    return {k: out[k].download(np.uint32, (n, sizes[k])) for k in out}


@pytest.mark.parametrize("dims,dtype", [((1024, 16, 4, 64, 2048), "bf16"), ((1024, 16, 4, 64, 2048), "fp32"),
                                        ((2048, 16, 2, 128, 5632), "bf16"), ((3072, 24, 8, 128, 3584), "bf16")],
                         ids=["k1024_bf16", "k1024_fp32", "tinyllama_ffn", "k3072"])
@pytest.mark.parametrize("with_bias", [False, True])
def test_fused_rows_match_one_token_calls(gpu, dims, dtype, with_bias):
    """skv_*_rows_f32 over n tokens == the one-token entry points on each row,
    bit for bit (weights read once for all rows; RoPE at first_position + r)."""
    H, Hq, Hkv, hd, inter = dims
    rng = np.random.default_rng(H + inter + with_bias)
    lib, D = gpu.lib(), gpu.DeviceBuffer
    shapes = (("q", Hq * hd, H), ("k", Hkv * hd, H), ("v", Hkv * hd, H), ("o", H, Hq * hd),
              ("g", inter, H), ("u", inter, H), ("d", H, inter))
    if dtype == "bf16":
        W = {n: _bf16_rows(rng, o, i) for n, o, i in shapes}
        W["dtype"] = gpu.DTYPE_BF16
    else:
        W = {n: (0.03 * rng.standard_normal((o, i))).astype(np.float32) for n, o, i in shapes}
        W["dtype"] = gpu.DTYPE_FP32
    dW = {n: D.from_numpy(W[n]) for n, _, _ in shapes}
    B = {n: (D.from_numpy(rng.standard_normal(o).astype(np.float32)) if with_bias else None) for n, o, _ in shapes}
    bp = lambda n: B[n].ptr if B[n] is not None else None
    for n_rows, position in ((2, 0), (5, 1000), (16, 7), (37, 16381), (3, -1)):
        x = rng.standard_normal((n_rows, H)).astype(np.float32)
        got = _fused_calls(gpu, lib, dims, W, dW, bp, x, position, rows_api=True)
        want = _fused_calls(gpu, lib, dims, W, dW, bp, x, position, rows_api=False)
        for k in got:
            assert np.array_equal(got[k], want[k]), f"{k}: rows={n_rows} position={position}"


def test_fused_rows_refuse_unsupported_shapes(gpu):
    """in_dim not a multiple of the wave-wide step, or too long to keep the
    rows in registers: SKV_ERR_UNSUPPORTED and nothing written."""
    lib, D = gpu.lib(), gpu.DeviceBuffer
    for K, dt in ((1000, gpu.DTYPE_BF16), (8192, gpu.DTYPE_BF16), (4096, gpu.DTYPE_FP32)):
        esz = 2 if dt == gpu.DTYPE_BF16 else 4
        w = D(64 * K * esz)
        x = D.from_numpy(np.ones((3, K), np.float32))
        res = D.from_numpy(np.zeros((3, 64), np.float32))
        y = D.from_numpy(np.full((3, 64), 7.0, np.float32))
        rc = lib.skv_linear_residual_rows_f32(x.ptr, 3, w.ptr, dt, 1, K, K, 64, None, res.ptr, y.ptr, None)
        assert rc == gpu.SKV_ERR_UNSUPPORTED, (K, dt)
    gpu.synchronize()
    assert np.array_equal(y.download(np.float32, (3, 64)), np.full((3, 64), 7.0, np.float32))


@pytest.mark.parametrize("hd", [64, 128])
def test_rope_rows_cos_sin_equal_host_libm(gpu, hd):
    """skv_rope_rows_f32 on (1, 0) pairs returns (cos, sin) exactly; over
    positions 0..32767 they equal the host's libm values rounded to float
    (the table skv_rope_f32 and the one-token fused projection use)."""
    import math
    lib, D = gpu.lib(), gpu.DeviceBuffer
    half, rows = hd // 2, 32768
    x = np.zeros((rows, hd), np.float32)
    x[:, :half] = 1.0
    dx = D.from_numpy(x)
    gpu._check(lib.skv_rope_rows_f32(dx.ptr, rows, 1, hd, 0, None))
    got = dx.download(np.float32, (rows, hd))
    inv = [float(np.float32(10000.0 ** (-2.0 * i / hd))) for i in range(half)]
    want_c = np.array([[math.cos(p * f) for f in inv] for p in range(rows)], np.float64).astype(np.float32)
    want_s = np.array([[math.sin(p * f) for f in inv] for p in range(rows)], np.float64).astype(np.float32)
    bad_c = np.count_nonzero(got[:, :half].view(np.uint32) != want_c.view(np.uint32))
    bad_s = np.count_nonzero(got[:, half:].view(np.uint32) != want_s.view(np.uint32))
    assert bad_c == 0 and bad_s == 0, f"{bad_c} cos and {bad_s} sin values differ from libm"
    # and the one-position kernel (host table) agrees at a few positions
    for p in (0, 1, 777, 32767):
        y = D.from_numpy(x[:1])
        gpu._check(lib.skv_rope_f32(y.ptr, 1, hd, p, None))
        assert np.array_equal(y.download(np.uint32, (1, hd))[0], got[p].view(np.uint32))


def _mm_reference(W, B, x, gamma, ctx, act_in, res, dims, position, eps=1e-5):
    """float64 restatement of the three projections of several tokens:
    rmsnorm, W x + bias, RoPE at position + r with the device's float32
    cos/sin (angle in double from the float32 inverse frequency), SwiGLU,
    residual."""
    H, Hq, Hkv, hd, inter = dims
    w = {k: oracle.bf16_to_f32(W[k]).astype(np.float64) for k in "qkvogud"}
    b = {k: (B[k].astype(np.float64) if B[k] is not None else 0.0) for k in "qkvogud"}
    x = x.astype(np.float64)
    xn = x / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps) * gamma.astype(np.float64)
    out = {k: xn @ w[k].T + b[k] for k in "qkv"}
    if position >= 0:
        half = hd // 2
        inv = np.array([np.float32(10000.0 ** (-2.0 * i / hd)) for i in range(half)], np.float64)
        ang = (position + np.arange(x.shape[0], dtype=np.float64))[:, None] * inv[None, :]
        c, s = np.cos(ang).astype(np.float32).astype(np.float64), np.sin(ang).astype(np.float32).astype(np.float64)
        for k, nh in (("q", Hq), ("k", Hkv)):
            y = out[k].reshape(x.shape[0], nh, hd)
            a0, b0 = y[:, :, :half].copy(), y[:, :, half:].copy()
            y[:, :, :half] = a0 * c[:, None, :] - b0 * s[:, None, :]
            y[:, :, half:] = a0 * s[:, None, :] + b0 * c[:, None, :]
            out[k] = y.reshape(x.shape[0], nh * hd)
    g, u = xn @ w["g"].T + b["g"], xn @ w["u"].T + b["u"]
    out["act"] = g / (1.0 + np.exp(-g)) * u
    out["o"] = ctx.astype(np.float64) @ w["o"].T + b["o"] + res
    out["d"] = act_in.astype(np.float64) @ w["d"].T + b["d"] + res
    return out


@pytest.mark.parametrize("dims", [(2048, 32, 4, 64, 5632), (1024, 8, 2, 128, 1536)], ids=["tinyllama", "hd128"])
@pytest.mark.parametrize("with_bias", [False, True])
def test_mm_projections_match_float64(gpu, dims, with_bias):
    """skv_*_mm_f32 (matrix cores, inputs split into bf16 hi + lo) against the
    float64 restatement: every output within 1e-4 of its matrix's rms (a
    dropped lo part errs by ~2e-3 relative, a wrong RoPE pair or token by
    O(1)); tokens 1 .. 300 (partial 64-token tiles), RoPE positions up to
    16,381 and none."""
    H, Hq, Hkv, hd, inter = dims
    rng = np.random.default_rng(H + inter + with_bias)
    lib, D = gpu.lib(), gpu.DeviceBuffer
    shapes = (("q", Hq * hd, H), ("k", Hkv * hd, H), ("v", Hkv * hd, H), ("o", H, Hq * hd),
              ("g", inter, H), ("u", inter, H), ("d", H, inter))
    W = {n: _bf16_rows(rng, o, i, 0.03) for n, o, i in shapes}
    dW = {n: D.from_numpy(W[n]) for n, _, _ in shapes}
    B = {n: (rng.standard_normal(o).astype(np.float32) if with_bias else None) for n, o, _ in shapes}
    dB = {n: (D.from_numpy(B[n]) if B[n] is not None else None) for n, _, _ in shapes}
    bp = lambda n: dB[n].ptr if dB[n] is not None else None
    strides = (ctypes.c_int64 * 3)(H, H, H)
    eps = ctypes.c_float(1e-5)
    for n, position in ((1, 0), (16, 7), (37, 1000), (64, -1), (300, 16381)):
        x = rng.standard_normal((n, H)).astype(np.float32)
        gamma = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
        ctx = rng.standard_normal((n, Hq * hd)).astype(np.float32)
        act_in = rng.standard_normal((n, inter)).astype(np.float32)
        res = rng.standard_normal((n, H)).astype(np.float32)
        dx, dg, dctx, dact, dres = (D.from_numpy(a) for a in (x, gamma, ctx, act_in, res))
        sizes = {"q": Hq * hd, "k": Hkv * hd, "v": Hkv * hd, "act": inter, "o": H, "d": H}
        out = {k: D(4 * n * m) for k, m in sizes.items()}
        for buf in out.values():
            buf.upload(np.full(buf.nbytes // 4, np.nan, np.float32))
        scratch = D(4 * n * H)
        gpu._check(lib.skv_fused_qkv_mm_f32(dx.ptr, n, dg.ptr, eps, dW["q"].ptr, dW["k"].ptr, dW["v"].ptr,
                                            gpu.DTYPE_BF16, 1, strides, bp("q"), bp("k"), bp("v"), H, Hq, Hkv,
                                            hd, position, out["q"].ptr, out["k"].ptr, out["v"].ptr, scratch.ptr,
                                            None))
        gpu._check(lib.skv_fused_gate_up_swiglu_mm_f32(dx.ptr, n, dg.ptr, eps, dW["g"].ptr, dW["u"].ptr,
                                                       gpu.DTYPE_BF16, 1, H, H, bp("g"), bp("u"), H, inter,
                                                       out["act"].ptr, scratch.ptr, None))
        gpu._check(lib.skv_linear_residual_mm_f32(dctx.ptr, n, dW["o"].ptr, gpu.DTYPE_BF16, 1, Hq * hd, Hq * hd,
                                                  H, bp("o"), dres.ptr, out["o"].ptr, None))
        gpu._check(lib.skv_linear_residual_mm_f32(dact.ptr, n, dW["d"].ptr, gpu.DTYPE_BF16, 1, inter, inter, H,
                                                  bp("d"), dres.ptr, out["d"].ptr, None))
        gpu.synchronize()
        ref = _mm_reference(W, B, x, gamma, ctx, act_in, res, dims, position)
        for k, m in sizes.items():
            got = out[k].download(np.float32, (n, m)).astype(np.float64)
            err = np.abs(got - ref[k]).max()
            bound = 1e-4 * np.sqrt((ref[k] ** 2).mean())
            assert np.isfinite(got).all() and err <= bound, f"{k}: rows={n} position={position} err={err:.3g} bound={bound:.3g}"


def test_mm_projections_refuse_unsupported_shapes(gpu):
    """fp32 weights, in_dim not a multiple of 128, an output count not a
    multiple of 32: SKV_ERR_UNSUPPORTED and nothing written."""
    lib, D = gpu.lib(), gpu.DeviceBuffer
    y = D.from_numpy(np.full((3, 64), 7.0, np.float32))
    res = D.from_numpy(np.zeros((3, 64), np.float32))
    for K, out_dim, dt in ((1024, 64, gpu.DTYPE_FP32), (1000, 64, gpu.DTYPE_BF16), (1024, 48, gpu.DTYPE_BF16)):
        esz = 2 if dt == gpu.DTYPE_BF16 else 4
        w = D(64 * K * esz)
        x = D.from_numpy(np.ones((3, K), np.float32))
        rc = lib.skv_linear_residual_mm_f32(x.ptr, 3, w.ptr, dt, 1, K, K, out_dim, None, res.ptr, y.ptr, None)
        assert rc == gpu.SKV_ERR_UNSUPPORTED, (K, out_dim, dt)
    gpu.synchronize()
    assert np.array_equal(y.download(np.float32, (3, 64)), np.full((3, 64), 7.0, np.float32))
