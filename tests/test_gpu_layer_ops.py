"""The decoder-layer sub-steps around the paged-KV path (skv_layer_ops.hip),
through the C ABI, against float64 numpy restatements of the reference's
behaviour: linear.cpp:113-163 (Y = X W, W logical [in, out], output-major rows
behind a transpose view or GEMM-ready), gemm_cuda.cu:172-202 (RMSNorm),
attention.cpp:96-135 (split-half RoPE, float inverse frequency, double angle),
transformer_block.cpp:315-323 (SwiGLU), the residual add.

Tolerance for the fp32-accumulated dot products: |gpu - ref| <= 1e-5 * sum|x w|
+ 1e-6 (the accumulation order differs from the reference loop, the rounding
bound scales with the sum of absolute products)."""
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
