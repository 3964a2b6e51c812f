"""The library-GEMM projections of long prompt chunks (skv_*_gemm_f32:
hipBLASLt bf16 GEMMs over the hi and lo parts of the fp32 inputs, with the
split and the epilogues as kernels of this library) against the float64
restatement of rmsnorm + projection + bias + RoPE / SwiGLU / residual, and
against the matrix-core kernels (skv_*_mm_f32) they replace on the prompt
path."""
import ctypes

import numpy as np
import pytest

import oracle
from test_gpu_layer_ops import _bf16_rows, _mm_reference

pytestmark = pytest.mark.gpu


def _padded(W, pad):
    """W's rows in a buffer with a row stride of in_dim + pad elements."""
    if pad == 0:
        return W, W.shape[1]
    out = np.zeros((W.shape[0], W.shape[1] + pad), W.dtype)
    out[:, :W.shape[1]] = W
    return out, W.shape[1] + pad


def _run_all(gpu, entry, dW, ld, bp, dims, n, position, dx, dg, dctx, dact, dres, out, normalized, ws, wsb):
    """The four projections of a layer through the gemm (entry = "gemm") or mm
    (entry = "mm") entry points."""
    lib = gpu.gemm_lib() if entry == "gemm" else gpu.lib()
    H, Hq, Hkv, hd, inter = dims
    eps = ctypes.c_float(1e-5)
    strides = (ctypes.c_int64 * 3)(ld["q"], ld["k"], ld["v"])
    extra = (ws.ptr, wsb) if entry == "gemm" else ()
    fn = lambda name: getattr(lib, f"skv_{name}_{entry}_f32")
    gpu._check(fn("fused_qkv")(dx.ptr, n, dg.ptr, eps, dW["q"].ptr, dW["k"].ptr, dW["v"].ptr, gpu.DTYPE_BF16, 1,
                               strides, bp("q"), bp("k"), bp("v"), H, Hq, Hkv, hd, position, out["q"].ptr,
                               out["k"].ptr, out["v"].ptr, normalized.ptr, *extra, None))
    gpu._check(fn("fused_gate_up_swiglu")(dx.ptr, n, dg.ptr, eps, dW["g"].ptr, dW["u"].ptr, gpu.DTYPE_BF16, 1,
                                          ld["g"], ld["u"], bp("g"), bp("u"), H, inter, out["act"].ptr,
                                          normalized.ptr, *extra, None))
    gpu._check(fn("linear_residual")(dctx.ptr, n, dW["o"].ptr, gpu.DTYPE_BF16, 1, ld["o"], Hq * hd, H, bp("o"),
                                     dres.ptr, out["o"].ptr, *extra, None))
    gpu._check(fn("linear_residual")(dact.ptr, n, dW["d"].ptr, gpu.DTYPE_BF16, 1, ld["d"], inter, H, bp("d"),
                                     dres.ptr, out["d"].ptr, *extra, None))


class _At:
    """A device address inside another buffer (kept alive by it)."""

    def __init__(self, buf, offset):
        self.buf, self.ptr = buf, buf.ptr + offset


def _upload_weights(D, W, names, pad, packed):
    """Device weights and row strides: each matrix in its own buffer, or
    (packed) the matrices of each group of `names` as consecutive row blocks
    of one buffer, as the Generator's loader places q/k/v and gate/up."""
    dW, ld = {}, {}
    groups = (("q", "k", "v"), ("g", "u")) if packed else ()
    for group in groups:
        stride = W[group[0]].shape[1] + max(pad.get(n, 0) for n in group)
        rows = np.concatenate([_padded(W[n], stride - W[n].shape[1])[0] for n in group])
        base = D.from_numpy(rows)
        first = 0
        for n in group:
            dW[n], ld[n] = _At(base, 2 * first * stride), stride
            first += W[n].shape[0]
    for n in names:
        if n not in dW:
            buf, ld[n] = _padded(W[n], pad.get(n, 0))
            dW[n] = D.from_numpy(buf)
    return dW, ld


@pytest.mark.parametrize("dims", [(2048, 32, 4, 64, 5632), (1024, 8, 2, 128, 1536)], ids=["tinyllama", "hd128"])
@pytest.mark.parametrize("with_bias", [False, True])
@pytest.mark.parametrize("packed", [False, True], ids=["separate", "packed"])
def test_gemm_projections_match_float64_and_mm(gpu, dims, with_bias, packed):
    """Every output within 1e-4 of its matrix's rms of the float64 result (a
    dropped lo part errs by ~2e-3 relative, a wrong RoPE pair, token or half
    by O(1)), each within 5e-5 (|ref| + rms) of the matrix-core kernels'
    (fp32 sums in another order), and the normalised rows bit-identical to
    theirs.  Tokens 1 .. 1,024 (the 1,024-token chunk of
    the prompt path), RoPE positions up to 16,381 and none, weight rows with a
    padded stride for o_proj and gate, and q/k/v and gate/up each packed in one
    allocation (one GEMM each) or apart."""
    H, Hq, Hkv, hd, inter = dims
    rng = np.random.default_rng(7 * H + inter + with_bias)
    lib, D = gpu.gemm_lib(), gpu.DeviceBuffer
    shapes = (("q", Hq * hd, H), ("k", Hkv * hd, H), ("v", Hkv * hd, H), ("o", H, Hq * hd),
              ("g", inter, H), ("u", inter, H), ("d", H, inter))
    W = {n: _bf16_rows(rng, o, i, 0.03) for n, o, i in shapes}
    dW, ld = _upload_weights(D, W, [n for n, _, _ in shapes], {"o": 64, "g": 64}, packed)
    B = {n: (rng.standard_normal(o).astype(np.float32) if with_bias else None) for n, o, _ in shapes}
    dB = {n: (D.from_numpy(B[n]) if B[n] is not None else None) for n, _, _ in shapes}
    bp = lambda n: dB[n].ptr if dB[n] is not None else None
    max_rows = 1024
    wsb = max(lib.skv_prompt_gemm_workspace_bytes(max_rows, K, outs)
              for K, outs in ((H, (Hq + 2 * Hkv) * hd), (H, 2 * inter), (Hq * hd, H), (inter, H)))
    ws = D(wsb)
    sizes = {"q": Hq * hd, "k": Hkv * hd, "v": Hkv * hd, "act": inter, "o": H, "d": H}
    for n, position in ((1, 0), (16, 7), (37, 1000), (64, -1), (300, 16381), (max_rows, 5)):
        x = rng.standard_normal((n, H)).astype(np.float32)
        gamma = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
        ctx = rng.standard_normal((n, Hq * hd)).astype(np.float32)
        act_in = rng.standard_normal((n, inter)).astype(np.float32)
        res = rng.standard_normal((n, H)).astype(np.float32)
        dx, dg, dctx, dact, dres = (D.from_numpy(a) for a in (x, gamma, ctx, act_in, res))
        got = {}
        for entry in ("gemm", "mm"):
            out = {k: D(4 * n * m) for k, m in sizes.items()}
            for buf in out.values():
                buf.upload(np.full(buf.nbytes // 4, np.nan, np.float32))
            normalized = D.from_numpy(np.full((n, H), np.nan, np.float32))
            _run_all(gpu, entry, dW, ld, bp, dims, n, position, dx, dg, dctx, dact, dres, out, normalized, ws, wsb)
            gpu.synchronize()
            got[entry] = {k: out[k].download(np.float32, (n, m)) for k, m in sizes.items()}
            got[entry]["xn"] = normalized.download(np.float32, (n, H))
        assert np.array_equal(got["gemm"]["xn"].view(np.uint32), got["mm"]["xn"].view(np.uint32)), n
        ref = _mm_reference(W, B, x, gamma, ctx, act_in, res, dims, position)
        for k in sizes:
            g = got["gemm"][k].astype(np.float64)
            rms = np.sqrt((ref[k] ** 2).mean())
            err = np.abs(g - ref[k]).max()
            assert np.isfinite(g).all() and err <= 1e-4 * rms, f"{k}: rows={n} position={position} err={err:.3g}"
            dmm = (np.abs(g - got["mm"][k]) / (np.abs(ref[k]) + rms)).max()
            assert dmm <= 5e-5, f"{k}: rows={n} position={position} gemm-mm={dmm:.3g} of |ref| + rms"


def test_gemm_residual_in_place_and_repeated_calls(gpu):
    """y aliasing the residual, and one workspace reused by calls of other
    sizes one after another (the second smaller): each result as the float64
    restatement."""
    lib, D = gpu.gemm_lib(), gpu.DeviceBuffer
    rng = np.random.default_rng(11)
    K, N = 1024, 512
    W = _bf16_rows(rng, N, K, 0.03)
    dW = D.from_numpy(W)
    wsb = lib.skv_prompt_gemm_workspace_bytes(200, K, N)
    ws = D(wsb)
    w64 = oracle.bf16_to_f32(W).astype(np.float64)
    for n in (200, 8, 131):
        x = rng.standard_normal((n, K)).astype(np.float32)
        res = rng.standard_normal((n, N)).astype(np.float32)
        dx, dy = D.from_numpy(x), D.from_numpy(res)
        gpu._check(lib.skv_linear_residual_gemm_f32(dx.ptr, n, dW.ptr, gpu.DTYPE_BF16, 1, K, K, N, None, dy.ptr,
                                                    dy.ptr, ws.ptr, wsb, None))
        gpu.synchronize()
        ref = x.astype(np.float64) @ w64.T + res
        got = dy.download(np.float32, (n, N)).astype(np.float64)
        assert np.abs(got - ref).max() <= 1e-4 * np.sqrt((ref ** 2).mean()), n


def test_gemm_projections_refuse_unsupported_shapes(gpu):
    """fp32 weights, in_dim not a multiple of 8, an output count not a multiple
    of 8, a bias not 16-byte aligned: SKV_ERR_UNSUPPORTED and nothing
    written."""
    lib, D = gpu.gemm_lib(), gpu.DeviceBuffer
    y = D.from_numpy(np.full((3, 64), 7.0, np.float32))
    res = D.from_numpy(np.zeros((3, 64), np.float32))
    for K, out_dim, dt in ((1024, 64, gpu.DTYPE_FP32), (1020, 64, gpu.DTYPE_BF16), (1024, 60, gpu.DTYPE_BF16)):
        esz = 2 if dt == gpu.DTYPE_BF16 else 4
        w = D(64 * K * esz)
        x = D.from_numpy(np.ones((3, K), np.float32))
        wsb = lib.skv_prompt_gemm_workspace_bytes(3, K, out_dim)
        ws = D(wsb)
        rc = lib.skv_linear_residual_gemm_f32(x.ptr, 3, w.ptr, dt, 1, K, K, out_dim, None, res.ptr, y.ptr, ws.ptr,
                                              wsb, None)
        assert rc == gpu.SKV_ERR_UNSUPPORTED, (K, out_dim, dt)
    K, bias = 1024, D(4 * 65)
    w, x = D(64 * K * 2), D.from_numpy(np.ones((3, K), np.float32))
    wsb = lib.skv_prompt_gemm_workspace_bytes(3, K, 64)
    ws = D(wsb)
    rc = lib.skv_linear_residual_gemm_f32(x.ptr, 3, w.ptr, gpu.DTYPE_BF16, 1, K, K, 64, bias.ptr + 4, res.ptr, y.ptr,
                                          ws.ptr, wsb, None)
    assert rc == gpu.SKV_ERR_UNSUPPORTED
    gpu.synchronize()
    assert np.array_equal(y.download(np.float32, (3, 64)), np.full((3, 64), 7.0, np.float32))


@pytest.mark.parametrize("dims", [(2048, 32, 4, 64, 5632), (1024, 8, 2, 128, 1536)], ids=["tinyllama", "hd128"])
@pytest.mark.parametrize("with_bias", [False, True])
@pytest.mark.parametrize("packed", [False, True], ids=["separate", "packed"])
def test_ffn_gemm_matches_two_calls_and_float64(gpu, dims, with_bias, packed):
    """skv_ffn_swiglu_gemm_f32 (rmsnorm, gate/up, SwiGLU written straight as
    down_proj's split operand, down_proj, + x) in place (y = x): within 1e-4
    of the rms of the float64 result, within 5e-5 (|ref| + rms) of
    skv_fused_gate_up_swiglu_gemm_f32 followed by skv_linear_residual_gemm_f32
    (the same operands; hipBLASLt may sum split K in another order), and the
    normalised rows bit-identical."""
    H, _, _, _, inter = dims
    rng = np.random.default_rng(3 * H + inter + with_bias + 2 * packed)
    lib, D = gpu.gemm_lib(), gpu.DeviceBuffer
    W = {n: _bf16_rows(rng, o, i, 0.03) for n, o, i in (("g", inter, H), ("u", inter, H), ("d", H, inter))}
    dW, ld = _upload_weights(D, W, ["g", "u", "d"], {}, False)
    if packed:
        base = D.from_numpy(np.concatenate([W["g"], W["u"]]))
        dW["g"], dW["u"] = _At(base, 0), _At(base, 2 * inter * H)
    B = {n: (rng.standard_normal(W[n].shape[0]).astype(np.float32) if with_bias else None) for n in "gud"}
    dB = {n: (D.from_numpy(B[n]) if B[n] is not None else None) for n in "gud"}
    bp = lambda n: dB[n].ptr if dB[n] is not None else None
    eps = ctypes.c_float(1e-5)
    max_rows = 1024
    wsb = lib.skv_prompt_gemm_workspace_bytes(max_rows, max(H, inter), max(2 * inter, H))
    ws = D(wsb)
    w64 = {n: oracle.bf16_to_f32(W[n]).astype(np.float64) for n in "gud"}
    b64 = {n: (B[n].astype(np.float64) if B[n] is not None else 0.0) for n in "gud"}
    for n in (1, 37, 300, max_rows):
        x = rng.standard_normal((n, H)).astype(np.float32)
        gamma = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
        dx, dg = D.from_numpy(x), D.from_numpy(gamma)
        # two calls: act through memory
        act, xn, y2 = D(4 * n * inter), D(4 * n * H), D(4 * n * H)
        gpu._check(lib.skv_fused_gate_up_swiglu_gemm_f32(dx.ptr, n, dg.ptr, eps, dW["g"].ptr, dW["u"].ptr,
                                                         gpu.DTYPE_BF16, 1, H, H, bp("g"), bp("u"), H, inter, act.ptr,
                                                         xn.ptr, ws.ptr, wsb, None))
        gpu._check(lib.skv_linear_residual_gemm_f32(act.ptr, n, dW["d"].ptr, gpu.DTYPE_BF16, 1, inter, inter, H,
                                                    bp("d"), dx.ptr, y2.ptr, ws.ptr, wsb, None))
        # one call, in place
        dy, xn1 = D.from_numpy(x), D(4 * n * H)
        gpu._check(lib.skv_ffn_swiglu_gemm_f32(dy.ptr, n, dg.ptr, eps, dW["g"].ptr, dW["u"].ptr, dW["d"].ptr,
                                               gpu.DTYPE_BF16, 1, H, H, inter, bp("g"), bp("u"), bp("d"), H, inter,
                                               dy.ptr, xn1.ptr, ws.ptr, wsb, None))
        gpu.synchronize()
        one, two = dy.download(np.float32, (n, H)), y2.download(np.float32, (n, H))
        assert np.array_equal(xn1.download(np.uint32, (n, H)), xn.download(np.uint32, (n, H))), n
        x64 = x.astype(np.float64)
        xn64 = x64 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + 1e-5) * gamma.astype(np.float64)
        g, u = xn64 @ w64["g"].T + b64["g"], xn64 @ w64["u"].T + b64["u"]
        ref = (g / (1.0 + np.exp(-g)) * u) @ w64["d"].T + b64["d"] + x64
        rms = np.sqrt((ref ** 2).mean())
        err = np.abs(one.astype(np.float64) - ref).max()
        assert np.isfinite(one).all() and err <= 1e-4 * rms, (n, err)
        dtwo = (np.abs(one.astype(np.float64) - two) / (np.abs(ref) + rms)).max()
        assert dtwo <= 5e-5, (n, dtwo)


def _digest_of_prompt_gemms():
    """SHA-256 of the outputs of a packed q/k/v GEMM call and a feed-forward
    GEMM call over seeded inputs (TinyLlama shapes, 256 and 2,048 tokens): the
    bits a process computes, for the cross-process comparison below."""
    import hashlib

    import stratakv_amd as skv

    skv.require_gpu()
    glib, D = skv.gemm_lib(), skv.DeviceBuffer
    H, Hq, Hkv, hd, inter = 2048, 32, 4, 64, 5632
    rng = np.random.default_rng(20261202)
    shapes = (("q", Hq * hd, H), ("k", Hkv * hd, H), ("v", Hkv * hd, H), ("g", inter, H), ("u", inter, H),
              ("d", H, inter))
    W = {n: _bf16_rows(rng, o, i, 0.03) for n, o, i in shapes}
    dW, ld = _upload_weights(D, W, [n for n, _, _ in shapes], {}, True)
    eps = ctypes.c_float(1e-5)
    strides = (ctypes.c_int64 * 3)(ld["q"], ld["k"], ld["v"])
    h = hashlib.sha256()
    for n in (256, 2048):
        wsb = max(glib.skv_prompt_gemm_workspace_bytes(n, H, (Hq + 2 * Hkv) * hd),
                  glib.skv_prompt_gemm_workspace_bytes(n, inter, 2 * inter))
        ws = D(wsb)
        dx = D.from_numpy(rng.standard_normal((n, H)).astype(np.float32))
        dg = D.from_numpy((1 + 0.1 * rng.standard_normal(H)).astype(np.float32))
        q, k, v, xn, y = D(4 * n * Hq * hd), D(4 * n * Hkv * hd), D(4 * n * Hkv * hd), D(4 * n * H), D(4 * n * H)
        skv._check(glib.skv_fused_qkv_gemm_f32(dx.ptr, n, dg.ptr, eps, dW["q"].ptr, dW["k"].ptr, dW["v"].ptr,
                                               skv.DTYPE_BF16, 1, strides, None, None, None, H, Hq, Hkv, hd, 3,
                                               q.ptr, k.ptr, v.ptr, xn.ptr, ws.ptr, wsb, None))
        skv._check(glib.skv_ffn_swiglu_gemm_f32(dx.ptr, n, dg.ptr, eps, dW["g"].ptr, dW["u"].ptr, dW["d"].ptr,
                                                skv.DTYPE_BF16, 1, ld["g"], ld["u"], ld["d"], None, None, None, H,
                                                inter, y.ptr, xn.ptr, ws.ptr, wsb, None))
        skv.synchronize()
        for buf, m in ((q, Hq * hd), (k, Hkv * hd), (v, Hkv * hd), (y, H)):
            h.update(buf.download(np.uint32, (n, m)).tobytes())
    return h.hexdigest()


def test_gemm_results_are_the_same_in_two_processes(gpu):
    """Each GEMM runs hipBLASLt's first-ranked algorithm for its shape, chosen
    by the library's heuristic and never by timing, so two fresh processes
    compute the same bits (and so does this one)."""
    import os
    import subprocess
    import sys

    here = os.path.dirname(os.path.abspath(__file__))
    code = (f"import sys; sys.path.insert(0, {here!r}); sys.path.insert(0, {os.path.dirname(here)!r}); "
            "import test_gpu_prompt_gemm as t; print(t._digest_of_prompt_gemms())")
    digests = []
    for _ in range(2):
        proc = subprocess.run([sys.executable, "-c", code], stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                              text=True, timeout=110)
        assert proc.returncode == 0, proc.stderr[-2000:]
        digests.append(proc.stdout.strip().splitlines()[-1])
    digests.append(_digest_of_prompt_gemms())
    assert digests[0] == digests[1] == digests[2], digests
