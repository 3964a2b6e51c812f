"""skv_paged_decode_append_noalloc: the fused append + decode without a
workspace argument (its partial results live in the library's own device
array).  Two calls in a row, the second with a smaller input, each compared
with skv_paged_decode_append on the same inputs through the C ABI: pools and
outputs bit for bit (the scratch holds every shape's full persistent grid, so
both calls split the work identically), and both against the oracle (pools
bit-exact against its scatter, outputs within 2e-3 + 1e-2 |ref| of its fp32
loops over the appended pools)."""
import ctypes

import numpy as np
import pytest

import oracle
from kvcase import assert_close

from test_gpu_fused import _case

pytestmark = pytest.mark.gpu


def _call(skv, c, noalloc):
    B = len(c["lens"])
    dk = skv.DeviceBuffer.from_numpy(c["k_pool"])
    dv = skv.DeviceBuffer.from_numpy(c["v_pool"])
    dt = skv.DeviceBuffer.from_numpy(c["tables"])
    dl = skv.DeviceBuffer.from_numpy(c["lens"])
    dq = skv.DeviceBuffer.from_numpy(c["q_dev"])
    dkn = skv.DeviceBuffer.from_numpy(c["k_new"])
    dvn = skv.DeviceBuffer.from_numpy(c["v_new"])
    shape = (B, c["Hq"], c["hd"])
    dout = skv.DeviceBuffer(4 * int(np.prod(shape)))
    dout.upload(np.full(shape, np.nan, np.float32))  # a missing store shows up
    kvd = skv.DTYPE_BF16 if c["kv_dtype"] == "bf16" else skv.DTYPE_FP32
    qd = skv.DTYPE_BF16 if c["q_dtype"] == "bf16" else skv.DTYPE_FP32
    mb = c["tables"].shape[1]
    if noalloc:
        skv._check(skv.lib().skv_paged_decode_append_noalloc(
            dq.ptr, qd, dkn.ptr, dvn.ptr, kvd, dk.ptr, dv.ptr, c["total"], dt.ptr, mb, dl.ptr, B,
            c["Hq"], c["Hkv"], c["hd"], c["bs"], ctypes.c_float(c["scale"]), dout.ptr, None))
    else:
        ws, wsb = skv.decode_workspace(B, c["Hq"], c["Hkv"], c["hd"])
        skv.paged_decode_append(dq, qd, dkn, dvn, kvd, dk, dv, c["total"], dt, mb, dl, B, c["Hq"],
                                c["Hkv"], c["hd"], c["bs"], c["scale"], dout, ws, wsb)
    skv.synchronize()
    return (dout.download(np.float32, shape), dk.download(np.uint16, c["k_pool"].shape),
            dv.download(np.uint16, c["v_pool"].shape))


def test_noalloc_matches_decode_append_twice(gpu):
    # Llama-3-8B geometry with long, cut segments; then a smaller TinyLlama
    # call with fp32 queries and rows (the scratch keeps the first call's data).
    first = _case(32, 8, 128, 16, [3001, 17, 2500, 4096, 1, 900, 1600, 2222], "bf16", "bf16", seed=71)
    second = _case(32, 4, 64, 16, [700, 33, 260], "fp32", "fp32", seed=72)
    for c, what in ((first, "first call"), (second, "second call, smaller")):
        out_n, k_n, v_n = _call(gpu, c, noalloc=True)
        out_w, k_w, v_w = _call(gpu, c, noalloc=False)
        assert np.array_equal(k_n, k_w) and np.array_equal(v_n, v_w), f"{what}: pools differ"
        assert np.array_equal(out_n.view(np.uint32), out_w.view(np.uint32)), f"{what}: outputs differ"
        k_ref, v_ref = c["k_pool"].copy(), c["v_pool"].copy()
        B = len(c["lens"])
        oracle.kv_append(c["k_new"].reshape(B, -1), c["v_new"].reshape(B, -1), k_ref, v_ref, c["tables"],
                         c["lens"] - 1, B, 1, c["Hkv"], c["hd"], c["bs"])
        assert np.array_equal(k_n, k_ref) and np.array_equal(v_n, v_ref), f"{what}: pools vs oracle"
        ref = oracle.paged_decode(c["q_ref"], k_ref, v_ref, c["tables"], c["lens"], c["Hkv"], c["bs"],
                                  c["scale"])
        assert_close(out_n, ref, what=what)


def test_noalloc_validates_like_decode_append(gpu):
    lib = gpu.lib()
    rc = lib.skv_paged_decode_append_noalloc(None, gpu.DTYPE_BF16, None, None, gpu.DTYPE_BF16, None, None,
                                             16, None, 1, None, 1, 32, 8, 128, 16, ctypes.c_float(0.1),
                                             None, None)
    assert rc == gpu.SKV_ERR_INVALID_ARGUMENT
    assert "skv_paged_decode_append_noalloc" in lib.skv_last_error().decode()
