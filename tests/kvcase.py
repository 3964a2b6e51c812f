"""Shared builders for paged-KV test cases: block tables laid out the way a
fresh BlockPool hands blocks out, bf16 pools, queries, and the GPU/oracle runs.

The attention tolerance is the one stated for this path: |gpu - ref| <=
2e-3 + 1e-2 * |ref| elementwise, against the reference's fp32 loops (oracle).
"""
from __future__ import annotations

import math

import numpy as np

import oracle

ATOL = 2e-3
RTOL = 1e-2


def n_blocks(L: int, bs: int) -> int:
    return 0 if L <= 0 else -(-L // bs)


def make_tables(lens, bs: int, total_blocks: int, layout: str, rng: np.random.Generator,
                extra_cols: int = 0) -> np.ndarray:
    """Block tables [B, max_blocks] (int32, -1 padded).

    sequential  -- sequences take consecutive ids, one after the other (a fresh
                   LIFO pool hands out 0, 1, 2, ... when nothing was freed).
    round_robin -- one block per live sequence in turn (fragmented pool).
    random      -- disjoint slices of a random permutation of the pool.
    """
    nbs = [n_blocks(int(L), bs) for L in lens]
    need = sum(nbs)
    assert need <= total_blocks, "pool too small for the requested contexts"
    max_blocks = max(1, max(nbs) + extra_cols)
    t = np.full((len(lens), max_blocks), -1, np.int32)
    if layout == "sequential":
        nxt = 0
        for b, nb in enumerate(nbs):
            t[b, :nb] = np.arange(nxt, nxt + nb)
            nxt += nb
    elif layout == "round_robin":
        nxt = 0
        for k in range(max(nbs) if nbs else 0):
            for b, nb in enumerate(nbs):
                if k < nb:
                    t[b, k] = nxt
                    nxt += 1
    elif layout == "random":
        perm = rng.permutation(total_blocks).astype(np.int32)
        pos = 0
        for b, nb in enumerate(nbs):
            t[b, :nb] = perm[pos:pos + nb]
            pos += nb
    else:
        raise ValueError(layout)
    return t


def bf16_normal(rng: np.random.Generator, shape) -> np.ndarray:
    return oracle.f32_to_bf16(rng.standard_normal(shape, dtype=np.float32))


def make_case(B, Hq, Hkv, hd, bs, lens, total_blocks=None, layout="random", q_dtype="bf16",
              seed=0, extra_cols=0):
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, np.int32)
    need = sum(n_blocks(int(L), bs) for L in lens)
    if total_blocks is None:
        total_blocks = need + 7
    tables = make_tables(lens, bs, total_blocks, layout, rng, extra_cols)
    k_pool = bf16_normal(rng, (total_blocks, bs, Hkv, hd))
    v_pool = bf16_normal(rng, (total_blocks, bs, Hkv, hd))
    q32 = rng.standard_normal((B, Hq, hd), dtype=np.float32)
    if q_dtype == "bf16":
        q_dev = oracle.f32_to_bf16(q32)
        q_ref = oracle.bf16_to_f32(q_dev)
    else:
        q_dev = q32
        q_ref = q32
    return dict(B=B, Hq=Hq, Hkv=Hkv, hd=hd, bs=bs, lens=lens, total_blocks=total_blocks,
                tables=tables, k_pool=k_pool, v_pool=v_pool, q_dev=q_dev, q_ref=q_ref,
                q_dtype=q_dtype, scale=1.0 / math.sqrt(hd))


def oracle_decode(case, precision="f32"):
    return oracle.paged_decode(case["q_ref"], case["k_pool"], case["v_pool"], case["tables"],
                               case["lens"], case["Hkv"], case["bs"], case["scale"],
                               precision=precision)


def gpu_decode(skv, case, single: bool = False, poison: bool = True):
    """Run the case through the C ABI; returns out [B, Hq, hd] float32."""
    c = case
    dq = skv.DeviceBuffer.from_numpy(c["q_dev"])
    dk = skv.DeviceBuffer.from_numpy(c["k_pool"])
    dv = skv.DeviceBuffer.from_numpy(c["v_pool"])
    dt = skv.DeviceBuffer.from_numpy(c["tables"])
    dl = skv.DeviceBuffer.from_numpy(c["lens"])
    out_shape = (c["B"], c["Hq"], c["hd"])
    dout = skv.DeviceBuffer(4 * int(np.prod(out_shape)))
    if poison:  # NaN everywhere so a missing store shows up
        dout.upload(np.full(out_shape, np.nan, np.float32))
    qd = skv.DTYPE_BF16 if c["q_dtype"] == "bf16" else skv.DTYPE_FP32
    if single:
        assert c["B"] == 1 and c["q_dtype"] == "fp32"
        ws, wsb = skv.single_decode_workspace(c["Hq"], c["Hkv"], c["hd"])
        skv.paged_attention_decode(dq, dk, dv, c["total_blocks"], dt, dout, int(c["lens"][0]),
                                   c["bs"], c["Hq"], c["Hkv"], c["hd"], c["scale"], ws, wsb)
    else:
        ws, wsb = skv.decode_workspace(c["B"], c["Hq"], c["Hkv"], c["hd"])
        skv.paged_decode(dq, qd, dk, dv, c["total_blocks"], dt, c["tables"].shape[1], dl, c["B"],
                         c["Hq"], c["Hkv"], c["hd"], c["bs"], c["scale"], dout, ws, wsb)
    skv.synchronize()
    return dout.download(np.float32, out_shape)


def assert_close(got, ref, atol=ATOL, rtol=RTOL, what=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape
    assert np.isfinite(got).all(), f"{what}: non-finite output (missing store?)"
    err = np.abs(got - ref)
    bound = atol + rtol * np.abs(ref)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(f"{what}: {int(bad.sum())} of {err.size} elements out of tolerance; "
                             f"worst at {i}: got {got[i]!r} ref {ref[i]!r} (max abs err {err.max():.3e})")
    return float(err.max())
