"""Pins the oracle's chunked prefill attention (oracle.paged_prefill): the
causal semantics of PagedAttention::forward for a multi-token chunk
(src/layers/attention.cpp:197-337: every token of the chunk is appended, then
attends to positions 0..its own, earlier chunk tokens included).

Checks, each chosen so a plausible slip fails one of them:
* the reference's own PagedAttention::forward (oracle/_ref) fed chunks of
  1, 5, 16 and 33 tokens, MHA and GQA, non-contiguous pages: an off-by-one in
  the causal limit, a chunk that sees its own future or does not see its
  earlier tokens, or a wrong position base all change the output;
* float64 brute force from the definition over a batch of sequences with
  different chunk and context lengths (sequence/offset bookkeeping);
* the last token of a chunk equals a decode at the full context (reduces to
  the pinned decode oracle).
"""
import math

import numpy as np
import pytest

import oracle
from kvcase import make_tables


def _pool_from_rows(k_rows, v_rows, Hkv, hd, bs, table, total):
    kp = np.zeros((total, bs, Hkv, hd), np.float32)
    vp = np.zeros_like(kp)
    for t in range(k_rows.shape[0]):
        kp[table[t // bs], t % bs] = k_rows[t]
        vp[table[t // bs], t % bs] = v_rows[t]
    return kp, vp


@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built (needs the StrataKV sources)")
@pytest.mark.parametrize("heads,kv_heads,hidden,bs", [(2, 2, 16, 4), (4, 1, 32, 4), (8, 2, 64, 3)])
def test_matches_reference_chunked_forward(heads, kv_heads, hidden, bs):
    chunks = [5, 1, 16, 33, 2]
    T = sum(chunks)
    total_blocks = 2 * (T // bs + 4)
    rng = np.random.default_rng(heads * 11 + bs)
    x = rng.standard_normal((T, hidden), dtype=np.float32)
    out_ref, q, k, v, table = oracle.ref_prefill_trace(hidden, heads, kv_heads, total_blocks, bs, x,
                                                       chunks)
    hd = hidden // heads
    assert any(table[i + 1] != table[i] + 1 for i in range(len(table) - 1)), "pages not interleaved"
    kp, vp = _pool_from_rows(k.reshape(T, kv_heads, hd), v.reshape(T, kv_heads, hd), kv_heads, hd,
                             bs, table, total_blocks)
    tables = np.array([table], np.int32)
    t0 = 0
    for n in chunks:
        # The chunk as one prefill call: n tokens ending at context t0 + n.
        got = oracle.paged_prefill(q[t0:t0 + n].reshape(n, heads, hd), kp, vp, tables,
                                   np.array([0, n]), np.array([t0 + n]), kv_heads, bs,
                                   1.0 / math.sqrt(hd))
        np.testing.assert_allclose(got.reshape(n, hidden), out_ref[t0:t0 + n], rtol=1e-5, atol=1e-6,
                                   err_msg=f"chunk at {t0} of {n} tokens")
        t0 += n


def _brute_force(q, kp, vp, tables, offsets, lens, Hkv, bs, scale):
    N, Hq, hd = q.shape
    G = Hq // Hkv
    out = np.zeros((N, Hq, hd))
    K = oracle.bf16_to_f32(kp).astype(np.float64)
    V = oracle.bf16_to_f32(vp).astype(np.float64)
    for b in range(len(lens)):
        n = offsets[b + 1] - offsets[b]
        for i in range(n):
            p = lens[b] - n + i
            pos = np.arange(p + 1)
            blocks = tables[b][pos // bs]
            for h in range(Hq):
                kk = K[blocks, pos % bs, h // G]
                vv = V[blocks, pos % bs, h // G]
                s = kk @ q[offsets[b] + i, h].astype(np.float64) * scale
                w = np.exp(s - s.max())
                out[offsets[b] + i, h] = (w / w.sum()) @ vv
    return out


def test_batch_matches_float64_brute_force():
    rng = np.random.default_rng(3)
    Hq, Hkv, hd, bs = 8, 2, 16, 4
    lens = np.array([9, 1, 40, 17], np.int32)          # contexts after the chunk
    chunk = np.array([9, 1, 5, 16])                     # tokens of each chunk
    offsets = np.concatenate([[0], np.cumsum(chunk)])
    total = sum(-(-int(L) // bs) for L in lens) + 3
    tables = make_tables(lens, bs, total, "random", rng)
    kp = oracle.f32_to_bf16(rng.standard_normal((total, bs, Hkv, hd), dtype=np.float32))
    vp = oracle.f32_to_bf16(rng.standard_normal((total, bs, Hkv, hd), dtype=np.float32))
    q = rng.standard_normal((int(offsets[-1]), Hq, hd), dtype=np.float32)
    got = oracle.paged_prefill(q, kp, vp, tables, offsets, lens, Hkv, bs, 1.0 / math.sqrt(hd))
    ref = _brute_force(q, kp, vp, tables, offsets, lens, Hkv, bs, 1.0 / math.sqrt(hd))
    np.testing.assert_allclose(got, ref, rtol=2e-5, atol=2e-6)


def test_last_chunk_token_is_a_decode():
    rng = np.random.default_rng(4)
    Hq, Hkv, hd, bs = 4, 4, 8, 2
    lens = np.array([11], np.int32)
    total = 8
    tables = make_tables(lens, bs, total, "random", rng)
    kp = oracle.f32_to_bf16(rng.standard_normal((total, bs, Hkv, hd), dtype=np.float32))
    vp = oracle.f32_to_bf16(rng.standard_normal((total, bs, Hkv, hd), dtype=np.float32))
    q = rng.standard_normal((6, Hq, hd), dtype=np.float32)
    pre = oracle.paged_prefill(q, kp, vp, tables, np.array([0, 6]), lens, Hkv, bs, 0.3)
    dec = oracle.paged_decode(q[5:6], kp, vp, tables, lens, Hkv, bs, 0.3)
    np.testing.assert_array_equal(pre[5:6], dec)
    first = oracle.paged_decode(q[0:1], kp, vp, tables, np.array([6], np.int32), Hkv, bs, 0.3)
    np.testing.assert_array_equal(pre[0:1], first)
