"""Pins the oracle's paged decode attention (src/layers/attention.cpp:263-337).

Independent checks, each chosen so a plausible slip fails at least one:
* the reference's own closed-form RoPE case (tests/phase6_smoke.cpp:60-96):
  scale, softmax direction, output weighting;
* float64 brute force written here from the formula (not the oracle loops);
* special cases: L = 1 gives v_0; equal keys give the mean of V; a dominant
  key selects its value; queries that are equal within a GQA group give equal
  outputs (group mapping); moving blocks in the pool while keeping the
  logical order leaves the output unchanged (table indirection);
* the reference's own PagedAttention::forward (oracle/_ref) run token by token
  with identity projections, MHA and GQA, on non-contiguous pages.
"""
import math

import numpy as np
import pytest

import oracle
from kvcase import make_case, oracle_decode


def _fp32_pool_case(k_rows, v_rows, q, Hkv, hd, bs, table):
    """Place rows [L, Hkv, hd] into an fp32 pool through `table`."""
    L = k_rows.shape[0]
    total = int(max(table)) + 1
    kp = np.zeros((total, bs, Hkv, hd), np.float32)
    vp = np.zeros_like(kp)
    for t in range(L):
        kp[table[t // bs], t % bs] = k_rows[t]
        vp[table[t // bs], t % bs] = v_rows[t]
    return kp, vp


def test_phase6_rope_closed_form():
    # hidden 4, 2 heads (hd 2), MHA.  Token 0 x=[1,0,1,0] at position 0 (no
    # rotation); token 1 x=[0,1,0,1] at position 1 rotates each head pair by 1 rad.
    s, c = math.sin(1.0), math.cos(1.0)
    k_rows = np.array([[[1, 0], [1, 0]], [[-s, c], [-s, c]]], np.float32)
    v_rows = np.array([[[1, 0], [1, 0]], [[0, 1], [0, 1]]], np.float32)
    q = np.array([[[-s, c], [-s, c]]], np.float32)
    kp, vp = _fp32_pool_case(k_rows, v_rows, q, 2, 2, 2, [0])
    out = oracle.paged_decode(q, kp, vp, np.array([[0]], np.int32), np.array([2], np.int32), 2, 2,
                              1.0 / math.sqrt(2.0))
    w = math.exp(1 / math.sqrt(2)) / (math.exp(-s / math.sqrt(2)) + math.exp(1 / math.sqrt(2)))
    np.testing.assert_allclose(out[0, :, 0], 1.0 - w, atol=1e-5)
    np.testing.assert_allclose(out[0, :, 1], w, atol=1e-5)
    first = oracle.paged_decode(q, kp, vp, np.array([[0]], np.int32), np.array([1], np.int32), 2, 2,
                                1.0 / math.sqrt(2.0))
    np.testing.assert_allclose(first[0, 0], [1.0, 0.0], atol=1e-5)


def _brute_force(case):
    """softmax(scale * q.k) . v straight from the definition, in float64."""
    B, Hq, Hkv, hd, bs = case["B"], case["Hq"], case["Hkv"], case["hd"], case["bs"]
    kp = oracle.bf16_to_f32(case["k_pool"]).astype(np.float64)
    vp = oracle.bf16_to_f32(case["v_pool"]).astype(np.float64)
    out = np.zeros((B, Hq, hd))
    for b in range(B):
        L = int(case["lens"][b])
        if L <= 0:
            continue
        pos = np.arange(L)
        blocks = case["tables"][b][pos // bs]
        K = kp[blocks, pos % bs]          # [L, Hkv, hd]
        V = vp[blocks, pos % bs]
        for h in range(Hq):
            g = h // (Hq // Hkv)
            sc = K[:, g, :] @ case["q_ref"][b, h].astype(np.float64) * case["scale"]
            p = np.exp(sc - sc.max())
            out[b, h] = (p / p.sum()) @ V[:, g, :]
    return out


@pytest.mark.parametrize("geom,bs", [((8, 2, 16), 4), ((4, 4, 8), 3), ((6, 3, 32), 16), ((32, 4, 64), 16)])
def test_matches_float64_brute_force(geom, bs):
    Hq, Hkv, hd = geom
    case = make_case(3, Hq, Hkv, hd, bs, [1, 37, 200], layout="random", seed=hd)
    got = oracle_decode(case)
    ref = _brute_force(case)
    np.testing.assert_allclose(got, ref, rtol=2e-5, atol=2e-6)
    np.testing.assert_allclose(oracle_decode(case, "f64"), ref, rtol=1e-10, atol=1e-12)


def test_single_token_returns_its_value():
    case = make_case(2, 8, 2, 16, 4, [1, 1], seed=3)
    got = oracle_decode(case)
    for b in range(2):
        blk = case["tables"][b, 0]
        v0 = oracle.bf16_to_f32(case["v_pool"][blk, 0])   # [Hkv, hd]
        np.testing.assert_array_equal(got[b], np.repeat(v0, 4, axis=0))


def test_equal_keys_average_values():
    case = make_case(1, 4, 2, 8, 4, [10], seed=4)
    case["k_pool"][:] = case["k_pool"][0, 0]
    got = oracle_decode(case)
    tbl = case["tables"][0]
    V = np.stack([oracle.bf16_to_f32(case["v_pool"][tbl[t // 4], t % 4]) for t in range(10)])
    np.testing.assert_allclose(got[0], np.repeat(V.mean(0), 2, axis=0), rtol=1e-5, atol=1e-6)


def test_dominant_key_selects_its_value():
    case = make_case(1, 2, 1, 8, 4, [9], seed=5, q_dtype="fp32")
    case["q_ref"][:] = 0.0
    case["q_ref"][0, :, 0] = 1.0
    case["k_pool"][:] = 0
    tbl = case["tables"][0]
    case["k_pool"][tbl[6 // 4], 6 % 4, 0, 0] = oracle.f32_to_bf16(np.array([400.0], np.float32))[0]
    got = oracle_decode(case)
    v6 = oracle.bf16_to_f32(case["v_pool"][tbl[1], 2, 0])
    np.testing.assert_allclose(got[0, 0], v6, rtol=1e-5, atol=1e-6)


def test_group_mapping_h_over_g():
    Hq, Hkv, hd = 8, 2, 16
    case = make_case(1, Hq, Hkv, hd, 4, [50], seed=6, q_dtype="fp32")
    case["q_ref"][0, :4] = case["q_ref"][0, 0]      # heads 0-3 read kv head 0
    case["q_ref"][0, 4:] = case["q_ref"][0, 0]      # heads 4-7 read kv head 1
    got = oracle_decode(case)
    assert np.array_equal(got[0, 0], got[0, 3]) and np.array_equal(got[0, 4], got[0, 7])
    assert not np.allclose(got[0, 0], got[0, 4])


def test_block_placement_invariance():
    case = make_case(2, 8, 2, 16, 4, [23, 41], layout="sequential", seed=8)
    base = oracle_decode(case)
    rng = np.random.default_rng(1)
    perm = rng.permutation(case["total_blocks"])      # block i moves to perm[i]
    moved = dict(case)
    moved["k_pool"] = np.empty_like(case["k_pool"])
    moved["v_pool"] = np.empty_like(case["v_pool"])
    moved["k_pool"][perm] = case["k_pool"]
    moved["v_pool"][perm] = case["v_pool"]
    moved["tables"] = np.where(case["tables"] >= 0, perm[np.maximum(case["tables"], 0)], -1).astype(np.int32)
    np.testing.assert_array_equal(oracle_decode(moved), base)


@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built (needs the StrataKV sources)")
@pytest.mark.parametrize("heads,kv_heads,hidden,bs", [(2, 2, 16, 2), (4, 1, 32, 4), (8, 2, 64, 3)])
def test_matches_reference_paged_attention(heads, kv_heads, hidden, bs):
    T = 40
    total_blocks = 2 * (T // bs + 2)
    rng = np.random.default_rng(heads * 7 + bs)
    x = rng.standard_normal((T, hidden), dtype=np.float32)
    out_ref, q, k, v, table = oracle.ref_attention_trace(hidden, heads, kv_heads, total_blocks, bs, x)
    hd = hidden // heads
    assert any(table[i + 1] != table[i] + 1 for i in range(len(table) - 1)), "pages not interleaved"
    kp, vp = _fp32_pool_case(k.reshape(T, kv_heads, hd), v.reshape(T, kv_heads, hd), None,
                             kv_heads, hd, bs, table)
    kp = np.concatenate([kp, np.zeros((total_blocks - kp.shape[0],) + kp.shape[1:], np.float32)])
    vp = np.concatenate([vp, np.zeros((total_blocks - vp.shape[0],) + vp.shape[1:], np.float32)])
    tables = np.array([table], np.int32)
    for t in range(T):
        got = oracle.paged_decode(q[t].reshape(1, heads, hd), kp, vp, tables,
                                  np.array([t + 1], np.int32), kv_heads, bs, 1.0 / math.sqrt(hd))
        np.testing.assert_allclose(got.reshape(-1), out_ref[t], rtol=1e-5, atol=1e-6,
                                   err_msg=f"token {t}")
