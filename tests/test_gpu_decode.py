"""Paged decode attention on the GPU (through the C ABI) against the oracle.

Tolerance: |gpu - ref| <= 2e-3 + 1e-2 * |ref| against the reference's fp32
two-pass loops (src/layers/attention.cpp:263-337), fp32 accumulation on the GPU.
"""
import math

import numpy as np
import pytest

import oracle
from kvcase import assert_close, gpu_decode, make_case, oracle_decode

pytestmark = pytest.mark.gpu

TL = (32, 4, 64)     # TinyLlama: Hq, Hkv, hd (G = 8)
L3 = (32, 8, 128)    # Llama-3-8B (G = 4)
L70 = (64, 8, 128)   # Llama-2-70B style (G = 8)


def _check(skv, case, what, single=False):
    got = gpu_decode(skv, case, single=single)
    ref = oracle_decode(case)
    err = assert_close(got, ref, what=what)
    truth = oracle_decode(case, precision="f64")
    # The GPU result is at least as close to the float64 truth as the bound allows.
    assert_close(got, truth, what=what + " vs f64")
    return err


@pytest.mark.parametrize("L", [1, 2, 15, 16, 17, 64, 65, 257, 4097])
def test_single_sequence_tinyllama_lengths(gpu, L):
    Hq, Hkv, hd = TL
    case = make_case(1, Hq, Hkv, hd, 16, [L], layout="random", seed=L)
    _check(gpu, case, f"TL L={L}")


@pytest.mark.parametrize("geom", [TL, L3, L70, (8, 8, 64), (16, 8, 128), (8, 4, 64)],
                         ids=["tl", "l3", "l70", "mha64", "g2_128", "g2_64"])
@pytest.mark.parametrize("q_dtype", ["bf16", "fp32"])
def test_batched_geometries(gpu, geom, q_dtype):
    Hq, Hkv, hd = geom
    lens = [1, 33, 300, 1024, 2049, 16, 5000, 7]
    case = make_case(len(lens), Hq, Hkv, hd, 16, lens, layout="random", q_dtype=q_dtype, seed=hd + Hq)
    _check(gpu, case, f"geom={geom} q={q_dtype}")


@pytest.mark.parametrize("B", [64, 3000])
@pytest.mark.parametrize("geom", [TL, L3], ids=["tl", "l3"])
def test_many_short_segments_with_empty_ones(gpu, geom, B):
    """Stream-K over short segments (1-5 blocks, a fifth of the sequences
    empty) in tables wider than the short-table limit.  The split puts empty
    slots before every segment's blocks, so ranges begin and end among them.
    At B=64 the ranges are 4 slots wide: some hold no block at all, and one
    segment is cut by several ranges."""
    Hq, Hkv, hd = geom
    rng = np.random.default_rng(B + hd)
    lens = rng.integers(1, 80, B).astype(np.int32)
    lens[rng.random(B) < 0.2] = 0
    case = make_case(B, Hq, Hkv, hd, 16, lens, layout="random", seed=B, extra_cols=20)
    assert case["tables"].shape[1] > 16   # the stream-K kernel, not the short-table one
    _check(gpu, case, f"short segments geom={geom} B={B}")


@pytest.mark.parametrize("layout", ["sequential", "round_robin", "random"])
def test_table_layouts(gpu, layout):
    Hq, Hkv, hd = L3
    lens = [3000, 100, 2500, 17, 4096]
    case = make_case(len(lens), Hq, Hkv, hd, 16, lens, layout=layout, seed=7)
    _check(gpu, case, f"layout={layout}")


@pytest.mark.parametrize("geom,bs", [((12, 4, 64), 16), ((8, 2, 96), 16), ((4, 4, 32), 8),
                                     ((16, 4, 128), 32), ((8, 1, 256), 16), ((6, 3, 40), 5),
                                     ((32, 4, 64), 1)],
                         ids=["g3", "hd96", "bs8", "bs32", "hd256", "odd", "bs1"])
def test_generic_path_shapes(gpu, geom, bs):
    """Shapes outside the fast kernels (any block size, head_dim <= 512, any group)."""
    Hq, Hkv, hd = geom
    lens = [1, 70, 513, 9]
    case = make_case(len(lens), Hq, Hkv, hd, bs, lens, layout="random", seed=bs + hd)
    _check(gpu, case, f"generic geom={geom} bs={bs}")


def test_single_entry_point_matches_reference_signature(gpu):
    """skv_paged_attention_decode: the reference's argument list (fp32 query)."""
    Hq, Hkv, hd = TL
    for L in (1, 16, 100, 4097):
        case = make_case(1, Hq, Hkv, hd, 16, [L], layout="random", q_dtype="fp32", seed=L + 3)
        _check(gpu, case, f"single L={L}", single=True)


def test_zero_length_and_padding_columns(gpu):
    """context_lens <= 0 gives zeros; table columns past a sequence are never read."""
    Hq, Hkv, hd = L3
    lens = [0, 40, -3, 1]
    case = make_case(len(lens), Hq, Hkv, hd, 16, lens, layout="random", seed=11, extra_cols=3)
    case["tables"][case["tables"] < 0] = 2**30  # garbage ids beyond each sequence
    got = gpu_decode(gpu, case)
    assert np.all(got[0] == 0) and np.all(got[2] == 0)
    ref = oracle_decode(dict(case, tables=np.where(case["tables"] >= case["total_blocks"], -1,
                                                   case["tables"])))
    assert_close(got, ref, what="zero-length batch")


def test_invalid_last_block_is_skipped(gpu):
    """A table entry outside the pool is not read (the kernels never fault on it)."""
    Hq, Hkv, hd = TL
    case = make_case(1, Hq, Hkv, hd, 16, [16 * 5], layout="random", seed=5)
    bad = dict(case)
    bad["tables"] = case["tables"].copy()
    bad["tables"][0, 4] = case["total_blocks"] + 100
    got = gpu_decode(gpu, bad)
    ref = oracle_decode(dict(case, lens=np.array([16 * 4], np.int32)))
    assert_close(got, ref, what="invalid last block")


def test_repeated_and_changed_calls(gpu):
    """Outputs are recomputed, not accumulated, across calls (and workspace reuse)."""
    Hq, Hkv, hd = L3
    a = make_case(3, Hq, Hkv, hd, 16, [5000, 64, 2000], seed=1)
    b = make_case(3, Hq, Hkv, hd, 16, [100, 3000, 1], seed=2)
    for case in (a, b, a):
        assert_close(gpu_decode(gpu, case), oracle_decode(case), what="repeat")


def test_group_sharing_identical_queries(gpu):
    """All query heads of a group with the same q give identical outputs."""
    Hq, Hkv, hd = L70
    case = make_case(2, Hq, Hkv, hd, 16, [777, 2048], seed=9)
    G = Hq // Hkv
    q = case["q_dev"].reshape(2, Hkv, G, hd)
    q[:] = q[:, :, :1, :]
    case["q_ref"] = oracle.bf16_to_f32(case["q_dev"])
    got = gpu_decode(gpu, case).reshape(2, Hkv, G, hd)
    assert np.array_equal(got, np.broadcast_to(got[:, :, :1, :], got.shape))


@pytest.mark.parametrize("geom", [TL, L3, L70, (8, 8, 64), (16, 1, 128), (16, 1, 64), (4, 4, 128)],
                         ids=["tl", "l3", "l70", "mha64", "g16_128", "g16_64", "mha128"])
@pytest.mark.parametrize("q_dtype", ["bf16", "fp32"])
def test_short_tables_one_workgroup_per_head(gpu, geom, q_dtype):
    """Tables of at most 12 (head_dim 64) or 8 (head_dim 128) blocks: one
    workgroup per (sequence, kv head) whose wavefronts split the blocks and
    merge in LDS.  Ragged lengths cover 1..4 busy wavefronts, empty sequences
    and table columns past a sequence."""
    Hq, Hkv, hd = geom
    cap = 16 * (12 if hd == 64 else 8)
    lens = [1, 0, 16, 17, 48, 49, cap - 1, cap, 33, -2, 100 if hd == 64 else 97]
    case = make_case(len(lens), Hq, Hkv, hd, 16, lens, layout="random", q_dtype=q_dtype, seed=hd + Hkv)
    assert case["tables"].shape[1] * 16 == cap
    got = gpu_decode(gpu, case)
    assert np.all(got[1] == 0) and np.all(got[9] == 0)
    ref = oracle_decode(dict(case, tables=np.where(case["tables"] < 0, -1, case["tables"])))
    assert_close(got, ref, what=f"short tables geom={geom} q={q_dtype}")


def test_long_context_split_merge(gpu):
    """One 32k-token sequence: many partitions merged with the log-sum-exp rule."""
    Hq, Hkv, hd = L3
    case = make_case(1, Hq, Hkv, hd, 16, [32768], layout="random", seed=21)
    _check(gpu, case, "L3 32k")


@pytest.mark.parametrize("geom", [TL, L3, (8, 1, 256)], ids=["tl", "l3", "generic"])
def test_unused_slots_holding_nan_are_never_used(gpu, geom):
    """Slots past a context in its last block may hold anything (freed data,
    uninitialised memory); NaN bit patterns there must not reach the output."""
    Hq, Hkv, hd = geom
    lens = [17, 40, 1, 250]
    case = make_case(len(lens), Hq, Hkv, hd, 16, lens, layout="random", seed=13)
    for b, L in enumerate(lens):
        last = case["tables"][b, (L - 1) // 16]
        case["k_pool"][last, L % 16 or 16:] = 0xFFFF
        case["v_pool"][last, L % 16 or 16:] = 0xFFFF
    unused = np.ones(case["total_blocks"], bool)
    unused[case["tables"][case["tables"] >= 0]] = False
    case["k_pool"][unused] = 0xFFFF
    case["v_pool"][unused] = 0xFFFF
    _check(gpu, case, f"nan slots {geom}")
