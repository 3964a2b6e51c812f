"""Pins the oracle's bf16 rules (src/cpu/tensor.cpp:193-229, gemm_cuda.cu:74-83).

Checks: the reference's own known-answer bytes (tests/phase7_smoke.cpp:41-53),
an independent nearest-value model computed in float64, and -- when
oracle/_ref was built -- Tensor::set_value of the reference itself on every
upper half-word and the rounding-critical lower half-words.
"""
import numpy as np
import pytest

import oracle


def _all_patterns():
    uppers = np.arange(0x10000, dtype=np.uint32)
    lowers = np.array([0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xC000, 0xFFFF], np.uint32)
    return (uppers[:, None] << 16 | lowers[None, :]).reshape(-1).view(np.float32)


def test_phase7_known_answer_bytes():
    # tests/phase7_smoke.cpp:41-53: 1.0 -> 80 3F, -2.5 -> 20 C0, 3.25 round-trips.
    h = oracle.f32_to_bf16(np.array([1.0, -2.5, 3.25], np.float32))
    raw = h.view(np.uint8)
    assert list(raw[:4]) == [0x80, 0x3F, 0x20, 0xC0]
    np.testing.assert_array_equal(oracle.bf16_to_f32(h), [1.0, -2.5, 3.25])


def test_widen_is_exact_for_every_pattern():
    h = np.arange(0x10000, dtype=np.uint16)
    expect = (h.astype(np.uint32) << 16).view(np.float32)
    got = oracle.bf16_to_f32(h)
    np.testing.assert_array_equal(got.view(np.uint32), expect.view(np.uint32))


def _nearest_model(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even to bf16 from float64 distances (finite inputs)."""
    x64 = x.astype(np.float64)
    bits = x.view(np.uint32)
    lo_bits = (bits >> 16).astype(np.uint32)           # toward zero
    lo = (lo_bits << 16).view(np.float32).astype(np.float64)
    hi_bits = lo_bits + 1                                # one bf16 ulp away from zero
    hi = np.where((hi_bits & 0x7F80) == 0x7F80,          # would become inf: use 2^128
                  np.copysign(2.0**128, x64),
                  ((hi_bits << 16).astype(np.uint32)).view(np.float32).astype(np.float64))
    dlo, dhi = np.abs(x64 - lo), np.abs(hi - x64)
    pick_hi = (dhi < dlo) | ((dhi == dlo) & ((lo_bits & 1) == 1))
    return np.where(pick_hi, hi_bits, lo_bits).astype(np.uint16)


def test_rne_matches_nearest_value_model():
    x = _all_patterns()
    finite = np.isfinite(x)
    got = oracle.f32_to_bf16(x[finite])
    np.testing.assert_array_equal(got, _nearest_model(x[finite]))
    rng = np.random.default_rng(0)
    y = rng.standard_normal(200000).astype(np.float32) * np.float32(1e3)
    np.testing.assert_array_equal(oracle.f32_to_bf16(y), _nearest_model(y))


def test_truncation_drops_low_half():
    x = _all_patterns()
    got = np.array([oracle.lib().oracle_f32_to_bf16_trunc(float(v)) for v in x[:5000]], np.uint16)
    np.testing.assert_array_equal(got, (x[:5000].view(np.uint32) >> 16).astype(np.uint16))


@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built (needs the StrataKV sources)")
def test_rne_matches_reference_set_value_including_nan():
    x = _all_patterns()
    np.testing.assert_array_equal(oracle.f32_to_bf16(x), oracle.ref_bf16_rne(x))
