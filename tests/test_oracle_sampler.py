"""The sampler oracle (oracle/sampler.py) against the reference's own Sampler
(src/generation/sampler.cpp, compiled into oracle/_ref): the same tokens for
the same logits, configuration and seed, over greedy, temperature, top-k,
top-p and combined filters, with ties and -0 in the logits; and the uniform
stream against std::mt19937 + generate_canonical.  CPU only."""
import ctypes
import os

import numpy as np
import pytest

from oracle import sampler as osamp

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = os.path.join(ROOT, "oracle", "_ref", "libstratakv_ref.so")


@pytest.fixture(scope="module")
def ref():
    if not os.path.exists(REF):
        pytest.skip("oracle/_ref is not built (the StrataKV sources are absent)")
    return ctypes.CDLL(REF)


def ref_rows(lib, logits, temp, k, p, seed):
    rows, vocab = logits.shape
    toks = np.zeros(rows, np.int32)
    failed = ctypes.c_int(-1)
    err = ctypes.create_string_buffer(256)
    rc = lib.ref_sample_rows(np.ascontiguousarray(logits, np.float32).ctypes.data_as(ctypes.c_void_p), rows, vocab,
                             ctypes.c_float(temp), k, ctypes.c_float(p), ctypes.c_uint32(seed),
                             toks.ctypes.data_as(ctypes.c_void_p), ctypes.byref(failed), err, 256)
    return rc, toks, err.value.decode()


def make_logits(rng, rows, vocab, kind):
    x = rng.standard_normal((rows, vocab)).astype(np.float32) * np.float32(2.0)
    if kind == "ties":
        x = np.round(x * 2) / 2          # many exact ties
        x[:, ::7] = 0.0
        x[:, 3::7] = -0.0
    elif kind == "peaked":
        x[:, rng.integers(0, vocab, rows)] += 12.0
    return x


@pytest.mark.parametrize("seed", [1, 77, 2**31 + 5])
def test_canonical_draws_match_mt19937(ref, seed):
    want = np.zeros(257)
    ref.ref_canonical_draws(ctypes.c_uint32(seed), 257, want.ctypes.data_as(ctypes.c_void_p))
    np.testing.assert_array_equal(osamp.canonical_draws(seed, 257), want)


CONFIGS = [(0.0, 0, 1.0), (1.0, 0, 1.0), (0.7, 0, 1.0), (1.0, 1, 1.0), (1.0, 5, 1.0), (1.3, 40, 1.0),
           (1.0, 0, 0.9), (1.0, 0, 0.5), (0.8, 0, 0.05), (1.0, 50, 0.8), (2.0, 3, 0.99), (1.0, 10**6, 0.7)]


@pytest.mark.parametrize("kind", ["normal", "ties", "peaked"])
@pytest.mark.parametrize("cfg", CONFIGS, ids=[f"T{t}-k{k}-p{p}" for t, k, p in CONFIGS])
def test_oracle_matches_reference_sampler(ref, cfg, kind):
    temp, k, p = cfg
    rng = np.random.default_rng(hash((cfg, kind)) % 2**32)
    for vocab, rows in ((1000, 40), (32000, 6)):
        logits = make_logits(rng, rows, vocab, kind)
        seed = int(rng.integers(0, 2**32))
        rc, want, err = ref_rows(ref, logits, temp, k, p, seed)
        assert rc == 0, err
        us = osamp.canonical_draws(seed, rows) if temp > 0 else np.zeros(rows)
        for r in range(rows):
            got, margin = osamp.sample(logits[r], temp, k, p, us[r])
            # a difference is allowed only where the draw sits on a boundary
            assert got == want[r] or margin < 1e-6, (r, got, want[r], margin)


def test_single_entry_vocabulary_draws_nothing(ref):
    # One logit: token 0 and no draw from the stream (discrete_distribution
    # with fewer than two weights).
    logits = np.array([[0.5], [1.5]], np.float32)
    rc, want, _ = ref_rows(ref, logits, 1.0, 0, 1.0, 9)
    assert rc == 0 and list(want) == [0, 0]
    assert osamp.sample(logits[0], 1.0, 0, 1.0, 0.3)[0] == 0


@pytest.mark.parametrize("bad,msg", [(np.nan, "Sampler: logits must all be finite"),
                                     (np.inf, "Sampler: logits must all be finite")])
def test_non_finite_logits_raise_like_reference(ref, bad, msg):
    logits = np.zeros((1, 16), np.float32)
    logits[0, 3] = bad
    for temp in (0.0, 1.0):
        rc, _, err = ref_rows(ref, logits, temp, 0, 1.0, 1)
        assert rc == 1 and err == msg
        with pytest.raises(ValueError, match=msg):
            osamp.sample(logits[0], temp, 0, 1.0, 0.5)


def test_scaled_overflow_raises_like_reference(ref):
    logits = np.full((1, 8), 3e38, np.float32)
    rc, _, err = ref_rows(ref, logits, 0.01, 0, 1.0, 1)
    assert rc == 1 and err == "Sampler: scaled logits are not finite"
    with pytest.raises(ValueError, match="scaled logits"):
        osamp.sample(logits[0], 0.01, 0, 1.0, 0.5)
