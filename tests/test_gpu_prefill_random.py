"""Seeded random chunked-prefill cases against the oracle: geometry, query
dtype, table layout, batch and, per sequence, a chunk of 1 to a few hundred
tokens at the end of a context of up to ~1,500 tokens, drawn per seed.  The
chunks meet tile edges (256 query rows per workgroup, so 256 / G tokens) and
the 64-key steps at every offset; the poisoned slots past each context
(NaN) must never reach an output.

Tolerance: |gpu - ref| <= 2e-3 + 1e-2 * |ref| (the prefill tests' bound).
"""
import numpy as np
import pytest

from test_gpu_prefill import _case, _gpu, _ref
from kvcase import assert_close

pytestmark = pytest.mark.gpu

GEOMS = [(32, 4, 64), (32, 8, 128), (64, 8, 128), (8, 8, 64), (16, 1, 128), (8, 4, 128), (16, 8, 64)]


@pytest.mark.parametrize("seed", range(32))
def test_random_prefill_case(gpu, seed):
    rng = np.random.default_rng(5000 + seed)
    Hq, Hkv, hd = GEOMS[rng.integers(0, len(GEOMS))]
    B = int(rng.integers(1, 6))
    chunk = rng.choice([1, 2, 15, 16, 17, 31, 32, 33, 63, 64, 65, 127, 128, 129, 255, 256, 300], B)
    ctx = chunk + rng.choice([0, 1, 15, 16, 17, 63, 64, 200, 1200], B)
    q_dtype = "fp32" if rng.random() < 0.3 else "bf16"
    layout = ["random", "sequential", "round_robin"][rng.integers(0, 3)]
    c = _case(Hq, Hkv, hd, 16, ctx, chunk, q_dtype, seed=seed, layout=layout)
    what = f"seed={seed} geom=({Hq},{Hkv},{hd}) q={q_dtype} {layout} chunks {list(chunk)} contexts {list(ctx)}"
    assert_close(_gpu(gpu, c), _ref(c), what=what)
