"""Token choice restated in numpy -- TEST INFRASTRUCTURE ONLY.

Follows src/generation/sampler.cpp:43-147 step by step, in the reference's
arithmetic: float32 values and weights, float32 sums accumulated in the
reference's loop order (np.add.accumulate is sequential), and the categorical
draw of libstdc++'s std::discrete_distribution (probabilities normalised by
their double sum, a double running sum with the last entry forced to 1, the
first index whose running sum is >= u).  The only intended difference is
np.exp against glibc's expf (both within an ulp of exp), so a choice can
differ only where u or top_p lies within rounding of a boundary; `sample`
reports how far from every boundary the choice was.
"""
from __future__ import annotations

import numpy as np


def argmax_first(values: np.ndarray) -> int:
    """First index of the maximum (the reference's strict > scan)."""
    return int(np.argmax(values))


def _seq_sum32(x: np.ndarray) -> np.float32:
    return np.add.accumulate(x.astype(np.float32), dtype=np.float32)[-1] if x.size else np.float32(0)


def sample(logits, temperature: float, top_k: int, top_p: float, u: float):
    """Returns (token, margin): margin is the smallest distance of u from the
    chosen bin's edges and of the top-p running mass from top_p (inf when a
    step does not apply).  Raises ValueError / RuntimeError like the reference."""
    values = np.asarray(logits, np.float32).copy()
    if not np.all(np.isfinite(values)):
        raise ValueError("Sampler: logits must all be finite")
    n = values.size
    if temperature == 0.0:
        return argmax_first(values), np.inf
    with np.errstate(over="ignore"):
        values = values / np.float32(temperature)
    if not np.all(np.isfinite(values)):
        raise ValueError("Sampler: scaled logits are not finite")
    idx = np.arange(n)
    order = np.lexsort((idx, -values.astype(np.float64)))  # value desc, index asc (-0 == +0)
    allowed = np.ones(n, bool)
    if 0 < top_k < n:
        allowed[order[top_k:]] = False
    margin = np.inf

    def weights_of(mask):
        m = values[mask].max()
        w = np.zeros(n, np.float32)
        w[mask] = np.exp((values[mask] - m).astype(np.float32)).astype(np.float32)
        return w

    w = weights_of(allowed)
    total = _seq_sum32(w[allowed])
    if not (total > 0) or not np.isfinite(total):
        raise RuntimeError("Sampler: invalid softmax distribution")
    if top_p < 1.0:
        cand = idx[allowed]
        porder = cand[np.lexsort((cand, -w[cand].astype(np.float64)))]
        q = (w[porder] / total).astype(np.float32)
        cum = np.add.accumulate(q, dtype=np.float32)
        before = np.concatenate([[np.float32(0)], cum[:-1]])
        keep = before < np.float32(top_p)
        allowed[porder[~keep]] = False
        margin = float(np.min(np.abs(cum.astype(np.float64) - top_p)))
        if not allowed.any():
            allowed[order[0]] = True
    w = weights_of(allowed)
    total = _seq_sum32(w[allowed])
    if not (total > 0) or not np.isfinite(total):
        raise RuntimeError("Sampler: invalid filtered distribution")
    p = (w / total).astype(np.float32).astype(np.float64)
    if n < 2:
        return 0, margin
    s = np.add.accumulate(p)[-1]
    cp = np.add.accumulate(p / s)
    cp[-1] = 1.0
    tok = int(np.searchsorted(cp, u, side="left"))
    lo = cp[tok - 1] if tok > 0 else 0.0
    margin = min(margin, abs(cp[tok] - u), abs(u - lo))
    return tok, margin


def canonical_draws(seed: int, n: int) -> np.ndarray:
    """The uniforms std::discrete_distribution takes from std::mt19937(seed):
    generate_canonical<double, 53> from two 32-bit outputs, low word first.
    numpy's legacy RandomState(seed) is the same MT19937 with the same
    init_genrand seeding, and randint over [0, 2^32) returns its raw words."""
    if n == 0:
        return np.zeros(0)
    words = np.random.RandomState(seed).randint(0, 2**32, size=2 * n, dtype=np.uint64).astype(np.float64)
    u = (words[0::2] + words[1::2] * 2.0**32) / 2.0**64
    return np.where(u >= 1.0, np.nextafter(1.0, 0.0), u)
