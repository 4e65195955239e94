"""Seeded synthetic inputs for the benchmark configurations (shared by bench.py and the tests).

All generators are deterministic in their seed (numpy PCG64). Token streams are Zipf(s) over ranks 1..vocab by
inverse-CDF sampling, token = rank - 1 (so token 0 is the most frequent).
"""
from __future__ import annotations

import numpy as np

SEED_C1, SEED_C2, SEED_C3, SEED_C4, SEED_C5 = 0xC1, 0xC2, 0xC3, 0xC4, 0xC5


def zipf_tokens(n: int, vocab: int = 32000, s: float = 1.1, seed: int = SEED_C1) -> np.ndarray:
    rng = np.random.default_rng(seed)
    w = np.arange(1, vocab + 1, dtype=np.float64) ** (-s)
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    u = rng.random(n)
    return np.minimum(np.searchsorted(cdf, u, side="right"), vocab - 1).astype(np.uint32)


def rrr_queries(tokens: np.ndarray, nq: int, vocab: int, seed: int):
    """access positions uniform in [0, n); rank (c, i): c half from the token stream, half uniform over the
    vocabulary; i uniform in [0, n]."""
    rng = np.random.default_rng(seed)
    n = tokens.size
    pos = rng.integers(0, n, nq, dtype=np.int64).astype(np.uint32)
    half = nq // 2
    c = np.empty(nq, np.uint32)
    c[:half] = tokens[rng.integers(0, n, half)]
    c[half:] = rng.integers(0, vocab, nq - half).astype(np.uint32)
    i = rng.integers(0, n + 1, nq, dtype=np.int64).astype(np.uint32)
    return pos, c, i
