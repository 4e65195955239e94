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


def fm_patterns(tokens: np.ndarray, n_cut: int, n_rand: int, vocab: int, seed: int, lmin: int = 8, lmax: int = 32):
    """Patterns for the FM workload, in text symbols (token + 1): n_cut windows of length U[lmin, lmax] cut at
    uniform text offsets, then n_rand patterns of uniform random tokens (almost never occurring). Returns the
    flattened symbols, start offsets and lengths (int32)."""
    rng = np.random.default_rng(seed)
    n = tokens.size
    lens = rng.integers(lmin, lmax + 1, n_cut + n_rand).astype(np.int32)
    starts = np.zeros(lens.size, np.int64)
    starts[1:] = np.cumsum(lens[:-1])
    flat = np.empty(int(lens.sum()), np.int32)
    offs = rng.integers(0, n - lmax, n_cut)
    idx = starts[:n_cut, None] + np.arange(lmax)[None, :]
    src = offs[:, None] + np.arange(lmax)[None, :]
    mask = np.arange(lmax)[None, :] < lens[:n_cut, None]
    flat[idx[mask]] = tokens[src[mask]].astype(np.int32) + 1
    r0 = int(starts[n_cut]) if n_rand else flat.size
    flat[r0:] = rng.integers(0, vocab, flat.size - r0).astype(np.int32) + 1
    return flat, starts.astype(np.int32), lens
