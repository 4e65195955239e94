"""Pins the oracle's entropy decoders (CPU, no GPU):

  * or_rans_block_decode (restates reference src/cuda/rans.cu:11-26) inverts an independent encoder written from
    the rANS construction (tests/legacy_helpers.rans_encode_blocks), including the special cases the reference's
    decoder must handle: a single-symbol distribution (freq = 4096, zero information per symbol), a last partial
    block, block size 1;
  * or_huffman_decode (restates include/chromofold/detail/block_huffman_device.cuh:12-19) decodes the vectorised
    packer bit for bit like the per-symbol packer, from any block offset;
  * a planted mistake is caught: flipping one byte of a rANS stream or one bit of a Huffman stream changes the
    decoded symbols.
"""
import numpy as np
import pytest

import oracle as O
from legacy_helpers import canonical_codes, huffman_lengths, huffman_stream, huffman_stream_np, rans_encode_blocks


def _freq12(counts):
    f = np.maximum(1, (counts * 4096 // max(counts.sum(), 1))).astype(np.int64)
    f[counts == 0] = 0
    f[np.argmax(f)] += 4096 - f.sum()
    return f


@pytest.mark.parametrize("n,V,block,seed", [(5000, 16, 64, 1), (4099, 256, 1024, 2), (777, 5, 1, 3),
                                            (20000, 3, 333, 4)])
def test_rans_roundtrip(n, V, block, seed):
    rng = np.random.default_rng(seed)
    p = rng.dirichlet(np.ones(V) * 0.5)
    sym = rng.choice(V, size=n, p=p)
    f = _freq12(np.bincount(sym, minlength=V))
    enc = rans_encode_blocks(sym, f, block)
    assert np.array_equal(O.rans_block_decode(*enc, block, n), sym)
    if block >= 64:  # (a 1-symbol block reads its bytes only after its one symbol is decoded)
        data = enc[0].copy()
        data[len(data) // 3] ^= 0x5A
        assert not np.array_equal(O.rans_block_decode(data, *enc[1:], block, n), sym)


def test_rans_single_symbol_distribution():
    sym = np.full(300, 7)
    f = np.zeros(16, np.int64)
    f[7] = 4096
    enc = rans_encode_blocks(sym, f, 64)
    assert enc[0][:-8].size == 0  # no information: no renormalisation bytes
    assert np.array_equal(O.rans_block_decode(*enc, 64, sym.size), sym)


@pytest.mark.parametrize("maxlen", [4, 9, 12])
def test_huffman_packers_agree_and_decode(maxlen):
    rng = np.random.default_rng(maxlen)
    sym = np.minimum(rng.geometric(0.3, 6000) - 1, 15)
    freq = np.bincount(sym, minlength=16)
    L = huffman_lengths(freq, maxlen)
    assert L.max() <= maxlen and sum(2.0 ** -int(x) for x in L if x) <= 1.0
    w1, b1, l1 = huffman_stream(sym, canonical_codes(L), maxlen, 64)
    w2, b2, l2 = huffman_stream_np(sym, L, maxlen, 64)
    n = min(w1.size, w2.size)
    assert np.array_equal(w1[:n], w2[:n]) and np.array_equal(b1, b2) and np.array_equal(l1, l2)
    for blk in (0, 5, len(b2) - 1):
        s0 = blk * 64
        assert np.array_equal(O.huffman_decode(w2, l2, maxlen, int(b2[blk]), sym.size - s0), sym[s0:])
    w3 = w2.copy()
    w3[3] ^= 1 << 17
    assert not np.array_equal(O.huffman_decode(w3, l2, maxlen, 0, sym.size), sym)


def test_dense_and_window_attention_reduce_to_paged():
    """or_dense_attention_f64 (and the windowed attention built on it) equals the reference-pinned paged oracle:
    one page holding all rows, query at the last token, causal window w <-> the last w rows."""
    rng = np.random.default_rng(12)
    T, D = 40, 32
    K = rng.standard_normal((T, D)).astype(np.float32)
    V = rng.standard_normal((T, D)).astype(np.float32)
    Q = rng.standard_normal((T, D)).astype(np.float32)
    for i, w in ((T - 1, 1000), (T - 1, 7), (10, 3), (0, 5)):
        paged, empty = O.paged_attention_f64(Q[i][None], 1, 1, D, 1, i, w if w < 1000 else 0, 0.3, [(0, 0, K, V)])
        assert empty == 0
        lo = max(0, i - w + 1)
        dense = O.dense_attention_f64(Q[i], K[lo:i + 1], V[lo:i + 1], 0.3)
        np.testing.assert_allclose(dense, paged[0], rtol=1e-6, atol=1e-7)
        win = O.kv_window_attention_f64(K, V, Q, i + 1, min(w, 512), 0.3)[i]
        np.testing.assert_allclose(win, paged[0], rtol=1e-6, atol=1e-7)


def test_qmatmul_oracle_special_cases():
    """y = x (q - zero)^T scale: a one-hot weight row selects one activation column; zero symbols give zero; a
    per-element scale array multiplies elementwise (a transposed operand or a dropped zero point fails these)."""
    rng = np.random.default_rng(3)
    B, M, K = 3, 5, 7
    x = rng.standard_normal((B, K))
    sym = np.full((M, K), 8)
    cols = rng.integers(0, K, M)
    sym[np.arange(M), cols] = 9  # (q - 8) = one-hot
    y = O.qmatmul_f64(x, sym, 2.0, 8)
    np.testing.assert_array_equal(y, 2.0 * x[:, cols])
    sc = rng.random((M, K)) + 0.5
    y2 = O.qmatmul_f64(x, sym, sc, 8)
    np.testing.assert_allclose(y2, x[:, cols] * sc[np.arange(M), cols][None, :])
