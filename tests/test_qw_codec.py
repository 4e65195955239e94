"""CPU checks of the cf_qw_matrix host encoder (libchromofold's C++ side, no GPU):

  * cf_qw_quantize_int4 equals its closed form (per (row, 64-column segment) absmax / 7, round half to even,
    clamp to [-8, 7], symbol = q + 8; all-zero segments get scale 1);
  * cf_qw_huffman_plan gives per-band code lengths that form a prefix code (Kraft sum <= 1, lengths <= 12) and
    cover every symbol the band uses;
  * cf_qw_huffman_encode round trips: every (row, segment) decoded from its own bit offset by the oracle's LUT
    decoder (with the canonical codes rebuilt from the lengths) gives back the symbols.
"""
import numpy as np
import pytest

import oracle as O
from legacy_helpers import canonical_codes


def _lut(lengths, maxlen=12):
    lut = np.zeros(1 << maxlen, np.int32)
    for s, (c, l) in canonical_codes(lengths).items():
        base = c << (maxlen - l)
        lut[base:base + (1 << (maxlen - l))] = s | (l << 8)
    return lut


@pytest.mark.parametrize("rows,cols,seed", [(40, 1000, 1), (16, 64, 2), (33, 4100, 3), (1, 1, 4)])
def test_quantize_and_roundtrip(rows, cols, seed):
    from chromofold_amd import qw
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((rows, cols)) / np.sqrt(cols)).astype(np.float32)
    if rows > 2:
        w[1, :] = 0.0          # all-zero row: scale 1, symbol 8
        w[2, ::7] *= 50.0      # outliers
    h = qw.encode_int4(w)
    nseg = (cols + 63) // 64
    pad = np.zeros((rows, nseg * 64), np.float32)
    pad[:, :cols] = w
    amax = np.abs(pad.reshape(rows, nseg, 64)).max(2)
    sc = np.where(amax > 0, amax / np.float32(7.0), 1.0).astype(np.float32)
    assert np.array_equal(h.scales, sc)
    q = np.clip(np.rint(w / np.repeat(sc, 64, 1)[:, :cols]), -8, 7) + 8
    assert np.array_equal(h.sym, q.astype(np.uint8))
    for b in range((rows + 15) // 16):
        L = h.code_lengths[16 * b:16 * b + 16].astype(int)
        used = np.unique(h.sym[16 * b:16 * b + 16])
        assert (L[used] > 0).all() and L.max() <= 12
        assert sum(2.0 ** -x for x in L if x) <= 1.0
    for r in range(rows):
        lut = _lut(h.code_lengths[16 * (r // 16):16 * (r // 16) + 16].astype(int))
        for s in range(nseg):
            n = min(64, cols - 64 * s)
            got = O.huffman_decode(h.words, lut, 12, int(h.seg_offsets[r, s]), n)
            assert np.array_equal(got, h.sym[r, 64 * s:64 * s + n]), (r, s)


def test_skewed_band_is_length_limited():
    """A band whose symbol counts are Fibonacci-like would need codes longer than 12 bits without the limit."""
    from chromofold_amd import qw
    fib = [1, 1]
    while len(fib) < 16:
        fib.append(fib[-1] + fib[-2])
    sym = np.repeat(np.arange(16, dtype=np.uint8), fib)[None, :]
    h = qw.encode_symbols(sym, np.ones((1, (sym.shape[1] + 63) // 64), np.float32))
    L = h.code_lengths[:16].astype(int)
    assert L.max() == 12 and sum(2.0 ** -x for x in L) <= 1.0
    lut = _lut(L)
    for s in range(h.seg_offsets.shape[1]):
        n = min(64, sym.shape[1] - 64 * s)
        assert np.array_equal(O.huffman_decode(h.words, lut, 12, int(h.seg_offsets[0, s]), n), sym[0, 64 * s:64 * s + n])


def test_validate_rules_host_only():
    """cf_qw_validate checks the descriptor on the host (no device access, so it runs without a GPU): version and
    size, codec, shape, NULL arrays, zero point, and a 16-byte aligned code-length table (the kernel reads a band's
    16 lengths with one 16-byte load)."""
    import ctypes as C
    from chromofold_amd import _abi as A
    from chromofold_amd import qw
    L = A.lib()
    base = 1 << 20  # fake aligned device addresses: never dereferenced

    def desc(**kw):
        f = dict(struct_size=C.sizeof(qw.cf_qw_matrix), abi_version=qw.QW_ABI_VERSION, codec=qw.QW_CODEC_HUFFMAN,
                 rows=64, cols=4096, zero=8, word_count=100, words=base, seg_offsets=base, code_lengths=base,
                 scales=base)
        f.update(kw)
        return qw.cf_qw_matrix(**f)

    ok = A.CF_OK
    bad = A.CF_ERR_INVALID_ARGUMENT
    assert L.cf_qw_validate(C.byref(desc())) == ok
    assert L.cf_qw_validate(C.byref(desc(code_lengths=base + 8))) == bad
    assert L.cf_qw_validate(C.byref(desc(code_lengths=base + 16))) == ok
    assert L.cf_qw_validate(C.byref(desc(abi_version=99))) == bad
    assert L.cf_qw_validate(C.byref(desc(codec=5))) == A.CF_ERR_UNSUPPORTED
    assert L.cf_qw_validate(C.byref(desc(rows=0))) == bad
    assert L.cf_qw_validate(C.byref(desc(scales=None))) == bad
    assert L.cf_qw_validate(C.byref(desc(zero=16))) == bad
    assert L.cf_qw_validate(C.byref(desc(word_count=0))) == bad
