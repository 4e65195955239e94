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
        L = h.tables[16 * b:16 * b + 16].astype(int)
        used = np.unique(h.sym[16 * b:16 * b + 16])
        assert (L[used] > 0).all() and L.max() <= 12
        assert sum(2.0 ** -x for x in L if x) <= 1.0
    for r in range(rows):
        lut = _lut(h.tables[16 * (r // 16):16 * (r // 16) + 16].astype(int))
        for s in range(nseg):
            n = min(64, cols - 64 * s)
            got = O.huffman_decode(h.words, lut, 12, int(h.offsets[r, s]), n)
            assert np.array_equal(got, h.sym[r, 64 * s:64 * s + n]), (r, s)


def test_skewed_band_is_length_limited():
    """A band whose symbol counts are Fibonacci-like would need codes longer than 12 bits without the limit."""
    from chromofold_amd import qw
    fib = [1, 1]
    while len(fib) < 16:
        fib.append(fib[-1] + fib[-2])
    sym = np.repeat(np.arange(16, dtype=np.uint8), fib)[None, :]
    h = qw.encode_symbols(sym, np.ones((1, (sym.shape[1] + 63) // 64), np.float32))
    L = h.tables[:16].astype(int)
    assert L.max() == 12 and sum(2.0 ** -x for x in L) <= 1.0
    lut = _lut(L)
    for s in range(h.offsets.shape[1]):
        n = min(64, sym.shape[1] - 64 * s)
        assert np.array_equal(O.huffman_decode(h.words, lut, 12, int(h.offsets[0, s]), n), sym[0, 64 * s:64 * s + n])


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
                 rows=64, cols=4096, zero=8, word_count=100, words=base, offsets=base, tables=base,
                 scales=base)
        f.update(kw)
        return qw.cf_qw_matrix(**f)

    ok = A.CF_OK
    bad = A.CF_ERR_INVALID_ARGUMENT
    assert L.cf_qw_validate(C.byref(desc())) == ok
    assert L.cf_qw_validate(C.byref(desc(tables=base + 8))) == bad
    assert L.cf_qw_validate(C.byref(desc(tables=base + 16))) == ok
    assert L.cf_qw_validate(C.byref(desc(abi_version=99))) == bad
    assert L.cf_qw_validate(C.byref(desc(codec=5))) == A.CF_ERR_UNSUPPORTED
    assert L.cf_qw_validate(C.byref(desc(rows=0))) == bad
    assert L.cf_qw_validate(C.byref(desc(scales=None))) == bad
    assert L.cf_qw_validate(C.byref(desc(zero=16))) == bad
    assert L.cf_qw_validate(C.byref(desc(word_count=0))) == bad
    # rANS descriptors: lane states and a 16-byte aligned word array, slot sizes in multiples of 8 (chunk_words may
    # be 0 only with a single chunk per band), and enough words for every band's slots
    rans = dict(codec=qw.QW_CODEC_RANS, states=base, chunk_words=0, last_words=8000, word_count=64 * 4000)
    assert L.cf_qw_validate(C.byref(desc(**rans))) == ok
    assert L.cf_qw_validate(C.byref(desc(**{**rans, "states": None}))) == bad
    assert L.cf_qw_validate(C.byref(desc(**{**rans, "last_words": 0}))) == bad
    assert L.cf_qw_validate(C.byref(desc(**{**rans, "last_words": 8004}))) == bad
    assert L.cf_qw_validate(C.byref(desc(**{**rans, "last_words": 32776}))) == bad
    assert L.cf_qw_validate(C.byref(desc(**{**rans, "word_count": 4 * 4000 - 1}))) == bad
    assert L.cf_qw_validate(C.byref(desc(**{**rans, "words": base + 8}))) == bad
    assert L.cf_qw_validate(C.byref(desc(**{**rans, "cols": 8192}))) == bad  # two chunks need chunk_words
    assert L.cf_qw_validate(C.byref(desc(**{**rans, "cols": 8192, "chunk_words": 8000, "word_count": 4 * 16000})))\
        == ok


# ------------------------------------------------------------------------------------------------ rANS pairs
def _rans(W):
    from chromofold_amd import qw
    return qw.encode_int4(W, qw.QW_CODEC_RANS)


def _freqs(h):
    """[bands, 256] pair frequencies from the descriptor's cumulative starts."""
    cum = h.tables.reshape(-1, 256).astype(np.int64)
    return np.diff(np.concatenate([cum, np.full((cum.shape[0], 1), 4096)], 1), axis=1)


def _rans_decode(h, mistake=0):
    return O.qw_rans_decode(h.words, h.chunk_words, h.last_words, h.offsets, h.states, h.tables, h.rows, h.cols,
                            mistake)


@pytest.mark.parametrize("rows,cols,seed", [(40, 1000, 1), (16, 256, 2), (33, 4100, 3), (1, 1, 4), (20, 8492, 5),
                                            (17, 12288, 6)])
def test_rans_roundtrip(rows, cols, seed):
    """The library's rANS encoder and the oracle's decoder invert each other on ragged shapes (rows past the last
    band, columns past the last stripe, a short last chunk, three full chunks), an all-zero row and outliers; every
    stripe ends with its lanes back at 2^16 and its cursor at the next stripe's first word."""
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((rows, cols)) / np.sqrt(cols)).astype(np.float32)
    if rows > 2:
        w[1, :] = 0.0
        w[2, ::7] *= 50.0
    h = _rans(w)
    sym, bad = _rans_decode(h)
    assert bad == 0 and np.array_equal(sym, h.sym)


def test_rans_planted_mistakes_fail_the_roundtrip():
    """Each planted decoder mistake breaks the round trip: words taken in reverse lane order, the lane-group and
    MFMA-block roles of the column map swapped, the state update off by one."""
    rng = np.random.default_rng(11)
    h = _rans(rng.standard_normal((48, 4096)).astype(np.float32))
    for mistake in (1, 2, 3):
        sym, bad = _rans_decode(h, mistake)
        assert not np.array_equal(sym, h.sym), mistake


def test_rans_tables_and_closed_forms():
    """Tables: cumulative starts from 0, frequencies summing to 4096, a pair the band holds has f >= 1 and an absent
    pair f = 0. Closed form:
    a band holding one pair only (an all-zero band: (zero, zero) everywhere) gets f = 4096 for it, its encoder
    never renormalises (f * (x >> 12) + (x & 4095) = x when f = 4096), so its lanes keep the initial 2^16 and it
    emits no word; the oracle still decodes it."""
    rng = np.random.default_rng(12)
    W = rng.standard_normal((48, 4096)).astype(np.float32)
    W[16:32] = 0.0
    h = _rans(W)
    F = _freqs(h)
    assert (F.sum(1) == 4096).all() and (h.tables.reshape(-1, 256)[:, 0] == 0).all()
    for b in range(3):
        s = h.sym[16 * b:16 * b + 16]
        pairs = np.unique(s[:, 0::2].astype(np.int64) | (s[:, 1::2].astype(np.int64) << 4))
        assert (F[b, pairs] >= 1).all() and F[b].astype(bool).sum() == pairs.size
    assert F[1, 8 | (8 << 4)] == 4096
    st = h.states.reshape(3, 16, 64)
    assert (st[1] == 65536).all()
    ns = 16
    assert (h.offsets.reshape(3, ns)[1] == 0).all()
    sym, bad = _rans_decode(h)
    assert bad == 0 and np.array_equal(sym, h.sym)


def test_rans_stream_length_matches_the_table_cost():
    """rANS codes within a rounding of the ideal length under its own table: a stripe's emitted words plus the
    information its final states hold (log2(x / 2^16) per lane) equal sum -log2(f_s / 4096) over the stripe's pairs
    to within 0.2 % — a broken renormalisation or a wrong cumulative start would shift it (checked on every stripe
    but a band's last, whose length the offsets give). The table itself costs less than 0.01 bits per pair over the
    band's empirical pair entropy."""
    rng = np.random.default_rng(13)
    rows, cols = 32, 4096
    h = _rans(rng.standard_normal((rows, cols)).astype(np.float32))
    F = _freqs(h).astype(np.float64)
    ns = cols // 256
    offs = h.offsets.reshape(-1, ns).astype(np.int64)
    states = h.states.reshape(-1, ns, 64).astype(np.float64)
    ideal = emitted = 0.0
    for b in range(rows // 16):
        s = h.sym[16 * b:16 * b + 16]
        pairs = s[:, 0::2].astype(np.int64) | (s[:, 1::2].astype(np.int64) << 4)
        cnt = np.bincount(pairs.ravel(), minlength=256).astype(np.float64)
        cost = -(cnt[cnt > 0] * np.log2(F[b][cnt > 0] / 4096)).sum()
        h0 = -(cnt[cnt > 0] * np.log2(cnt[cnt > 0] / cnt.sum())).sum()
        assert cost - h0 < 0.01 * cnt.sum()
        known = pairs[:, :(ns - 1) * 128]  # stripes 0 .. ns - 2 (128 pairs of each row per stripe)
        ideal += -np.log2(F[b][known.ravel()] / 4096).sum()
        emitted += 16 * (offs[b, ns - 1] - offs[b, 0]) + np.log2(states[b, :ns - 1] / 65536).sum()
    assert abs(emitted - ideal) < 0.002 * ideal, (emitted, ideal)
