"""Pins the CPU oracle's succinct structures against the reference's committed fixtures and closed forms.

Fixtures (tests/golden/fixtures/, copied data from the reference's packaging/fixtures/):
  tiny.cfrw  RRR wavelet of a BWT (n=4097, 7 levels) + 64 access / 64 rank goldens
  tiny.cffm  FM-index (n=8193, sigma 65, sample 16) + 528 count goldens and their located positions
  tiny.cfwv  packed wavelet (n=4096, 8 levels) + raw tokens + 64 access / 64 rank goldens
  tiny.cfrr  single RRR bitvector (n=8192) + 64 rank1 goldens
"""
import numpy as np
import pytest

import cf_fixtures as F
import oracle as O


def _rrrw_from(d):
    return O.RrrwArrays(d["bits"], d["cwords"], d["nsb"], d["na"], d["classes"], d["offsets"], d["rank_a"],
                        d["rank_d"], d["off_a"], d["off_d"], d["offbase"], d["zeros"])


RRRW_FIELDS = ["classes", "offsets", "rank_a", "rank_d", "off_a", "off_d", "offbase", "zeros"]


def test_rrr_tables_closed_form():
    from math import comb, ceil, log2
    binom, width = O.rrr_tables()
    for n in range(16):
        for k in range(16):
            assert binom[n * 16 + k] == (comb(n, k) if k <= n else 0)
    for k in range(16):
        c = comb(15, k)
        assert width[k] == (ceil(log2(c)) if c > 1 else 0)


def test_cfrw_goldens():
    d = F.load_cfrw()
    w = _rrrw_from(d)
    assert np.array_equal(O.rrrw_access(w, d["pos"]), d["access_golden"])
    assert np.array_equal(O.rrrw_rank(w, d["rank_c"], d["rank_i"]), d["rank_golden"])


def test_cfrw_layout_roundtrip():
    """Decode every position, rebuild with the oracle builder: all arrays byte-identical to the fixture."""
    d = F.load_cfrw()
    w = _rrrw_from(d)
    seq = O.rrrw_access(w, np.arange(d["n"], dtype=np.uint32))
    w2 = O.rrrw_build(seq, d["bits"])
    for f in RRRW_FIELDS:
        assert np.array_equal(getattr(w2, f), d[f]), f
    assert (w2.cwords, w2.nsb, w2.na, w2.offsets.size) == (d["cwords"], d["nsb"], d["na"], d["owords"])
    assert w2.rrr_bytes == d["rrr_bytes"]
    # closed forms over the recovered sequence: rank(c, i) == count of c in seq[:i]
    rng = np.random.default_rng(5)
    c = rng.integers(0, 1 << d["bits"], 300).astype(np.uint32)
    i = rng.integers(0, d["n"] + 1, 300).astype(np.uint32)
    exp = np.array([(seq[:ii] == cc).sum() for cc, ii in zip(c, i)], np.uint32)
    assert np.array_equal(O.rrrw_rank(w, c, i), exp)


def test_rrrw_closed_form_zipf():
    rng = np.random.default_rng(11)
    for n, bits in [(1, 1), (15, 3), (16, 4), (961, 5), (3000, 9), (20000, 15)]:
        tok = rng.integers(0, 1 << bits, n).astype(np.uint32)
        w = O.rrrw_build(tok, bits)
        assert np.array_equal(O.rrrw_access(w, np.arange(n, dtype=np.uint32)), tok)
        c = rng.integers(0, 1 << bits, 200).astype(np.uint32)
        i = rng.integers(0, n + 1, 200).astype(np.uint32)
        exp = np.array([(tok[:ii] == cc).sum() for cc, ii in zip(c, i)], np.uint32)
        assert np.array_equal(O.rrrw_rank(w, c, i), exp)


def _invert_bwt(bwt: np.ndarray) -> np.ndarray:
    """Text s (ending in sentinel 0) from its BWT: LF(i) is i's slot in the stable sort of the BWT, and walking
    LF from row 0 (the sentinel suffix) yields the text right to left."""
    n = bwt.size
    lf = np.empty(n, np.int64)
    lf[np.argsort(bwt, kind="stable")] = np.arange(n)
    s = np.empty(n, np.int64)
    s[n - 1] = 0
    p = 0
    for k in range(n - 2, -1, -1):
        s[k] = bwt[p]
        p = lf[p]
    return s


def test_cffm_goldens_and_rebuild():
    d = F.load_cffm()
    w = _rrrw_from(d)
    f = O.FmArrays(w, d["C"], d["mwords"], d["msb"], d["sval"], d["sigma"], d["n"], d["sa_sample"])
    cnt = O.fm_count(f, d["pat"], d["pstart"], d["plen"])
    assert np.array_equal(cnt, d["count_golden"])
    lo, hi = O.fm_ranges(f, d["pat"], d["pstart"], d["plen"])
    assert np.array_equal((hi - lo).astype(np.uint32), d["count_golden"])
    rows = np.concatenate([np.arange(a, b, dtype=np.int32) for a, b in zip(lo, hi)])
    pos = O.fm_locate(f, rows)
    at = 0
    for t in range(d["pstart"].size):
        k = int(hi[t] - lo[t])
        got = np.sort(pos[at:at + k])
        at += k
        assert np.array_equal(got, d["locpos"][d["locoff"][t]:d["locoff"][t + 1]]), t
    # rebuild the whole index from the text recovered out of the fixture's own BWT
    bwt = O.rrrw_access(w, np.arange(d["n"], dtype=np.uint32)).astype(np.int64)
    s = _invert_bwt(bwt)
    assert s[-1] == 0 and (s[:-1] >= 1).all()
    tokens = (s[:-1] - 1).astype(np.uint32)
    f2, bwt2 = O.fm_build(tokens, d["sa_sample"])
    assert np.array_equal(bwt2, bwt)
    for k in ["C", "mwords", "msb", "sval"]:
        assert np.array_equal(getattr(f2, k), d[k]), k
    for k in RRRW_FIELDS:
        assert np.array_equal(getattr(f2.w, k), d[k]), k
    # ground truth: counts == naive substring search over the recovered text
    for t in range(0, d["pstart"].size, 7):
        p = d["pat"][d["pstart"][t]:d["pstart"][t] + d["plen"][t]] - 1
        assert O.naive_count(tokens.astype(np.int32), p) == d["count_golden"][t]


def test_suffix_array_methods_agree_and_brute_force():
    rng = np.random.default_rng(3)
    for n, v in [(1, 1), (2, 2), (7, 2), (50, 3), (500, 5), (4000, 40)]:
        tok = rng.integers(0, v, n)
        s = O.fm_text(tok)
        a = O.suffix_array(s, "doubling")
        b = O.suffix_array(s, "radix")
        assert np.array_equal(a, b)
        if s.size <= 600:
            brute = sorted(range(s.size), key=lambda i: list(s[i:]))
            assert list(a) == brute


def test_cfwv_goldens_and_rebuild():
    d = F.load_cfwv()
    lv, nw, nb = d["levels"], d["nwords"], d["nblocks"]
    acc = O.packed_access(d["bitplanes"], d["superblocks"], d["zeros"], lv, nw, nb, d["pos"])
    assert np.array_equal(acc, d["access_golden"])
    assert np.array_equal(acc, d["tokens"][d["pos"]])
    rk = O.packed_rank(d["bitplanes"], d["superblocks"], d["zeros"], lv, nw, nb, d["rank_c"], d["rank_i"])
    assert np.array_equal(rk, d["rank_golden"])
    bp, sb, z, nw2, nb2 = O.packed_build(d["tokens"], lv)
    assert (nw2, nb2) == (nw, nb)
    assert np.array_equal(bp, d["bitplanes"]) and np.array_equal(sb, d["superblocks"])
    assert np.array_equal(z, d["zeros"])


def test_cfrr_goldens_and_rebuild():
    d = F.load_cfrr()
    got = O.rrr_rank1(d["classes"], d["offsets"], d["sbrank"], d["sboff"], d["pos"])
    assert np.array_equal(got, d["rank_golden"])
    bits = O.rrr_decode_all(d["classes"], d["offsets"], d["nblocks"])[:d["n"]]
    prefix = np.concatenate([[0], np.cumsum(bits, dtype=np.int64)])
    assert np.array_equal(prefix[d["pos"]].astype(np.uint32), d["rank_golden"])
    e = O.rrr_plane_build(bits)
    for k in ["classes", "offsets", "sbrank", "sboff"]:
        assert np.array_equal(e[k], d[k]), k
    assert (e["class_bits"], e["offset_bits"]) == (d["class_bits"], d["offset_bits"])
