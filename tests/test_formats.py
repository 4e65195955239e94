"""The exchange-format module chromofold_amd.formats (CPU).

Pinned by the reference's committed files: tiny.cfwv / tiny.cfrr / tiny.cfrw / tiny.cffm parse to the same arrays
as the independent struct loaders of tests/cf_fixtures.py and write back byte for byte; .cfrw / .cffm also agree
with the C library's readers (cf_rrrw_file_read / cf_fm_file_read). The formats without a reference file
(.cfrs, .cffw, .cfkv, .cfdc, .cfsg) round-trip synthetic contents and reject malformed files; their layouts are the
exporter docstrings' (reference tools/export_*.py) and the GPU tests drive the kernels from such files.
"""
import os

import numpy as np
import pytest

import cf_fixtures as F
from chromofold_amd import formats as X
from chromofold_amd import search as S

FIX = {"tiny.cfwv": (F.load_cfwv, {"bitplanes": "words", "pos": "positions", "access_golden": "golden_tokens"}),
       "tiny.cfrr": (F.load_cfrr, {"pos": "positions", "rank_golden": "golden_rank1"}),
       "tiny.cfrw": (F.load_cfrw, {}), "tiny.cffm": (F.load_cffm, {})}


@pytest.mark.parametrize("name", sorted(FIX))
def test_reference_files_parse_and_write_back(tmp_path, name):
    loader, rename = FIX[name]
    kind, d = X.read(F._path(name))
    assert kind == name.split(".")[1]
    ref = loader()
    for k, v in ref.items():
        if isinstance(v, np.ndarray):
            assert np.array_equal(d[rename.get(k, k)], v), k
    out = str(tmp_path / name)
    X.write(out, kind, d)
    assert open(out, "rb").read() == open(F._path(name), "rb").read()


def test_index_files_agree_with_the_library_readers():
    _, rw = X.read(F._path("tiny.cfrw"))
    lib = S.read_cfrw(F._path("tiny.cfrw"))
    for k in ("classes", "offsets", "rank_a", "rank_d", "off_a", "off_d", "offbase", "zeros", "pos", "rank_golden"):
        assert np.array_equal(rw[k], lib[k]), k
    _, fm = X.read(F._path("tiny.cffm"))
    lib = S.read_cffm(F._path("tiny.cffm"))
    for k in ("C", "mwords", "msb", "sval", "pat", "locoff", "locpos", "count_golden"):
        assert np.array_equal(fm[k], lib[k]), k


def _synthetic(kind, rng):
    spec = X.SPECS[kind]
    small = {"cfrs": dict(n=700, block=64, V=9, M=4096, nblocks=11, data_bytes=333, slotlen=4096, h0=2.5,
                          rans_bits=2000, huff_bits=2100),
             "cffw": dict(M=5, K=70, B=3, bits=4, block=64, maxlen=8, zero=8, nwords=40, nblocks=6, lutlen=256,
                          scale=0.25, resident_bytes=999, dense_bytes=1400),
             "cfkv": dict(seq=30, dim=16, nq=7, window=8, bits=4, block=64, zero=8, kmaxlen=8, knwords=20,
                          knblocks=8, klutlen=256, vmaxlen=6, vnwords=18, vnblocks=8, vlutlen=64, softmax_scale=0.25,
                          resident_bytes=500, dense_bytes=3840),
             "cfdc": dict(N=4, nbase=50, ndelta=9, vocab=1000, total_tokens=230),
             "cfsg": dict(n=500, bits=3, vocab=8, emb_rows=8, dim=6, cwords=5, nsb=2, na=1, owords=9, npos=13,
                          rrr_bytes=77)}[kind]
    d = dict(small)
    for name, dt, cnt in spec.arrays:
        t = X._dtype(dt, small)
        n = int(cnt(small))
        d[name] = (rng.standard_normal(n).astype(t) if t.kind == "f" else
                   rng.integers(0, np.iinfo(t).max if t.itemsize < 4 else 1 << 30, n).astype(t))
    return d


@pytest.mark.parametrize("kind", ["cfrs", "cffw", "cfkv", "cfdc", "cfsg"])
def test_synthetic_round_trip_and_malformed(tmp_path, kind):
    rng = np.random.default_rng(len(kind))
    d = _synthetic(kind, rng)
    p = str(tmp_path / f"x.{kind}")
    X.write(p, kind, d)
    k2, back = X.read(p)
    assert k2 == kind
    for name, v in d.items():
        if isinstance(v, np.ndarray):
            assert np.array_equal(back[name], v), name
        else:
            assert back[name] == pytest.approx(v), name
    raw = open(p, "rb").read()
    for label, blob in {"trunc": raw[:-1], "extra": raw + b"\0", "magic": b"ZZZZ" + raw[4:],
                        "version": raw[:4] + (9).to_bytes(4, "little") + raw[8:], "short": raw[:6]}.items():
        q = tmp_path / f"{label}.{kind}"
        q.write_bytes(blob)
        with pytest.raises(ValueError):
            X.read(str(q))
    name0 = X.SPECS[kind].arrays[0][0]
    bad = dict(d)
    bad[name0] = np.asarray(d[name0])[:-1]
    with pytest.raises(ValueError, match="header implies"):
        X.write(str(tmp_path / "bad"), kind, bad)
