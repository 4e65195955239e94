"""On-disk .cfrw v1 / .cffm v1 readers and writers of the library (cf_rrrw_file_* / cf_fm_file_*), CPU only.

Pinned three ways:
- against the committed fixtures written by the reference builder (tests/golden/fixtures/tiny.cfrw, tiny.cffm),
  parsed by the independent struct-based loaders in tests/cf_fixtures.py;
- by write-back: reading a fixture and writing it again must reproduce the file byte for byte;
- against the reference tool itself (oracle/_ref/build_index, reference tools/build_index.cpp:413-438, 496-526)
  on fresh seeds, when that tool is built: its files read back and re-written byte-identically, and the oracle's
  own RRR/FM arrays written through the library equal the tool's file.
"""
import subprocess

import numpy as np
import pytest

import cf_fixtures as F
from chromofold_amd import _abi as A
from chromofold_amd import search as S
import oracle as O

WAVELET = ("classes", "offsets", "rank_a", "rank_d", "off_a", "off_d", "offbase", "zeros")
RRRW_Q = ("pos", "access_golden", "rank_c", "rank_i", "rank_golden")
FM = ("C", "mwords", "msb", "sval", "pat", "pstart", "plen", "count_golden", "locoff", "locpos")


def _same(d, ref, keys):
    for k in keys:
        assert np.array_equal(np.asarray(d[k]), np.asarray(ref[k])), k


def test_ctypes_mirrors_match_c_struct_sizes():
    import ctypes as C
    assert C.sizeof(S.cf_rrrw_file_header) == 64
    assert C.sizeof(S.cf_fm_file_header) == 80
    assert C.sizeof(S.cf_rrrw_file_queries) == 5 * 8
    assert C.sizeof(S.cf_fm_file_arrays) == 10 * 8


def test_read_cfrw_fixture_matches_independent_loader():
    d, ref = S.read_cfrw(F._path("tiny.cfrw")), F.load_cfrw()
    for k in ("n", "bits", "vocab", "nblocks", "nsb", "cwords", "na", "owords", "rrr_bytes", "packed_bytes"):
        assert d[k] == ref[k], k
    assert np.float32(d["h0"]) == np.float32(ref["h0"])
    assert d["nq"] == ref["pos"].size and d["nr"] == ref["rank_c"].size
    _same(d, ref, WAVELET + RRRW_Q)


def test_read_cffm_fixture_matches_independent_loader():
    d, ref = S.read_cffm(F._path("tiny.cffm")), F.load_cffm()
    for k in ("n", "bits", "vocab", "sigma", "nblocks", "nsb", "cwords", "na", "owords", "sa_sample", "rrr_bytes"):
        assert d[k] == ref[k], k
    assert d["npat"] == ref["pstart"].size and d["nloc"] == ref["locpos"].size
    _same(d, ref, WAVELET + FM)


@pytest.mark.parametrize("name,rd,wr", [("tiny.cfrw", S.read_cfrw, S.write_cfrw),
                                        ("tiny.cffm", S.read_cffm, S.write_cffm)])
def test_write_back_is_byte_identical(tmp_path, name, rd, wr):
    src = F._path(name)
    out = str(tmp_path / name)
    wr(out, rd(src))
    assert open(out, "rb").read() == open(src, "rb").read()


def test_cfrw_without_query_sections_round_trips(tmp_path):
    d = S.read_cfrw(F._path("tiny.cfrw"))
    bare = {k: v for k, v in d.items() if k not in RRRW_Q}
    out = str(tmp_path / "bare.cfrw")
    S.write_cfrw(out, bare)
    back = S.read_cfrw(out)
    assert back["nq"] == 0 and back["nr"] == 0
    _same(back, d, WAVELET)
    # the same file through the independent loader
    _same(F.load_cfrw(out), d, WAVELET)


def test_cffm_without_pattern_section_round_trips(tmp_path):
    d = S.read_cffm(F._path("tiny.cffm"))
    bare = {k: v for k, v in d.items() if k not in ("pat", "pstart", "plen", "count_golden", "locoff", "locpos")}
    out = str(tmp_path / "bare.cffm")
    S.write_cffm(out, bare)
    back = S.read_cffm(out)
    assert back["npat"] == 0 and back["nloc"] == 0 and back["locoff"].tolist() == [0]
    _same(back, d, WAVELET + ("C", "mwords", "msb", "sval"))
    _same(F.load_cffm(out), d, WAVELET + ("C", "mwords", "msb", "sval"))


@pytest.mark.parametrize("name,rd", [("tiny.cfrw", S.read_cfrw), ("tiny.cffm", S.read_cffm)])
def test_malformed_files_are_rejected(tmp_path, name, rd):
    raw = open(F._path(name), "rb").read()
    cases = {
        "truncated": raw[:-4],
        "extra": raw + b"\0\0\0\0",
        "header_only": raw[:40],
        "bad_magic": b"XXXX" + raw[4:],
        "bad_version": raw[:4] + (2).to_bytes(4, "little") + raw[8:],
        "empty": b"",
    }
    for label, blob in cases.items():
        p = tmp_path / f"{label}_{name}"
        p.write_bytes(blob)
        with pytest.raises(A.CfError):
            rd(str(p))
    with pytest.raises(A.CfError):
        rd(str(tmp_path / "does_not_exist"))


def test_reader_rejects_header_mismatch(tmp_path):
    """cf_rrrw_file_read checks that the caller's header is the file's (arrays were sized from it)."""
    import ctypes as C
    L = A.lib()
    path = F._path("tiny.cfrw").encode()
    h = S.cf_rrrw_file_header()
    A.check(L.cf_rrrw_file_read_header(path, C.byref(h)), "read_header")
    h.owords += 1
    arrays = S.cf_rrrw_arrays()
    q = S.cf_rrrw_file_queries()
    assert L.cf_rrrw_file_read(path, C.byref(h), C.byref(arrays), C.byref(q)) != 0


def test_null_arguments_are_rejected(tmp_path):
    import ctypes as C
    L = A.lib()
    h = S.cf_rrrw_file_header()
    assert L.cf_rrrw_file_read_header(None, C.byref(h)) != 0
    assert L.cf_rrrw_file_read_header(F._path("tiny.cfrw").encode(), None) != 0
    assert L.cf_rrrw_file_write(str(tmp_path / "x").encode(), None, None, None) != 0
    hf = S.cf_fm_file_header()
    assert L.cf_fm_file_read_header(None, C.byref(hf)) != 0
    assert L.cf_fm_file_write(str(tmp_path / "y").encode(), C.byref(hf), None, None) != 0


@pytest.mark.parametrize("bits", [3, 9])
def test_oracle_build_written_by_library_reads_back(tmp_path, bits):
    rng = np.random.default_rng(bits)
    n = 40_000
    tokens = rng.integers(0, 1 << bits, n).astype(np.uint32)
    w = O.rrrw_build(tokens, bits)
    d = {k: getattr(w, k) for k in WAVELET}
    d.update(n=n, bits=bits, vocab=1 << bits, nblocks=(n + 14) // 15, nsb=w.nsb, cwords=w.cwords, na=w.na,
             owords=w.offsets.size, rrr_bytes=w.rrr_bytes, packed_bytes=(n * bits + 7) // 8, h0=0.5)
    pos = rng.integers(0, n, 100).astype(np.uint32)
    d["pos"], d["access_golden"] = pos, O.rrrw_access(w, pos).astype(np.uint32)
    out = str(tmp_path / "o.cfrw")
    S.write_cfrw(out, d)
    back = F.load_cfrw(out)
    _same(back, d, WAVELET + ("pos", "access_golden"))
    assert back["rank_c"].size == 0


needs_tool = pytest.mark.skipif(O.ref_build_index() is None, reason="oracle/_ref/build_index not built")


@needs_tool
@pytest.mark.parametrize("n,vocab,seed", [(7001, 40, 3), (30011, 700, 11)])
def test_reference_tool_files_round_trip_byte_identically(tmp_path, n, vocab, seed):
    rw, fm = str(tmp_path / "r.cfrw"), str(tmp_path / "r.cffm")
    subprocess.run([O.ref_build_index(), rw, "--n", str(n), "--vocab", str(vocab), "--queries", "64", "--rank",
                    "64", "--seed", str(seed), "--fm", fm, "--patterns", "16", "--plen", "3", "--sa-sample", "8"],
                   check=True, capture_output=True, timeout=120)
    for src, rd, wr in ((rw, S.read_cfrw, S.write_cfrw), (fm, S.read_cffm, S.write_cffm)):
        out = src + ".again"
        d = rd(src)
        wr(out, d)
        assert open(out, "rb").read() == open(src, "rb").read(), src
    # the library reader agrees with the independent loader on the tool's files
    _same(S.read_cfrw(rw), F.load_cfrw(rw), WAVELET + RRRW_Q)
    _same(S.read_cffm(fm), F.load_cffm(fm), WAVELET + FM)


@needs_tool
def test_oracle_arrays_through_library_writer_equal_reference_tool_file(tmp_path):
    """The file a caller writes from independently built arrays (the oracle's RRR build of the tool's BWT) plus the
    tool's header scalars and query sections is the tool's file, byte for byte."""
    n, vocab, seed = 12007, 200, 5
    rw, tok = str(tmp_path / "t.cfrw"), str(tmp_path / "t.tok")
    subprocess.run([O.ref_build_index(), rw, "--n", str(n), "--vocab", str(vocab), "--queries", "50", "--rank",
                    "50", "--seed", str(seed), "--dump-tokens", tok], check=True, capture_output=True, timeout=120)
    raw = np.fromfile(tok, dtype=np.uint8)
    tokens = raw[8:].view(np.int32)
    s = np.concatenate([tokens.astype(np.int64) + 1, [0]]).astype(np.int32)
    sa = O.suffix_array(s)
    bwt = s[(sa.astype(np.int64) - 1) % s.size].astype(np.uint32)
    ref = F.load_cfrw(rw)
    w = O.rrrw_build(bwt, ref["bits"])
    d = {k: getattr(w, k) for k in WAVELET}
    for k in ("n", "bits", "vocab", "nblocks", "nsb", "cwords", "na", "owords", "rrr_bytes", "packed_bytes", "h0"):
        d[k] = ref[k]
    for k in RRRW_Q:
        d[k] = ref[k]
    out = str(tmp_path / "mine.cfrw")
    S.write_cfrw(out, d)
    assert open(out, "rb").read() == open(rw, "rb").read()


def _strip_packed_bytes(raw: bytes) -> bytes:
    """.cfrw bytes without the 8-byte packed_bytes figure (offset 60: magic, version, n, nine u32, rrr_bytes)."""
    return raw[:60] + raw[68:]


def _save_from_host(path, d, bwt):
    import torch
    idx = S.RrrWaveletIndex.from_host({**{k: d[k] for k in WAVELET}, "bits": d["bits"], "cwords": d["cwords"],
                                       "nsb": d["nsb"], "na": d["na"]}, device="cpu")
    lay = S.cf_rrrw_layout(n=d["n"], bits=d["bits"], nblocks=d["nblocks"], cwords=d["cwords"], nsb=d["nsb"],
                           na=d["na"], owords=d["owords"], rrr_bytes=d["rrr_bytes"])
    S.save_cfrw(path, idx, lay, d["vocab"], torch.from_numpy(np.ascontiguousarray(bwt).view(np.int32)),
                {k: d[k] for k in RRRW_Q})


def test_save_cfrw_header_figures_match_fixture(tmp_path):
    """save_cfrw derives h0 like the reference writers; fed tiny.cfrw's own arrays (host tensors) and the BWT they
    encode, it reproduces the file except packed_bytes. That figure is informational (the packed bit-plane
    wavelet's footprint): tiny.cfrw was written by the Python exporter (tools/export_rrr_wavelet.py:96), which takes
    it from the warp_compress package's GPUWavelet.index_bytes() (package not in the reference tree), while
    save_cfrw uses the C++ builder's formula (tools/build_index.cpp:404-405), pinned against that tool below."""
    d = F.load_cfrw()
    w = O.RrrwArrays(d["bits"], d["cwords"], d["nsb"], d["na"], *[d[f] for f in WAVELET])
    bwt = O.rrrw_access(w, np.arange(d["n"], dtype=np.uint32))
    out = str(tmp_path / "s.cfrw")
    _save_from_host(out, d, bwt)
    got, ref = open(out, "rb").read(), open(F._path("tiny.cfrw"), "rb").read()
    assert _strip_packed_bytes(got) == _strip_packed_bytes(ref)


@needs_tool
@pytest.mark.parametrize("n,vocab,seed", [(9000, 64, 2), (20000, 1000, 9)])
def test_save_cfrw_equals_reference_tool_file(tmp_path, n, vocab, seed):
    rw, tok = str(tmp_path / "t.cfrw"), str(tmp_path / "t.tok")
    subprocess.run([O.ref_build_index(), rw, "--n", str(n), "--vocab", str(vocab), "--queries", "32", "--rank",
                    "32", "--seed", str(seed), "--dump-tokens", tok], check=True, capture_output=True, timeout=120)
    tokens = np.fromfile(tok, dtype=np.uint8)[8:].view(np.int32)
    s = np.concatenate([tokens.astype(np.int64) + 1, [0]]).astype(np.int32)
    sa = O.suffix_array(s)
    bwt = s[(sa.astype(np.int64) - 1) % s.size].astype(np.uint32)
    out = str(tmp_path / "s.cfrw")
    _save_from_host(out, F.load_cfrw(rw), bwt)
    assert open(out, "rb").read() == open(rw, "rb").read()
