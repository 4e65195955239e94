"""Loaders for the reference's committed golden fixtures (data only, copied to tests/golden/fixtures/).

Binary layouts follow the reference exporter docstrings: .cfrw tools/export_rrr_wavelet.py:11-19,
.cffm tools/export_fm_index.py:19-29, .cfwv tools/export_reference.py:8-17, .cfrr tools/export_rrr.py:9-16.
Everything is little-endian and written field by field (no padding).
"""
from __future__ import annotations

import os
import struct

import numpy as np

FIXTURE_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "fixtures")


class _Reader:
    def __init__(self, path: str):
        with open(path, "rb") as f:
            self.buf = f.read()
        self.at = 0

    def magic(self) -> bytes:
        m = self.buf[self.at:self.at + 4]
        self.at += 4
        return m

    def scalars(self, fmt: str):
        vals = struct.unpack_from("<" + fmt, self.buf, self.at)
        self.at += struct.calcsize("<" + fmt)
        return vals

    def array(self, dtype, count: int) -> np.ndarray:
        dt = np.dtype(dtype).newbyteorder("<")
        a = np.frombuffer(self.buf, dtype=dt, count=int(count), offset=self.at).astype(np.dtype(dtype)).copy()
        self.at += a.nbytes
        return a

    def done(self) -> bool:
        return self.at == len(self.buf)


def _path(name: str) -> str:
    return os.path.join(FIXTURE_DIR, name)


def load_cfrw(path: str | None = None) -> dict:
    r = _Reader(path or _path("tiny.cfrw"))
    assert r.magic() == b"CFRW"
    (version, n, bits, vocab, nblocks, nsb, cwords, na, owords, nq, nr, rrr_bytes, packed_bytes, h0) = r.scalars(
        "IQIIIIIIIIIQQf")
    assert version == 1
    d = dict(version=version, n=n, bits=bits, vocab=vocab, nblocks=nblocks, nsb=nsb, cwords=cwords, na=na,
             owords=owords, rrr_bytes=rrr_bytes, packed_bytes=packed_bytes, h0=h0)
    d["classes"] = r.array(np.uint32, bits * cwords)
    d["offsets"] = r.array(np.uint32, owords)
    d["rank_a"] = r.array(np.int32, bits * na)
    d["rank_d"] = r.array(np.uint16, bits * (nsb + 1))
    d["off_a"] = r.array(np.int32, bits * na)
    d["off_d"] = r.array(np.uint16, bits * (nsb + 1))
    d["offbase"] = r.array(np.int32, bits)
    d["zeros"] = r.array(np.int32, bits)
    d["pos"] = r.array(np.uint32, nq)
    d["access_golden"] = r.array(np.uint32, nq)
    d["rank_c"] = r.array(np.uint32, nr)
    d["rank_i"] = r.array(np.uint32, nr)
    d["rank_golden"] = r.array(np.uint32, nr)
    assert r.done()
    return d


def load_cffm(path: str | None = None) -> dict:
    r = _Reader(path or _path("tiny.cffm"))
    assert r.magic() == b"CFFM"
    (version, n, bits, vocab, sigma, nblocks, nsb, cwords, na, owords, sa_sample, mw, msb, nsval, npat, patflat,
     nloc, rrr_bytes) = r.scalars("IQIIIIIIIIIIIIIIIQ")
    assert version == 1
    d = dict(version=version, n=n, bits=bits, vocab=vocab, sigma=sigma, nblocks=nblocks, nsb=nsb, cwords=cwords,
             na=na, owords=owords, sa_sample=sa_sample, rrr_bytes=rrr_bytes)
    d["classes"] = r.array(np.uint32, bits * cwords)
    d["offsets"] = r.array(np.uint32, owords)
    d["rank_a"] = r.array(np.int32, bits * na)
    d["rank_d"] = r.array(np.uint16, bits * (nsb + 1))
    d["off_a"] = r.array(np.int32, bits * na)
    d["off_d"] = r.array(np.uint16, bits * (nsb + 1))
    d["offbase"] = r.array(np.int32, bits)
    d["zeros"] = r.array(np.int32, bits)
    d["C"] = r.array(np.int32, sigma)
    d["mwords"] = r.array(np.uint32, mw)
    d["msb"] = r.array(np.int32, msb)
    d["sval"] = r.array(np.int32, nsval)
    d["pat"] = r.array(np.int32, patflat)
    d["pstart"] = r.array(np.int32, npat)
    d["plen"] = r.array(np.int32, npat)
    d["count_golden"] = r.array(np.uint32, npat)
    d["locoff"] = r.array(np.int32, npat + 1)
    d["locpos"] = r.array(np.int32, nloc)
    assert r.done()
    return d


def load_cfwv(path: str | None = None) -> dict:
    r = _Reader(path or _path("tiny.cfwv"))
    assert r.magic() == b"CFWV"
    version, levels, n, nwords, nblocks, nq, nr, token_bytes, vocab = r.scalars("IIQIIIIII")
    assert version == 3
    d = dict(version=version, levels=levels, n=n, nwords=nwords, nblocks=nblocks, token_bytes=token_bytes,
             vocab=vocab)
    d["bitplanes"] = r.array(np.uint32, levels * nwords)
    d["superblocks"] = r.array(np.int32, levels * (nblocks + 1))
    d["zeros"] = r.array(np.int32, levels)
    d["pos"] = r.array(np.uint32, nq)
    d["access_golden"] = r.array(np.uint32, nq)
    d["rank_c"] = r.array(np.uint32, nr)
    d["rank_i"] = r.array(np.uint32, nr)
    d["rank_golden"] = r.array(np.uint32, nr)
    tdt = {1: np.uint8, 2: np.uint16, 4: np.uint32}[token_bytes]
    d["tokens"] = r.array(tdt, n).astype(np.uint32)
    assert r.done()
    return d


def load_cfrr(path: str | None = None) -> dict:
    r = _Reader(path or _path("tiny.cfrr"))
    assert r.magic() == b"CFRR"
    (version, n, T, SB, nblocks, nsb, cwords, owords, nq, density, class_bits, offset_bits) = r.scalars(
        "IQIIIIIIIfQQ")
    assert version == 1
    d = dict(version=version, n=n, T=T, SB=SB, nblocks=nblocks, nsb=nsb, cwords=cwords, owords=owords,
             density=density, class_bits=class_bits, offset_bits=offset_bits)
    d["classes"] = r.array(np.uint32, cwords)
    d["offsets"] = r.array(np.uint32, owords)
    d["sbrank"] = r.array(np.int32, nsb + 1)
    d["sboff"] = r.array(np.int32, nsb + 1)
    d["pos"] = r.array(np.uint32, nq)
    d["rank_golden"] = r.array(np.uint32, nq)
    assert r.done()
    return d
