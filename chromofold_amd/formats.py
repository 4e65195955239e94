"""Readers and writers of the reference's binary exchange formats (host side).

Every format is little-endian: a 4-byte magic, a u32 version, header scalars written back to back without padding,
then the arrays back to back; the readers check the magic, the version and the exact file size the header
implies. Layouts follow the reference's exporter docstrings:

    .cfwv v3  tools/export_reference.py:8-13 (plus the trailing token array the exporter writes after the goldens)
    .cfrr v1  tools/export_rrr.py:10-14
    .cfrw v1  tools/export_rrr_wavelet.py:12-19 (also read / written by the C library: cf_rrrw_file_*)
    .cffm v1  tools/export_fm_index.py:19-28 (also read / written by the C library: cf_fm_file_*)
    .cfrs v1  tools/export_rans.py:13-17
    .cffw v1  tools/export_fused_matmul.py:14-17
    .cfkv v1  tools/export_kv_attention.py:14-21
    .cfdc v1  tools/export_delta.py:13-16
    .cfsg v1  tools/export_sparse_gather.py:14-20

`read(path)` returns (kind, dict of header fields and numpy arrays); `write(path, kind, fields)` checks that every
array has the length the header gives it and writes the file. Field names are the docstrings' (array names as
listed there; header counts as named there).
"""
from __future__ import annotations

import struct
from dataclasses import dataclass
from typing import Callable

import numpy as np

U8, U16, U32, I32, F32 = np.uint8, np.uint16, np.uint32, np.int32, np.float32


@dataclass(frozen=True)
class Spec:
    magic: bytes
    version: int
    header: tuple   # (name, struct code) after magic + version
    arrays: tuple   # (name, dtype or callable(header) -> dtype, count(header) -> int)


def _rrrw_arrays(bits="bits"):
    return (("classes", U32, lambda h: h[bits] * h["cwords"]), ("offsets", U32, lambda h: h["owords"]),
            ("rank_a", I32, lambda h: h[bits] * h["na"]), ("rank_d", U16, lambda h: h[bits] * (h["nsb"] + 1)),
            ("off_a", I32, lambda h: h[bits] * h["na"]), ("off_d", U16, lambda h: h[bits] * (h["nsb"] + 1)),
            ("offbase", I32, lambda h: h[bits]), ("zeros", I32, lambda h: h[bits]))


SPECS: dict[str, Spec] = {
    "cfwv": Spec(b"CFWV", 3,
                 (("levels", "I"), ("n", "Q"), ("nwords", "I"), ("nblocks", "I"), ("nqueries", "I"), ("nrank", "I"),
                  ("token_bytes", "I"), ("vocab", "I")),
                 (("words", U32, lambda h: h["levels"] * h["nwords"]),
                  ("superblocks", I32, lambda h: h["levels"] * (h["nblocks"] + 1)),
                  ("zeros", I32, lambda h: h["levels"]),
                  ("positions", U32, lambda h: h["nqueries"]), ("golden_tokens", U32, lambda h: h["nqueries"]),
                  ("rank_c", U32, lambda h: h["nrank"]), ("rank_i", U32, lambda h: h["nrank"]),
                  ("rank_golden", U32, lambda h: h["nrank"]),
                  ("tokens", lambda h: {1: U8, 2: U16, 4: U32}[h["token_bytes"]], lambda h: h["n"]))),
    "cfrr": Spec(b"CFRR", 1,
                 (("n", "Q"), ("T", "I"), ("SB", "I"), ("nblocks", "I"), ("nsb", "I"), ("cwords", "I"),
                  ("owords", "I"), ("nqueries", "I"), ("density", "f"), ("class_bits", "Q"), ("offset_bits", "Q")),
                 (("classes", U32, lambda h: h["cwords"]), ("offsets", U32, lambda h: h["owords"]),
                  ("sbrank", I32, lambda h: h["nsb"] + 1), ("sboff", I32, lambda h: h["nsb"] + 1),
                  ("positions", U32, lambda h: h["nqueries"]), ("golden_rank1", U32, lambda h: h["nqueries"]))),
    "cfrw": Spec(b"CFRW", 1,
                 (("n", "Q"), ("bits", "I"), ("vocab", "I"), ("nblocks", "I"), ("nsb", "I"), ("cwords", "I"),
                  ("na", "I"), ("owords", "I"), ("nqueries", "I"), ("nrank", "I"), ("rrr_bytes", "Q"),
                  ("packed_bytes", "Q"), ("h0", "f")),
                 _rrrw_arrays() + (
                     ("pos", U32, lambda h: h["nqueries"]), ("access_golden", U32, lambda h: h["nqueries"]),
                     ("rank_c", U32, lambda h: h["nrank"]), ("rank_i", U32, lambda h: h["nrank"]),
                     ("rank_golden", U32, lambda h: h["nrank"]))),
    "cffm": Spec(b"CFFM", 1,
                 (("n", "Q"), ("bits", "I"), ("vocab", "I"), ("sigma", "I"), ("nblocks", "I"), ("nsb", "I"),
                  ("cwords", "I"), ("na", "I"), ("owords", "I"), ("sa_sample", "I"), ("mwords_len", "I"),
                  ("msb_len", "I"), ("nsval", "I"), ("npat", "I"), ("patflat", "I"), ("nloc", "I"),
                  ("rrr_bytes", "Q")),
                 _rrrw_arrays() + (
                     ("C", I32, lambda h: h["sigma"]), ("mwords", U32, lambda h: h["mwords_len"]),
                     ("msb", I32, lambda h: h["msb_len"]), ("sval", I32, lambda h: h["nsval"]),
                     ("pat", I32, lambda h: h["patflat"]), ("pstart", I32, lambda h: h["npat"]),
                     ("plen", I32, lambda h: h["npat"]), ("count_golden", U32, lambda h: h["npat"]),
                     ("locoff", I32, lambda h: h["npat"] + 1), ("locpos", I32, lambda h: h["nloc"]))),
    "cfrs": Spec(b"CFRS", 1,
                 (("n", "Q"), ("block", "I"), ("V", "I"), ("M", "I"), ("nblocks", "I"), ("data_bytes", "I"),
                  ("slotlen", "I"), ("h0", "f"), ("rans_bits", "Q"), ("huff_bits", "Q")),
                 (("data", U8, lambda h: h["data_bytes"]), ("byte_off", I32, lambda h: h["nblocks"]),
                  ("state0", U32, lambda h: h["nblocks"]), ("slot2sym", I32, lambda h: h["slotlen"]),
                  ("freq", I32, lambda h: h["V"]), ("cum", I32, lambda h: h["V"]), ("golden", I32, lambda h: h["n"]))),
    "cffw": Spec(b"CFFW", 1,
                 (("M", "I"), ("K", "I"), ("B", "I"), ("bits", "I"), ("block", "I"), ("maxlen", "I"), ("zero", "I"),
                  ("nwords", "I"), ("nblocks", "I"), ("lutlen", "I"), ("scale", "f"), ("resident_bytes", "Q"),
                  ("dense_bytes", "Q")),
                 (("words", U32, lambda h: h["nwords"]), ("block_off", I32, lambda h: h["nblocks"]),
                  ("lut", I32, lambda h: h["lutlen"]), ("x", F32, lambda h: h["B"] * h["K"]),
                  ("y_golden", F32, lambda h: h["B"] * h["M"]))),
    "cfkv": Spec(b"CFKV", 1,
                 (("seq", "I"), ("dim", "I"), ("nq", "I"), ("window", "I"), ("bits", "I"), ("block", "I"),
                  ("zero", "I"), ("kmaxlen", "I"), ("knwords", "I"), ("knblocks", "I"), ("klutlen", "I"),
                  ("vmaxlen", "I"), ("vnwords", "I"), ("vnblocks", "I"), ("vlutlen", "I"), ("softmax_scale", "f"),
                  ("resident_bytes", "Q"), ("dense_bytes", "Q")),
                 (("kwords", U32, lambda h: h["knwords"]), ("kboff", I32, lambda h: h["knblocks"]),
                  ("klut", I32, lambda h: h["klutlen"]), ("vwords", U32, lambda h: h["vnwords"]),
                  ("vboff", I32, lambda h: h["vnblocks"]), ("vlut", I32, lambda h: h["vlutlen"]),
                  ("kscale", F32, lambda h: h["dim"]), ("vscale", F32, lambda h: h["seq"]),
                  ("Q", F32, lambda h: h["nq"] * h["dim"]), ("golden", F32, lambda h: h["nq"] * h["dim"]))),
    "cfdc": Spec(b"CFDC", 1,
                 (("N", "I"), ("nbase", "I"), ("ndelta", "I"), ("vocab", "I"), ("total_tokens", "Q")),
                 (("base", I32, lambda h: h["nbase"]), ("lengths", I32, lambda h: h["N"]),
                  ("dstart", I32, lambda h: h["N"]), ("dlen", I32, lambda h: h["N"]),
                  ("dpos", I32, lambda h: h["ndelta"]), ("dval", I32, lambda h: h["ndelta"]),
                  ("ostart", I32, lambda h: h["N"] + 1), ("originals", I32, lambda h: h["total_tokens"]))),
    "cfsg": Spec(b"CFSG", 1,
                 (("n", "Q"), ("bits", "I"), ("vocab", "I"), ("emb_rows", "I"), ("dim", "I"), ("cwords", "I"),
                  ("nsb", "I"), ("na", "I"), ("owords", "I"), ("npos", "I"), ("rrr_bytes", "Q")),
                 _rrrw_arrays() + (
                     ("embedding", F32, lambda h: h["emb_rows"] * h["dim"]),
                     ("positions", U32, lambda h: h["npos"]), ("golden", F32, lambda h: h["npos"] * h["dim"]))),
}
KIND_BY_MAGIC = {s.magic: k for k, s in SPECS.items()}


def _dtype(d, h) -> np.dtype:
    return np.dtype(d(h) if isinstance(d, Callable) and not isinstance(d, type) else d)


def _header_fmt(spec: Spec) -> str:
    return "<4sI" + "".join(code for _, code in spec.header)


def read(path: str) -> tuple[str, dict]:
    """Parse a file of any of the formats above; raises ValueError on a bad magic, version or size."""
    with open(path, "rb") as f:
        buf = f.read()
    if len(buf) < 8 or buf[:4] not in KIND_BY_MAGIC:
        raise ValueError(f"{path}: unknown magic {buf[:4]!r}")
    kind = KIND_BY_MAGIC[buf[:4]]
    spec = SPECS[kind]
    fmt = _header_fmt(spec)
    if len(buf) < struct.calcsize(fmt):
        raise ValueError(f"{path}: truncated header")
    vals = struct.unpack_from(fmt, buf, 0)
    if vals[1] != spec.version:
        raise ValueError(f"{path}: {kind} version {vals[1]} (expected {spec.version})")
    h = {name: v for (name, _), v in zip(spec.header, vals[2:])}
    at = struct.calcsize(fmt)
    need = at + sum(int(cnt(h)) * _dtype(dt, h).itemsize for _, dt, cnt in spec.arrays)
    if len(buf) != need:
        raise ValueError(f"{path}: {len(buf)} bytes, the header implies {need}")
    out = dict(h)
    for name, dt, cnt in spec.arrays:
        t = _dtype(dt, h).newbyteorder("<")
        n = int(cnt(h))
        out[name] = np.frombuffer(buf, dtype=t, count=n, offset=at).astype(t.newbyteorder("="))
        at += n * t.itemsize
    return kind, out


def write(path: str, kind: str, fields: dict) -> None:
    """Write `fields` (every header field and array of the format) as a `kind` file."""
    spec = SPECS[kind]
    h = {name: fields[name] for name, _ in spec.header}
    parts = [struct.pack(_header_fmt(spec), spec.magic, spec.version, *[h[name] for name, _ in spec.header])]
    for name, dt, cnt in spec.arrays:
        a = np.ascontiguousarray(fields[name], dtype=_dtype(dt, h)).ravel()
        if a.size != int(cnt(h)):
            raise ValueError(f"{kind}.{name}: {a.size} elements, the header implies {int(cnt(h))}")
        parts.append(a.astype(a.dtype.newbyteorder("<")).tobytes())
    with open(path, "wb") as f:
        for p in parts:
            f.write(p)
