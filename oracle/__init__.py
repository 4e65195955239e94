"""CPU oracle for the chromoFold hot path — TEST INFRASTRUCTURE ONLY.

ctypes bindings over ``oracle/liboracle.so`` (built from ``oracle/*.cpp`` by ``oracle/Makefile``). Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import this package, and only
as the checker or the timed CPU baseline; the product package ``chromofold_amd`` never imports it.

Each wrapper names the reference function it restates; the C++ sources carry the file:line citations.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_DIR = os.path.join(HERE, "_ref")

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run `make -C oracle`)")
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


P = C.c_void_p
I32, I64, U32 = C.c_int32, C.c_int64, C.c_uint32


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


class OrRrrw(C.Structure):
    _fields_ = [("classes", P), ("offsets", P), ("rank_a", P), ("rank_d", P), ("off_a", P), ("off_d", P),
                ("offbase", P), ("zeros", P), ("bits", C.c_int), ("cwords", C.c_int), ("nsb", C.c_int),
                ("na", C.c_int)]


class OrFm(C.Structure):
    _fields_ = [("w", OrRrrw), ("C", P), ("mwords", P), ("msb", P), ("sval", P), ("sigma", C.c_int),
                ("n", C.c_int), ("sa_sample", C.c_int)]


def _declare(L):
    sig = {
        "or_rrr_tables": (None, [P, P]),
        "or_num_threads": (C.c_int, []),
        "or_set_threads": (None, [C.c_int]),
        "or_rrrw_build": (P, [P, I64, C.c_int]),
        "or_rrrw_info": (None, [P, P]),
        "or_rrrw_copy": (None, [P] * 9),
        "or_rrrw_free": (None, [P]),
        "or_rrrw_rank1": (C.c_int, [P, C.c_int, C.c_int]),
        "or_rrrw_access": (None, [P, P, P, I64]),
        "or_rrrw_rank": (None, [P, P, P, P, I64]),
        "or_suffix_array_doubling": (None, [P, I32, P]),
        "or_suffix_array_radix": (None, [P, I32, P]),
        "or_fm_build": (I32, [P, P, I32, I32, I32, P, P, P, P]),
        "or_fm_ranges": (None, [P, P, P, P, P, P, I64]),
        "or_fm_count": (None, [P, P, P, P, P, I64]),
        "or_fm_locate": (None, [P, P, P, I64]),
        "or_naive_positions": (I64, [P, I64, P, C.c_int, P, I64]),
        "or_packed_build": (None, [P, I64, C.c_int, P, P, P]),
        "or_packed_access": (None, [P, P, P, C.c_int, C.c_int, C.c_int, P, P, I64]),
        "or_packed_rank": (None, [P, P, P, C.c_int, C.c_int, C.c_int, P, P, P, I64]),
        "or_packed_rank1": (C.c_int, [P, P, C.c_int]),
        "or_rrr_rank1": (None, [P, P, P, P, P, P, I64]),
        "or_rrr_plane_build": (P, [P, I64]),
        "or_rrr_plane_info": (None, [P, P]),
        "or_rrr_plane_copy": (None, [P, P, P, P, P]),
        "or_rrr_plane_free": (None, [P]),
        "or_rrr_decode_all": (None, [P, P, I64, I64, P]),
        "or_kv_fixture_quantize": (None, [P, P, U32, U32, U32, P, P, P, P, P, P]),
        "or_pack_fixed": (None, [P, C.c_uint64, U32, P]),
        "or_huffman_decode": (None, [P, P, C.c_int, I64, I64, P]),
        "or_rans_block_decode": (None, [P, P, P, P, P, P, C.c_int, C.c_int, P]),
        "or_qw_rans_decode": (C.c_int, [P, U32, U32, P, P, P, U32, U32, C.c_int, P]),
        "or_paged_attention_f64": (C.c_int, [P, U32, U32, U32, U32, U32, U32, C.c_float, U32, P, P, P, P, P, P,
                                             P, P, U32, U32, P]),
        "or_dense_attention_f64": (None, [P, U32, P, P, U32, C.c_float, P]),
        "or_kv_window_attention_f64": (None, [P, P, P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, P]),
        "or_kv_decode_group": (C.c_int, [P, P, U32, P, P, P, P, P, P, P]),
        "or_kv_pool_attention": (C.c_int, [P, P, U32, P, P, P, P, U32, U32, U32, U32, C.c_float, P, C.c_int]),
        "or_kv_quantize_page_absmax": (None, [P, U32, P, P]),
        "or_nib_seal": (C.c_int, [P, U32, U32, P, P, P, P, P]),
        "or_nib_attention": (None, [U32, P, P, P, P, P, P, U32, P, P, U32, U32, P, U32, U32, U32, U32, U32,
                                    C.c_float, U32, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name, None)
        if fn is None:
            continue
        fn.restype = res
        fn.argtypes = args


def set_threads(t: int) -> None:
    lib().or_set_threads(int(t))


def num_threads() -> int:
    return int(lib().or_num_threads())


def rrr_tables() -> tuple[np.ndarray, np.ndarray]:
    """binom[16*16] and width[16] (reference tools/build_index.cpp:31-42)."""
    b = np.zeros(256, np.int32)
    w = np.zeros(16, np.int32)
    lib().or_rrr_tables(_ptr(b), _ptr(w))
    return b, w


# ------------------------------------------------------------------ RRR wavelet matrix
@dataclass
class RrrwArrays:
    """Host arrays of an RRR wavelet matrix, field-for-field the cf_rrrw_view / .cfrw payload."""
    bits: int
    cwords: int
    nsb: int
    na: int
    classes: np.ndarray
    offsets: np.ndarray
    rank_a: np.ndarray
    rank_d: np.ndarray
    off_a: np.ndarray
    off_d: np.ndarray
    offbase: np.ndarray
    zeros: np.ndarray
    rrr_bytes: int = 0

    def view(self) -> OrRrrw:
        return OrRrrw(_ptr(self.classes), _ptr(self.offsets), _ptr(self.rank_a), _ptr(self.rank_d),
                      _ptr(self.off_a), _ptr(self.off_d), _ptr(self.offbase), _ptr(self.zeros),
                      self.bits, self.cwords, self.nsb, self.na)


def rrrw_build(tokens: np.ndarray, bits: int) -> RrrwArrays:
    """RRR wavelet matrix of `tokens` (reference tools/build_index.cpp:172-218)."""
    tok = np.ascontiguousarray(tokens, dtype=np.uint32)
    L = lib()
    h = L.or_rrrw_build(_ptr(tok), tok.size, bits)
    info = np.zeros(10, np.int64)
    L.or_rrrw_info(h, _ptr(info))
    b, cw, nsb, na, ow, ncls, nra, nrd, rb = (int(x) for x in info[:9])
    a = RrrwArrays(b, cw, nsb, na, np.zeros(ncls, np.uint32), np.zeros(ow, np.uint32), np.zeros(nra, np.int32),
                   np.zeros(nrd, np.uint16), np.zeros(nra, np.int32), np.zeros(nrd, np.uint16),
                   np.zeros(b, np.int32), np.zeros(b, np.int32), rb)
    L.or_rrrw_copy(h, _ptr(a.classes), _ptr(a.offsets), _ptr(a.rank_a), _ptr(a.rank_d), _ptr(a.off_a),
                   _ptr(a.off_d), _ptr(a.offbase), _ptr(a.zeros))
    L.or_rrrw_free(h)
    return a


def rrrw_access(w: RrrwArrays, pos: np.ndarray) -> np.ndarray:
    pos = np.ascontiguousarray(pos, np.uint32)
    out = np.zeros(pos.size, np.uint32)
    v = w.view()
    lib().or_rrrw_access(C.byref(v), _ptr(pos), _ptr(out), pos.size)
    return out


def rrrw_rank(w: RrrwArrays, sym: np.ndarray, pos: np.ndarray) -> np.ndarray:
    sym = np.ascontiguousarray(sym, np.uint32)
    pos = np.ascontiguousarray(pos, np.uint32)
    out = np.zeros(pos.size, np.uint32)
    v = w.view()
    lib().or_rrrw_rank(C.byref(v), _ptr(sym), _ptr(pos), _ptr(out), pos.size)
    return out


# ------------------------------------------------------------------ suffix array / FM-index
def suffix_array(s: np.ndarray, method: str = "radix") -> np.ndarray:
    s = np.ascontiguousarray(s, np.int32)
    sa = np.zeros(s.size, np.int32)
    fn = lib().or_suffix_array_radix if method == "radix" else lib().or_suffix_array_doubling
    fn(_ptr(s), s.size, _ptr(sa))
    return sa


@dataclass
class FmArrays:
    w: RrrwArrays
    C: np.ndarray
    mwords: np.ndarray
    msb: np.ndarray
    sval: np.ndarray
    sigma: int
    n: int
    sa_sample: int

    def view(self) -> OrFm:
        return OrFm(self.w.view(), _ptr(self.C), _ptr(self.mwords), _ptr(self.msb), _ptr(self.sval), self.sigma,
                    self.n, self.sa_sample)


def fm_text(tokens: np.ndarray) -> np.ndarray:
    """s = (tokens + 1) ++ [0] (reference tools/build_index.cpp:369-371)."""
    s = np.empty(tokens.size + 1, np.int32)
    s[:-1] = np.asarray(tokens, np.int64) + 1
    s[-1] = 0
    return s


def fm_build(tokens: np.ndarray, sa_sample: int, sa: np.ndarray | None = None) -> tuple[FmArrays, np.ndarray]:
    """Full FM build: SA -> BWT -> RRR wavelet -> C/marks/msb/sval (reference build_index.cpp:368-469)."""
    s = fm_text(tokens)
    n = s.size
    if sa is None:
        sa = suffix_array(s)
    bwt = s[(sa.astype(np.int64) - 1) % n].astype(np.int32)
    sigma = int(bwt.max()) + 1
    bits = max(1, int(sigma - 1).bit_length())
    w = rrrw_build(bwt.astype(np.uint32), bits)
    nw = (n + 31) // 32
    nb = (nw + 7) // 8
    Ct = np.zeros(sigma, np.int32)
    mw = np.zeros(nw, np.uint32)
    msb = np.zeros(nb + 1, np.int32)
    sval = np.zeros(n // sa_sample + 2, np.int32)
    ns = lib().or_fm_build(_ptr(sa), _ptr(bwt), n, sigma, sa_sample, _ptr(Ct), _ptr(mw), _ptr(msb), _ptr(sval))
    return FmArrays(w, Ct, mw, msb, sval[:ns].copy(), sigma, n, sa_sample), bwt


def fm_ranges(f: FmArrays, pat: np.ndarray, pstart: np.ndarray, plen: np.ndarray):
    lo = np.zeros(pstart.size, np.int32)
    hi = np.zeros(pstart.size, np.int32)
    v = f.view()
    lib().or_fm_ranges(C.byref(v), _ptr(pat), _ptr(pstart), _ptr(plen), _ptr(lo), _ptr(hi), pstart.size)
    return lo, hi


def fm_count(f: FmArrays, pat: np.ndarray, pstart: np.ndarray, plen: np.ndarray) -> np.ndarray:
    out = np.zeros(pstart.size, np.uint32)
    v = f.view()
    lib().or_fm_count(C.byref(v), _ptr(pat), _ptr(pstart), _ptr(plen), _ptr(out), pstart.size)
    return out


def fm_locate(f: FmArrays, rows: np.ndarray) -> np.ndarray:
    rows = np.ascontiguousarray(rows, np.int32)
    out = np.zeros(rows.size, np.int32)
    v = f.view()
    lib().or_fm_locate(C.byref(v), _ptr(rows), _ptr(out), rows.size)
    return out


def naive_positions(seq: np.ndarray, pat: np.ndarray, cap: int = 1 << 20) -> np.ndarray:
    seq = np.ascontiguousarray(seq, np.int32)
    pat = np.ascontiguousarray(pat, np.int32)
    out = np.zeros(cap, np.int32)
    k = lib().or_naive_positions(_ptr(seq), seq.size, _ptr(pat), pat.size, _ptr(out), cap)
    return out[:min(k, cap)].copy()


def naive_count(seq: np.ndarray, pat: np.ndarray) -> int:
    seq = np.ascontiguousarray(seq, np.int32)
    pat = np.ascontiguousarray(pat, np.int32)
    return int(lib().or_naive_positions(_ptr(seq), seq.size, _ptr(pat), pat.size, None, 0))


# ------------------------------------------------------------------ packed wavelet / RRR bitvector
def packed_build(tokens: np.ndarray, levels: int):
    tok = np.ascontiguousarray(tokens, np.uint32)
    n = tok.size
    nwords = (n + 31) // 32
    nblocks = (nwords + 7) // 8
    bp = np.zeros(levels * nwords, np.uint32)
    sb = np.zeros(levels * (nblocks + 1), np.int32)
    z = np.zeros(levels, np.int32)
    lib().or_packed_build(_ptr(tok), n, levels, _ptr(bp), _ptr(sb), _ptr(z))
    return bp, sb, z, nwords, nblocks


def packed_access(bp, sb, z, levels, nwords, nblocks, pos):
    pos = np.ascontiguousarray(pos, np.uint32)
    out = np.zeros(pos.size, np.uint32)
    lib().or_packed_access(_ptr(bp), _ptr(sb), _ptr(z), levels, nwords, nblocks, _ptr(pos), _ptr(out), pos.size)
    return out


def packed_rank(bp, sb, z, levels, nwords, nblocks, sym, pos):
    sym = np.ascontiguousarray(sym, np.uint32)
    pos = np.ascontiguousarray(pos, np.uint32)
    out = np.zeros(pos.size, np.uint32)
    lib().or_packed_rank(_ptr(bp), _ptr(sb), _ptr(z), levels, nwords, nblocks, _ptr(sym), _ptr(pos), _ptr(out),
                         pos.size)
    return out


def rrr_rank1(classes, offsets, sbrank, sboff, pos) -> np.ndarray:
    pos = np.ascontiguousarray(pos, np.uint32)
    out = np.zeros(pos.size, np.uint32)
    lib().or_rrr_rank1(_ptr(classes), _ptr(offsets), _ptr(sbrank), _ptr(sboff), _ptr(pos), _ptr(out), pos.size)
    return out


def rrr_plane_build(bits01: np.ndarray):
    b = np.ascontiguousarray(bits01, np.uint8)
    L = lib()
    h = L.or_rrr_plane_build(_ptr(b), b.size)
    info = np.zeros(7, np.int64)
    L.or_rrr_plane_info(h, _ptr(info))
    nblocks, nsb, cwords, owords = (int(x) for x in info[:4])
    cls = np.zeros(cwords, np.uint32)
    off = np.zeros(owords, np.uint32)
    sbr = np.zeros(nsb + 1, np.int32)
    sbo = np.zeros(nsb + 1, np.int32)
    L.or_rrr_plane_copy(h, _ptr(cls), _ptr(off), _ptr(sbr), _ptr(sbo))
    L.or_rrr_plane_free(h)
    return dict(nblocks=nblocks, nsb=nsb, cwords=cwords, owords=owords, class_bits=int(info[4]),
                offset_bits=int(info[5]), zeros=int(info[6]), classes=cls, offsets=off, sbrank=sbr, sboff=sbo)


def rrr_decode_all(classes, offsets, nblocks: int, off_base_bit: int = 0) -> np.ndarray:
    out = np.zeros(nblocks * 15, np.uint8)
    lib().or_rrr_decode_all(_ptr(classes), _ptr(offsets), nblocks, off_base_bit, _ptr(out))
    return out


# ------------------------------------------------------------------ paged KV
def kv_decode_group(blob: np.ndarray, tables: np.ndarray | None, head: int, head_dim: int, states=None,
                    full: bool = False):
    """Decode one kv_codec_ext group blob -> (k_sym [4, 16, D], v_sym [4, 16, D], k_scales[4], v_scales[4],
    token_counts[4]); full=True appends (end_states [2, 64] uint32, chain flag). `states` [2, 64] are the lane states
    the previous group of the chain ended with, needed when the blob continues a chain (header chain == 0)."""
    blob = np.ascontiguousarray(blob, np.uint8)
    ks = np.zeros((4, 16, head_dim), np.uint8)
    vs = np.zeros((4, 16, head_dim), np.uint8)
    ksc = np.zeros(4, np.float32)
    vsc = np.zeros(4, np.float32)
    tc = np.zeros(4, np.uint32)
    st = np.zeros((2, 64), np.uint32) if states is None else np.array(states, np.uint32).reshape(2, 64)
    chain = C.c_uint32(0)
    if states is None and kv_group_continues(blob):
        raise ValueError("the group continues a chain: pass the states its predecessor ended with")
    tab = None if tables is None else np.ascontiguousarray(tables, np.uint8)
    rc = lib().or_kv_decode_group(_ptr(blob), _ptr(tab), head, _ptr(ks), _ptr(vs), _ptr(ksc), _ptr(vsc), _ptr(tc),
                                  _ptr(st), C.byref(chain))
    if rc != 0:
        raise ValueError("group blob failed to decode")
    return (ks, vs, ksc, vsc, tc, st, chain.value) if full else (ks, vs, ksc, vsc, tc)


def kv_group_continues(blob: np.ndarray) -> bool:
    """True for a RANS_HYBRID group blob that continues the chain of the group before it."""
    b = np.asarray(blob, np.uint8)
    return int(b[:4].view(np.uint32)[0]) == 2 and int(b[8:10].view(np.uint16)[0]) == 0


def kv_decode_run(blobs, tables, head: int, head_dim: int):
    """Decode the groups of one (sequence, KV head) in token order, carrying each chain's lane states from a group
    to the one that continues it, and check that every chain ends with all states at 2^16 (the encoder's start).
    blobs: list of group blobs (each long enough to hold its group). Returns a list of 5-tuples as kv_decode_group."""
    out, states = [], None
    for g, blob in enumerate(blobs):
        ks, vs, ksc, vsc, tc, st, chain = kv_decode_group(blob, tables, head, head_dim,
                                                           states if kv_group_continues(blob) else None, full=True)
        ends = g + 1 == len(blobs) or not kv_group_continues(blobs[g + 1])
        is_rans = int(np.asarray(blob, np.uint8)[:4].view(np.uint32)[0]) == 2
        if is_rans and ends and not (st == 65536).all():
            raise ValueError(f"chain ending at group {g} does not return to the initial states")
        states = st if is_rans else None
        out.append((ks, vs, ksc, vsc, tc))
    return out


def kv_pool_attention(pool, group_offsets, seq_tokens, query_pos, tables, queries, kv_heads: int, head_dim: int,
                      softmax_scale: float, nseq: int | None = None, threads: int = 0):
    """float64 attention of one query row per sequence over a batched pool (host copies of the cf_kv_batched_desc
    arrays; group_offsets [S, H, max_groups]), for the first `nseq` sequences on `threads` OpenMP threads (0 = all).
    Returns out [nseq, q_heads, D] float32; raises when a blob fails to decode."""
    group_offsets = np.ascontiguousarray(group_offsets, np.uint32)
    S, H, G = group_offsets.shape
    nseq = S if nseq is None else nseq
    queries = np.ascontiguousarray(queries, np.float32)
    qh = queries.shape[1]
    out = np.zeros((nseq, qh, head_dim), np.float32)
    bad = lib().or_kv_pool_attention(_ptr(np.ascontiguousarray(pool, np.uint8)), _ptr(group_offsets), G,
                                     _ptr(np.ascontiguousarray(seq_tokens, np.uint32)),
                                     _ptr(np.ascontiguousarray(query_pos, np.uint32)),
                                     _ptr(np.ascontiguousarray(tables, np.uint8)), _ptr(queries), nseq, H, qh,
                                     head_dim, softmax_scale, _ptr(out), threads)
    if bad:
        raise ValueError(f"{bad} (sequence, head) units failed to decode")
    return out


def kv_quantize_absmax(x: np.ndarray):
    x = np.ascontiguousarray(x, np.float32)
    sym = np.zeros(x.size, np.uint8)
    sc = C.c_float(0)
    lib().or_kv_quantize_page_absmax(_ptr(x), x.size, _ptr(sym), C.byref(sc))
    return sym.reshape(x.shape), sc.value


def kv_fixture_quantize(k: np.ndarray, v: np.ndarray, bits: int):
    """reference kv_gpu_fixture encode_page quantiser: (k_sym, v_sym, k_scales[D], v_scales[T], k_deq, v_deq)."""
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    T, D = k.shape
    out = [np.zeros((T, D), np.uint8), np.zeros((T, D), np.uint8), np.zeros(D, np.float32), np.zeros(T, np.float32),
           np.zeros((T, D), np.float32), np.zeros((T, D), np.float32)]
    lib().or_kv_fixture_quantize(_ptr(k), _ptr(v), T, D, bits, *[_ptr(a) for a in out])
    return tuple(out)


def pack_fixed(sym: np.ndarray, bits: int) -> np.ndarray:
    sym = np.ascontiguousarray(sym, np.uint8).ravel()
    words = np.zeros((sym.size * bits + 31) // 32, np.uint32)
    lib().or_pack_fixed(_ptr(sym), sym.size, bits, _ptr(words))
    return words


def huffman_decode(words, lut, maxlen: int, pos: int, n: int) -> np.ndarray:
    out = np.zeros(n, np.int32)
    lib().or_huffman_decode(_ptr(np.ascontiguousarray(words, np.uint32)), _ptr(np.ascontiguousarray(lut, np.int32)),
                            maxlen, pos, n, _ptr(out))
    return out


def rans_block_decode(data, byte_off, state0, slot2sym, freq, cum, block: int, n: int) -> np.ndarray:
    out = np.zeros(n, np.int32)
    a = [np.ascontiguousarray(data, np.uint8), np.ascontiguousarray(byte_off, np.int32),
         np.ascontiguousarray(state0, np.uint32), np.ascontiguousarray(slot2sym, np.int32),
         np.ascontiguousarray(freq, np.int32), np.ascontiguousarray(cum, np.int32)]
    lib().or_rans_block_decode(*[_ptr(x) for x in a], block, n, _ptr(out))
    return out


def qw_rans_decode(words, chunk_words: int, last_words: int, offsets, states, cums, rows: int, cols: int,
                   mistake: int = 0):
    """Decode a CF_QW_CODEC_RANS matrix (chromofold_qw.h) to its [rows, cols] u8 symbols; returns (symbols, number of
    inconsistent stripes)."""
    out = np.zeros((rows, cols), np.uint8)
    a = [np.ascontiguousarray(words).view(np.uint16), np.ascontiguousarray(offsets, np.uint32),
         np.ascontiguousarray(states, np.uint32), np.ascontiguousarray(cums, np.uint16)]
    bad = lib().or_qw_rans_decode(_ptr(a[0]), chunk_words, last_words, _ptr(a[1]), _ptr(a[2]), _ptr(a[3]), rows,
                                  cols, mistake, _ptr(out))
    return out, int(bad)


def paged_attention_f64(q, q_heads, kv_heads, D, gqa, query_token, window, scale, pages, tail=None):
    """pages: list of (kv_head, token_begin, K [n, D], V [n, D]) dequantised; tail: (token_begin, K [n, kvh, D],
    V [n, kvh, D]) or None. Returns (out [q_heads, D], number of heads with no visible token)."""
    q = np.ascontiguousarray(q, np.float32)
    n = len(pages)
    kvh = np.array([p[0] for p in pages], np.uint32)
    tok0 = np.array([p[1] for p in pages], np.uint32)
    ntok = np.array([p[2].shape[0] for p in pages], np.uint32)
    off = np.zeros(n, np.uint64)
    if n:
        off[1:] = np.cumsum(ntok[:-1])
        K = np.ascontiguousarray(np.concatenate([p[2] for p in pages]), np.float32)
        V = np.ascontiguousarray(np.concatenate([p[3] for p in pages]), np.float32)
    else:
        K = V = np.zeros((1, D), np.float32)
    if tail is not None:
        t0, tk, tv = tail
        tk = np.ascontiguousarray(tk, np.float32)
        tv = np.ascontiguousarray(tv, np.float32)
        tn = tk.shape[0]
    else:
        t0, tk, tv, tn = 0, None, None, 0
    out = np.zeros((q_heads, D), np.float32)
    empty = lib().or_paged_attention_f64(_ptr(q), q_heads, kv_heads, D, gqa, query_token, window, scale, n,
                                         _ptr(kvh), _ptr(tok0), _ptr(ntok), _ptr(off), _ptr(K), _ptr(V), _ptr(tk),
                                         _ptr(tv), t0, tn, _ptr(out))
    return out, empty


def dense_attention_f64(q, k, v, scale):
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    out = np.zeros(q.shape[-1], np.float32)
    lib().or_dense_attention_f64(_ptr(q), q.shape[-1], _ptr(k), _ptr(v), k.shape[0], scale, _ptr(out))
    return out


def kv_window_attention_f64(K, V, Q, nq: int, window: int, sscale: float) -> np.ndarray:
    """reference fused_kv_attention.cu:27-65 over dequantised K/V [seq, dim] (fp64 accumulation)."""
    K, V, Q = (np.ascontiguousarray(a, np.float32) for a in (K, V, Q))
    seq, dim = K.shape
    out = np.zeros((nq, dim), np.float32)
    lib().or_kv_window_attention_f64(_ptr(K), _ptr(V), _ptr(Q), seq, dim, nq, window, sscale, _ptr(out))
    return out


def qmatmul_f64(x: np.ndarray, sym: np.ndarray, scale, zero) -> np.ndarray:
    """reference fused_matmul.cu:17-38: y[b, m] = sum_k x[b, k] * ((q[m, k] - zero) * scale), in float64. `scale` is
    a scalar (per tensor) or an array broadcastable to q (e.g. per (row, 64-column block) scales repeated over the
    block)."""
    w = (sym.astype(np.float64) - zero) * np.asarray(scale, np.float64)
    return (np.asarray(x, np.float64) @ w.T).astype(np.float64)


# ------------------------------------------------------------------ the reference's own CPU code (oracle/_ref)
# Built by `make -C oracle ref` from the reference sources where /root/reference is mounted; absent elsewhere.
_ref = None


@dataclass
class NibPage:
    """One sealed int4 nibble page (host arrays), the cf_device_page_descriptor payload."""
    k_payload: np.ndarray
    v_payload: np.ndarray
    k_scales: np.ndarray
    v_scales: np.ndarray
    token_begin: int
    token_count: int


def nib_seal(x: np.ndarray, block_size: int):
    """Seal one fp32 stream (reference src/cuda/device_kv_seal_attention.cu:72-113). Returns (payload u8, scales
    f32, saturated) or raises ValueError naming the NaN/Inf counts."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    nb = (x.size + block_size - 1) // block_size
    payload = np.zeros((x.size + 1) // 2, np.uint8)
    scales = np.zeros(nb, np.float32)
    sat, nan, inf = (np.zeros(1, np.uint64) for _ in range(3))
    rc = lib().or_nib_seal(_ptr(x), x.size, block_size, _ptr(payload), _ptr(scales), _ptr(sat), _ptr(nan), _ptr(inf))
    if rc != 0:
        raise ValueError(f"page rejected: {int(nan[0])} NaN, {int(inf[0])} Inf")
    return payload, scales, int(sat[0])


def nib_seal_page(k: np.ndarray, v: np.ndarray, token_begin: int, block_size: int) -> NibPage:
    """Seal K and V [tokens, kv_heads, head_dim] fp32 into one page."""
    kp, ks, _ = nib_seal(k, block_size)
    vp, vs, _ = nib_seal(v, block_size)
    return NibPage(kp, vp, ks, vs, token_begin, int(k.shape[0]))


def nib_dequant(payload: np.ndarray, scales: np.ndarray, values: int, block_size: int) -> np.ndarray:
    """(symbol - 8) * scale[i // block] for i < values (float64)."""
    sym = np.empty(values, np.int64)
    sym[0::2] = payload[: (values + 1) // 2] & 0x0F
    sym[1::2] = payload[: values // 2] >> 4
    return (sym - 8).astype(np.float64) * scales[np.arange(values) // block_size].astype(np.float64)


def nib_attention(pages: list, block_size: int, q: np.ndarray, query_begin: int, kv_heads: int, gqa: int,
                  scale: float, window: int = 0, active_k=None, active_v=None, active_begin: int = 0) -> np.ndarray:
    """Attention of q [q_tokens, kv_heads * gqa, head_dim] over sealed pages then the fp32 active page
    (reference device_kv_seal_attention.cu:116-187), float64 accumulation; returns float32."""
    q = np.ascontiguousarray(q, np.float32)
    qt, _, D = q.shape
    out = np.zeros_like(q)
    arr = lambda xs, t: (t * len(xs))(*[x.ctypes.data for x in xs]) if xs else None
    keep = [p.k_payload for p in pages] + [p.v_payload for p in pages]
    tb = np.array([p.token_begin for p in pages] or [0], np.uint32)
    tc = np.array([p.token_count for p in pages] or [0], np.uint32)
    ak = None if active_k is None else np.ascontiguousarray(active_k, np.float32)
    av = None if active_v is None else np.ascontiguousarray(active_v, np.float32)
    acount = 0 if ak is None else int(ak.shape[0])
    lib().or_nib_attention(len(pages), arr([p.k_payload for p in pages], C.c_void_p),
                           arr([p.v_payload for p in pages], C.c_void_p), arr([p.k_scales for p in pages], C.c_void_p),
                           arr([p.v_scales for p in pages], C.c_void_p), _ptr(tb), _ptr(tc), block_size, _ptr(ak),
                           _ptr(av), active_begin, acount, _ptr(q), qt, query_begin, kv_heads, gqa, D, scale, window,
                           _ptr(out))
    del keep
    return out


@dataclass
class RtPage:
    """One page of the batched attention runtime (cf_attention_execute_async, production_attention.h): K and V
    [tokens][kv_heads][head_dim] as two's-complement int4 nibbles, two per byte with the even index in the low
    nibble, one scale per block of `block_size` values of a (token, KV head) row. A payload or scale of None is a
    page with a NULL pointer."""
    k_payload: np.ndarray | None
    v_payload: np.ndarray | None
    k_scales: np.ndarray | None
    v_scales: np.ndarray | None
    token_begin: int
    token_count: int
    head_dim: int
    block_size: int


def rt_quantize(x: np.ndarray, block_size: int):
    """Test-fixture encoder of the runtime's page format (the reference has none: its seal engine writes offset-8
    symbols): x [tokens, kv_heads, head_dim] -> (payload u8, scales f32). Per row block: scale = absmax / 7 (1 for
    an all-zero block), value = clamp(rint(x / scale), -8, 7) stored as its low 4 bits."""
    x = np.ascontiguousarray(x, np.float32)
    T, H, D = x.shape
    bpr = (D + block_size - 1) // block_size
    pad = np.zeros((T, H, bpr * block_size), np.float32)
    pad[:, :, :D] = x
    blocks = pad.reshape(T, H, bpr, block_size)
    amax = np.abs(blocks).max(axis=3)
    scales = np.where(amax > 0, amax / np.float32(7.0), np.float32(1.0)).astype(np.float32)
    q = np.clip(np.rint(blocks / scales[..., None]), -8, 7).astype(np.int64)
    nib = (q.reshape(T, H, bpr * block_size)[:, :, :D].ravel() & 15).astype(np.uint8)
    if nib.size % 2:
        nib = np.concatenate([nib, np.zeros(1, np.uint8)])
    payload = (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8)
    return payload, scales.ravel()


def rt_dequant(payload: np.ndarray, scales: np.ndarray, tokens: int, kv_heads: int, head_dim: int,
               page_head_dim: int, block_size: int) -> np.ndarray:
    """[tokens, kv_heads, head_dim] float64 of one runtime page stream: reference production_attention.cu:41-46
    (two's-complement nibble times its scale) with the scale index of :85-86 / :106-107
    ((token * kv_heads + kv_head) * ceil(page head_dim / block_size) + d / block_size)."""
    n = tokens * kv_heads * head_dim
    i = np.arange(n)
    byte = payload[i >> 1].astype(np.int64)
    nib = np.where(i & 1, byte >> 4, byte & 15)
    val = np.where(nib >= 8, nib - 16, nib)
    bph = (page_head_dim + block_size - 1) // block_size
    sidx = (i // head_dim) * bph + (i % head_dim) // block_size
    return (val * scales[sidx].astype(np.float64)).reshape(tokens, kv_heads, head_dim)


def rt_attention_f64(q: np.ndarray, kv_heads: int, gqa: int, query_token_begin: int, window: int, scale: float,
                     pages: list, active_k=None, active_v=None, active_begin: int = 0) -> np.ndarray:
    """One batch item of cf_attention_execute_async in float64: reference production_attention.cu:59-139. q is
    [q_heads, head_dim] (the query values as the kernel reads them); query head h reads KV head h // gqa; pages in
    order, then the active tail ([n, kv_heads, head_dim] fp32); a page with a NULL pointer is skipped (:81); a
    position p is attended unless window > 0 and p + window < query_token_begin (:83, :116: no causal bound; the
    sum is taken without 32-bit wraparound); score = q.k * scale; a head with nothing attended is zeros."""
    q = np.asarray(q, np.float64)
    QH, D = q.shape
    ks, vs, pos = [], [], []
    for pg in pages:
        if pg.k_payload is None or pg.v_payload is None or pg.k_scales is None or pg.v_scales is None:
            continue
        ks.append(rt_dequant(pg.k_payload, pg.k_scales, pg.token_count, kv_heads, D, pg.head_dim, pg.block_size))
        vs.append(rt_dequant(pg.v_payload, pg.v_scales, pg.token_count, kv_heads, D, pg.head_dim, pg.block_size))
        pos.append(pg.token_begin + np.arange(pg.token_count, dtype=np.int64))
    if active_k is not None and len(active_k):
        ks.append(np.asarray(active_k, np.float64).reshape(-1, kv_heads, D))
        vs.append(np.asarray(active_v, np.float64).reshape(-1, kv_heads, D))
        pos.append(active_begin + np.arange(len(active_k), dtype=np.int64))
    out = np.zeros((QH, D))
    if not ks:
        return out
    K, V, P = np.concatenate(ks), np.concatenate(vs), np.concatenate(pos)
    vis = np.ones(len(P), bool) if window == 0 else P + window >= query_token_begin
    if not vis.any():
        return out
    for h in range(QH):
        kv = h // gqa
        s = (K[vis, kv, :] @ q[h]) * scale
        w = np.exp(s - s.max())
        out[h] = (w @ V[vis, kv, :]) / w.sum()
    return out


def ref_lib() -> C.CDLL | None:
    """oracle/_ref/libcfref.so (reference kv_gpu_fixture/kv_reference/kv_runtime behind ref_shim.cpp) or None."""
    global _ref
    path = os.path.join(REF_DIR, "libcfref.so")
    if _ref is None and os.path.exists(path):
        _ref = C.CDLL(path)
        _ref.cfref_fixture_page.restype = C.c_int
        _ref.cfref_fixture_page.argtypes = [C.c_int, P, P, U32, U32, U32, U32, U32] + [P] * 8 + [U32, P, U32, P]
        _ref.cfref_seal_dequant.restype = C.c_int
        _ref.cfref_seal_dequant.argtypes = [P, P, U32, U32, U32, U32, P, P]
        _ref.cfref_paged_attention.restype = C.c_int
        _ref.cfref_paged_attention.argtypes = [P, U32, U32, U32, U32, U32, C.c_float, U32, P, P, P, P, P, P, P, P,
                                               U32, U32, P]
    return _ref


def ref_build_index() -> str | None:
    """Path of oracle/_ref/build_index (reference tools/build_index.cpp compiled from its source) or None."""
    path = os.path.join(REF_DIR, "build_index")
    return path if os.path.exists(path) else None


def ref_fixture_page(bits: int, k: np.ndarray, v: np.ndarray, kv_head: int = 0, block: int = 64):
    """reference gpu_fixture::encode_int{4,8}_page -> dict of its words, scales, dequantised values, offsets."""
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    T, D = k.shape
    cap = (T * D * 8 + 31) // 32 + 4
    capb = T * D // block + 4
    out = dict(kw=np.zeros(cap, np.uint32), vw=np.zeros(cap, np.uint32), ks=np.zeros(D, np.float32),
               vs=np.zeros(T, np.float32), kdeq=np.zeros((T, D), np.float32), vdeq=np.zeros((T, D), np.float32),
               kboff=np.zeros(capb, np.int32), vboff=np.zeros(capb, np.int32))
    lut = np.zeros(256, np.int32)
    cnt = np.zeros(6, np.uint32)
    rc = ref_lib().cfref_fixture_page(bits, _ptr(k), _ptr(v), T, D, kv_head, block, cap,
                                      *[_ptr(out[n]) for n in ["kw", "vw", "ks", "vs", "kdeq", "vdeq", "kboff",
                                                               "vboff"]], capb, _ptr(lut), 256, _ptr(cnt))
    if rc != 0:
        raise ValueError("reference encoder rejected the page")
    out["kw"], out["vw"] = out["kw"][:cnt[0]], out["vw"][:cnt[1]]
    out["kboff"], out["vboff"] = out["kboff"][:cnt[2]], out["vboff"][:cnt[3]]
    out["lut"], out["zero_point"] = lut[:cnt[4]], int(cnt[5])
    return out


def ref_seal_dequant(k: np.ndarray, v: np.ndarray, token_begin: int, kv_head: int):
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    T, D = k.shape
    kd, vd = np.zeros((T, D), np.float32), np.zeros((T, D), np.float32)
    if ref_lib().cfref_seal_dequant(_ptr(k), _ptr(v), token_begin, T, kv_head, D, _ptr(kd), _ptr(vd)) != 0:
        raise ValueError("reference seal rejected the page")
    return kd, vd


def ref_paged_attention(q, q_heads, kv_heads, D, query_token, window, scale, pages, tail=None):
    """reference::paged_attention over int4 pages sealed from raw (kv_head, token_begin, K, V) and an optional
    (token_begin, K [n, kvh, D], V [n, kvh, D]) tail. Returns out [q_heads, D], or None if the reference threw."""
    q = np.ascontiguousarray(q, np.float32)
    n = len(pages)
    kvh = np.array([p[0] for p in pages], np.uint32)
    tok0 = np.array([p[1] for p in pages], np.uint32)
    ntok = np.array([p[2].shape[0] for p in pages], np.uint32)
    off = np.zeros(max(n, 1), np.uint64)
    if n:
        off[1:n] = np.cumsum(ntok[:-1])
    K = np.ascontiguousarray(np.concatenate([p[2] for p in pages]) if n else np.zeros((1, D)), np.float32)
    V = np.ascontiguousarray(np.concatenate([p[3] for p in pages]) if n else np.zeros((1, D)), np.float32)
    t0, tk, tv, tn = 0, None, None, 0
    if tail is not None:
        t0, tk, tv = tail
        tk, tv = np.ascontiguousarray(tk, np.float32), np.ascontiguousarray(tv, np.float32)
        tn = tk.shape[0]
    out = np.zeros((q_heads, D), np.float32)
    rc = ref_lib().cfref_paged_attention(_ptr(q), q_heads, kv_heads, D, query_token, window, scale, n, _ptr(kvh),
                                         _ptr(tok0), _ptr(ntok), _ptr(off), _ptr(K), _ptr(V), _ptr(tk), _ptr(tv),
                                         t0, tn, _ptr(out))
    return out if rc == 0 else None
