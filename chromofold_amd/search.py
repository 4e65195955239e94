"""Host-side mirror of the compressed-domain search interface (RRR wavelet matrix, FM-index).

Mirrors the reference's C ABI `include/chromofold/chromofold_search.h` (cf_rrrw_access_async, cf_rrrw_rank_async,
cf_fm_count_async, cf_fm_ranges_async, cf_fm_locate_async): device-resident index arrays are held as torch tensors
(plumbing for HBM allocation and streams); every query runs through libchromofold.so. Errors surface as CfError
carrying the cf_status the C entry point returned.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np
import torch

from . import _abi as A


def _dev(a: np.ndarray, device) -> torch.Tensor:
    """Upload a host array bit-for-bit (unsigned types ride in same-width signed torch dtypes)."""
    a = np.ascontiguousarray(a)
    view = {np.dtype(np.uint32): np.int32, np.dtype(np.uint16): np.int16, np.dtype(np.uint8): np.uint8}
    if a.dtype in view:
        a = a.view(view[a.dtype])
    return torch.from_numpy(a).to(device)


def _ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def stream_ptr(stream: torch.cuda.Stream | None = None):
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


# binom[16*16] / width[16]: fixed by the RRR format (T = 15); built here the same way every reference caller does
# (reference benchmarks/rrr_wavelet.cu:95-106).
def rrr_tables() -> tuple[np.ndarray, np.ndarray]:
    from math import comb
    binom = np.array([[comb(n, k) if k <= n else 0 for k in range(16)] for n in range(16)], np.int32).ravel()
    width = np.array([(int(comb(15, k) - 1).bit_length() if comb(15, k) > 1 else 0) for k in range(16)], np.int32)
    return binom, width


@dataclass
class RrrWaveletIndex:
    """Device-resident RRR wavelet matrix (the cf_rrrw_view arrays)."""
    bits: int
    cwords: int
    nsb: int
    na: int
    tensors: dict
    lines: "torch.Tensor | None" = None  # the derived line layout, built on first use (build_lines)
    quads: "torch.Tensor | None" = None  # the derived 4-ary layout (build_quads), over quads_n symbols
    quads_n: int = 0

    @classmethod
    def from_host(cls, arrays, device="cuda") -> "RrrWaveletIndex":
        """`arrays` has attributes or keys classes, offsets, rank_a, rank_d, off_a, off_d, offbase, zeros, bits,
        cwords, nsb, na (the .cfrw payload)."""
        get = (lambda k: arrays[k]) if isinstance(arrays, dict) else (lambda k: getattr(arrays, k))
        binom, width = rrr_tables()
        t = {k: _dev(np.asarray(get(k)), device) for k in
             ["classes", "offsets", "rank_a", "rank_d", "off_a", "off_d", "offbase", "zeros"]}
        t["binom"] = _dev(binom, device)
        t["width"] = _dev(width, device)
        return cls(int(get("bits")), int(get("cwords")), int(get("nsb")), int(get("na")), t)

    def view(self) -> A.cf_rrrw_view:
        t = self.tensors
        return A.cf_rrrw_view(_ptr(t["classes"]), _ptr(t["offsets"]), _ptr(t["rank_a"]), _ptr(t["rank_d"]),
                              _ptr(t["off_a"]), _ptr(t["off_d"]), _ptr(t["offbase"]), _ptr(t["zeros"]),
                              _ptr(t["width"]), _ptr(t["binom"]), self.bits, self.cwords, self.nsb, self.na)

    def device_bytes(self) -> int:
        return sum(v.numel() * v.element_size() for k, v in self.tensors.items() if k not in ("binom", "width"))

    def access_into(self, positions: torch.Tensor, out: torch.Tensor, stream=None) -> None:
        st = A.lib().cf_rrrw_access_async(self.view(), _ptr(positions), _ptr(out), positions.numel(),
                                          stream_ptr(stream))
        A.check(st, "cf_rrrw_access_async")

    def rank_into(self, symbols: torch.Tensor, positions: torch.Tensor, out: torch.Tensor, stream=None) -> None:
        st = A.lib().cf_rrrw_rank_async(self.view(), _ptr(symbols), _ptr(positions), _ptr(out),
                                        positions.numel(), stream_ptr(stream))
        A.check(st, "cf_rrrw_rank_async")

    def access(self, positions: torch.Tensor) -> torch.Tensor:
        out = torch.empty_like(positions, dtype=torch.int32)
        self.access_into(positions, out)
        return out

    # ---- the derived line layout (cf_rrrw_lines_*): same results, one 64-byte line per level
    def build_lines(self, stream=None) -> torch.Tensor:
        """Builds (once) and returns the line layout of this matrix (a uint8 device tensor)."""
        if self.lines is None:
            v = self.view()
            nb = int(A.lib().cf_rrrw_lines_bytes(v))
            if nb == 0:
                raise A.CfError(A.CF_ERR_UNSUPPORTED, "cf_rrrw_lines_bytes")
            lines = torch.empty(nb, dtype=torch.uint8, device=self.tensors["classes"].device)
            A.check(A.lib().cf_rrrw_lines_build_async(v, _ptr(lines), nb, stream_ptr(stream)),
                    "cf_rrrw_lines_build_async")
            self.lines = lines
        return self.lines

    def access_lines_into(self, positions: torch.Tensor, out: torch.Tensor, stream=None) -> None:
        A.check(A.lib().cf_rrrw_access_lines_async(self.view(), _ptr(self.build_lines(stream)), _ptr(positions),
                                                   _ptr(out), positions.numel(), stream_ptr(stream)),
                "cf_rrrw_access_lines_async")

    def rank_lines_into(self, symbols: torch.Tensor, positions: torch.Tensor, out: torch.Tensor, stream=None) -> None:
        A.check(A.lib().cf_rrrw_rank_lines_async(self.view(), _ptr(self.build_lines(stream)), _ptr(symbols),
                                                 _ptr(positions), _ptr(out), positions.numel(), stream_ptr(stream)),
                "cf_rrrw_rank_lines_async")

    # ---- the derived 4-ary layout (cf_rrrw_quads_*): same results, ceil(bits / 2) records per query
    def build_quads(self, n: int, stream=None) -> torch.Tensor:
        """Builds (once) the 4-ary layout of the matrix's n symbols."""
        if self.quads is None or self.quads_n != n:
            v = self.view()
            L = A.lib()
            nb, nw = int(L.cf_rrrw_quads_bytes(v, n)), int(L.cf_rrrw_quads_workspace_bytes(v, n))
            if nb == 0:
                raise A.CfError(A.CF_ERR_UNSUPPORTED, "cf_rrrw_quads_bytes")
            dev = self.tensors["classes"].device
            quads = torch.empty(nb, dtype=torch.uint8, device=dev)
            ws = torch.empty(nw, dtype=torch.uint8, device=dev)
            A.check(L.cf_rrrw_quads_build_async(v, n, _ptr(quads), nb, _ptr(ws), nw, stream_ptr(stream)),
                    "cf_rrrw_quads_build_async")
            torch.cuda.current_stream(dev).synchronize() if stream is None else stream.synchronize()  # ws is freed
            self.quads, self.quads_n = quads, n
        return self.quads

    def access_quads_into(self, positions: torch.Tensor, out: torch.Tensor, stream=None) -> None:
        A.check(A.lib().cf_rrrw_access_quads_async(self.view(), self.quads_n, _ptr(self.quads), _ptr(positions),
                                                   _ptr(out), positions.numel(), stream_ptr(stream)),
                "cf_rrrw_access_quads_async")

    def rank_quads_into(self, symbols: torch.Tensor, positions: torch.Tensor, out: torch.Tensor, stream=None) -> None:
        A.check(A.lib().cf_rrrw_rank_quads_async(self.view(), self.quads_n, _ptr(self.quads), _ptr(symbols),
                                                 _ptr(positions), _ptr(out), positions.numel(), stream_ptr(stream)),
                "cf_rrrw_rank_quads_async")

    def gather_fused_lines_into(self, emb: torch.Tensor, positions: torch.Tensor, out: torch.Tensor,
                                stream=None) -> None:
        """out[t, :] = emb[access(positions[t]), :] (cf_sparse_gather_fused_lines_async)."""
        A.check(A.lib().cf_sparse_gather_fused_lines_async(self.view(), _ptr(self.build_lines(stream)), _ptr(emb),
                                                           emb.shape[1], _ptr(positions), _ptr(out), positions.numel(),
                                                           stream_ptr(stream)),
                "cf_sparse_gather_fused_lines_async")

    def gather_fused_quads_into(self, emb: torch.Tensor, positions: torch.Tensor, out: torch.Tensor,
                                stream=None) -> None:
        """out[t, :] = emb[access(positions[t]), :] over the 4-ary layout (cf_sparse_gather_fused_quads_async);
        build_quads(n) first."""
        if self.quads is None:
            raise A.CfError(A.CF_ERR_INVALID_ARGUMENT, "cf_sparse_gather_fused_quads_async: build_quads(n) first")
        A.check(A.lib().cf_sparse_gather_fused_quads_async(self.view(), self.quads_n, _ptr(self.quads), _ptr(emb),
                                                           emb.shape[1], _ptr(positions), _ptr(out), positions.numel(),
                                                           stream_ptr(stream)),
                "cf_sparse_gather_fused_quads_async")

    def rank(self, symbols: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        out = torch.empty_like(positions, dtype=torch.int32)
        self.rank_into(symbols, positions, out)
        return out


def to_u32(t: torch.Tensor) -> np.ndarray:
    """Device int32 tensor holding u32 bits -> host uint32 array."""
    return t.cpu().numpy().view(np.uint32)


def u32_dev(a, device="cuda") -> torch.Tensor:
    return _dev(np.asarray(a, dtype=np.uint32), device)


A.declare("cf_suffix_array_workspace_bytes", A.U64, [A.I32, A.I32])
A.declare("cf_suffix_array", A.I32, [A.P, A.I32, A.I32, A.P, A.P, A.U64, A.P])


@dataclass
class FmIndex:
    """Device-resident FM-index (the cf_fm_view arrays): RRR wavelet of the BWT + C table + sampled SA."""
    w: RrrWaveletIndex
    sigma: int
    n: int
    sa_sample: int
    tensors: dict
    lines: "torch.Tensor | None" = None  # the derived line layout, built on first use (build_lines)
    quads: "torch.Tensor | None" = None  # the derived 4-ary layout, built on first use (build_quads)

    @classmethod
    def from_host(cls, arrays, device="cuda") -> "FmIndex":
        """`arrays` has the .cffm payload: an RRR wavelet (attribute `w` or the wavelet keys) plus C, mwords, msb,
        sval, sigma, n, sa_sample."""
        get = (lambda k: arrays[k]) if isinstance(arrays, dict) else (lambda k: getattr(arrays, k))
        w = RrrWaveletIndex.from_host(arrays if isinstance(arrays, dict) else arrays.w, device)
        t = {k: _dev(np.asarray(get(k)), device) for k in ["C", "mwords", "msb", "sval"]}
        return cls(w, int(get("sigma")), int(get("n")), int(get("sa_sample")), t)

    def view(self) -> A.cf_fm_view:
        t = self.tensors
        return A.cf_fm_view(self.w.view(), _ptr(t["C"]), _ptr(t["mwords"]), _ptr(t["msb"]), _ptr(t["sval"]),
                            self.sigma, self.n, self.sa_sample)

    def count(self, pat: torch.Tensor, pstart: torch.Tensor, plen: torch.Tensor, stream=None) -> torch.Tensor:
        out = torch.empty(pstart.numel(), dtype=torch.int32, device=pstart.device)
        A.check(A.lib().cf_fm_count_async(self.view(), _ptr(pat), _ptr(pstart), _ptr(plen), _ptr(out),
                                          pstart.numel(), stream_ptr(stream)), "cf_fm_count_async")
        return out

    def ranges(self, pat, pstart, plen, stream=None):
        lo = torch.empty(pstart.numel(), dtype=torch.int32, device=pstart.device)
        hi = torch.empty_like(lo)
        A.check(A.lib().cf_fm_ranges_async(self.view(), _ptr(pat), _ptr(pstart), _ptr(plen), _ptr(lo), _ptr(hi),
                                           pstart.numel(), stream_ptr(stream)), "cf_fm_ranges_async")
        return lo, hi

    def locate(self, rows: torch.Tensor, out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
        out = torch.empty_like(rows, dtype=torch.int32) if out is None else out
        A.check(A.lib().cf_fm_locate_async(self.view(), _ptr(rows), _ptr(out), rows.numel(), stream_ptr(stream)),
                "cf_fm_locate_async")
        return out

    # ---- the derived line layout (cf_fm_lines_*): same results, one 64-byte line per rank1
    def build_lines(self, stream=None) -> torch.Tensor:
        """Builds (once) and returns the line layout of this index (a uint8 device tensor)."""
        if self.lines is None:
            v = self.view()
            nb = int(A.lib().cf_fm_lines_bytes(v))
            if nb == 0:
                raise A.CfError(A.CF_ERR_INVALID_ARGUMENT, "cf_fm_lines_bytes")
            lines = torch.empty(nb, dtype=torch.uint8, device=self.tensors["C"].device)
            A.check(A.lib().cf_fm_lines_build_async(v, _ptr(lines), nb, stream_ptr(stream)), "cf_fm_lines_build_async")
            self.lines = lines
        return self.lines

    def count_lines(self, pat, pstart, plen, out=None, stream=None) -> torch.Tensor:
        out = torch.empty(pstart.numel(), dtype=torch.int32, device=pstart.device) if out is None else out
        A.check(A.lib().cf_fm_count_lines_async(self.view(), _ptr(self.build_lines(stream)), _ptr(pat), _ptr(pstart),
                                                _ptr(plen), _ptr(out), pstart.numel(), stream_ptr(stream)),
                "cf_fm_count_lines_async")
        return out

    def ranges_lines(self, pat, pstart, plen, stream=None):
        lo = torch.empty(pstart.numel(), dtype=torch.int32, device=pstart.device)
        hi = torch.empty_like(lo)
        A.check(A.lib().cf_fm_ranges_lines_async(self.view(), _ptr(self.build_lines(stream)), _ptr(pat), _ptr(pstart),
                                                 _ptr(plen), _ptr(lo), _ptr(hi), pstart.numel(), stream_ptr(stream)),
                "cf_fm_ranges_lines_async")
        return lo, hi

    def locate_lines(self, rows: torch.Tensor, out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
        out = torch.empty_like(rows, dtype=torch.int32) if out is None else out
        A.check(A.lib().cf_fm_locate_lines_async(self.view(), _ptr(self.build_lines(stream)), _ptr(rows), _ptr(out),
                                                 rows.numel(), stream_ptr(stream)), "cf_fm_locate_lines_async")
        return out

    # ---- the derived 4-ary layout (cf_fm_quads_*): same results, ceil(bits / 2) records per walk
    def build_quads(self, stream=None) -> torch.Tensor:
        if self.quads is None:
            v = self.view()
            L = A.lib()
            nb, nw = int(L.cf_fm_quads_bytes(v)), int(L.cf_fm_quads_workspace_bytes(v))
            if nb == 0:
                raise A.CfError(A.CF_ERR_INVALID_ARGUMENT, "cf_fm_quads_bytes")
            dev = self.tensors["C"].device
            quads = torch.empty(nb, dtype=torch.uint8, device=dev)
            ws = torch.empty(nw, dtype=torch.uint8, device=dev)
            A.check(L.cf_fm_quads_build_async(v, _ptr(quads), nb, _ptr(ws), nw, stream_ptr(stream)),
                    "cf_fm_quads_build_async")
            torch.cuda.current_stream(dev).synchronize() if stream is None else stream.synchronize()  # ws is freed
            self.quads = quads
        return self.quads

    def count_quads(self, pat, pstart, plen, out=None, stream=None) -> torch.Tensor:
        out = torch.empty(pstart.numel(), dtype=torch.int32, device=pstart.device) if out is None else out
        A.check(A.lib().cf_fm_count_quads_async(self.view(), _ptr(self.build_quads(stream)), _ptr(pat), _ptr(pstart),
                                                _ptr(plen), _ptr(out), pstart.numel(), stream_ptr(stream)),
                "cf_fm_count_quads_async")
        return out

    def ranges_quads(self, pat, pstart, plen, stream=None):
        lo = torch.empty(pstart.numel(), dtype=torch.int32, device=pstart.device)
        hi = torch.empty_like(lo)
        A.check(A.lib().cf_fm_ranges_quads_async(self.view(), _ptr(self.build_quads(stream)), _ptr(pat), _ptr(pstart),
                                                 _ptr(plen), _ptr(lo), _ptr(hi), pstart.numel(), stream_ptr(stream)),
                "cf_fm_ranges_quads_async")
        return lo, hi

    def locate_quads(self, rows: torch.Tensor, out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
        out = torch.empty_like(rows, dtype=torch.int32) if out is None else out
        A.check(A.lib().cf_fm_locate_quads_async(self.view(), _ptr(self.build_quads(stream)), _ptr(rows), _ptr(out),
                                                 rows.numel(), stream_ptr(stream)), "cf_fm_locate_quads_async")
        return out


def gpu_suffix_array(s: torch.Tensor, stream=None) -> torch.Tensor:
    """Suffix array of the int32 device text `s` (sentinel-terminated) via cf_suffix_array."""
    n = s.numel()
    mx = int(s.max().item())
    wsb = int(A.lib().cf_suffix_array_workspace_bytes(n, mx))
    if wsb == 0:
        raise A.CfError(A.CF_ERR_UNSUPPORTED, "cf_suffix_array_workspace_bytes")
    ws = torch.empty(wsb, dtype=torch.uint8, device=s.device)
    sa = torch.empty(n, dtype=torch.int32, device=s.device)
    A.check(A.lib().cf_suffix_array(_ptr(s), n, mx, _ptr(sa), _ptr(ws), wsb, stream_ptr(stream)), "cf_suffix_array")
    return sa


# ------------------------------------------------------------------------------------------------ on-device builds
class cf_rrrw_layout(C.Structure):
    _fields_ = [("n", A.U64), ("bits", A.U32), ("nblocks", A.U32), ("cwords", A.U32), ("nsb", A.U32), ("na", A.U32),
                ("owords", A.U32), ("rrr_bytes", A.U64), ("level_owords", A.U32 * 32)]


class cf_rrrw_arrays(C.Structure):
    _fields_ = [(k, A.P) for k in ("classes", "offsets", "rank_a", "rank_d", "off_a", "off_d", "offbase", "zeros")]


A.declare("cf_rrrw_build_workspace_bytes", A.U64, [A.U64, A.U32])
A.declare("cf_rrrw_build", A.I32, [A.P, A.U64, A.U32, A.P, A.U64, C.POINTER(cf_rrrw_layout), A.P])
A.declare("cf_rrrw_build_copy", A.I32, [A.P, C.POINTER(cf_rrrw_layout), C.POINTER(cf_rrrw_arrays), A.P])
A.declare("cf_fm_build_workspace_bytes", A.U64, [A.I32, A.I32])
A.declare("cf_rrrw_lines_bytes", A.U64, [A.cf_rrrw_view])
A.declare("cf_rrrw_lines_build_async", A.I32, [A.cf_rrrw_view, A.P, A.U64, A.P])
A.declare("cf_rrrw_access_lines_async", A.I32, [A.cf_rrrw_view, A.P, A.P, A.P, A.SZ, A.P])
A.declare("cf_rrrw_rank_lines_async", A.I32, [A.cf_rrrw_view, A.P, A.P, A.P, A.P, A.SZ, A.P])
A.declare("cf_fm_quads_bytes", A.U64, [A.cf_fm_view])
A.declare("cf_fm_quads_workspace_bytes", A.U64, [A.cf_fm_view])
A.declare("cf_fm_quads_build_async", A.I32, [A.cf_fm_view, A.P, A.U64, A.P, A.U64, A.P])
A.declare("cf_fm_count_quads_async", A.I32, [A.cf_fm_view, A.P, A.P, A.P, A.P, A.P, A.SZ, A.P])
A.declare("cf_fm_ranges_quads_async", A.I32, [A.cf_fm_view, A.P, A.P, A.P, A.P, A.P, A.P, A.SZ, A.P])
A.declare("cf_fm_locate_quads_async", A.I32, [A.cf_fm_view, A.P, A.P, A.P, A.SZ, A.P])
A.declare("cf_rrrw_quads_bytes", A.U64, [A.cf_rrrw_view, A.U64])
A.declare("cf_rrrw_quads_workspace_bytes", A.U64, [A.cf_rrrw_view, A.U64])
A.declare("cf_rrrw_quads_build_async", A.I32, [A.cf_rrrw_view, A.U64, A.P, A.U64, A.P, A.U64, A.P])
A.declare("cf_rrrw_access_quads_async", A.I32, [A.cf_rrrw_view, A.U64, A.P, A.P, A.P, A.SZ, A.P])
A.declare("cf_rrrw_rank_quads_async", A.I32, [A.cf_rrrw_view, A.U64, A.P, A.P, A.P, A.P, A.SZ, A.P])
A.declare("cf_sparse_gather_fused_lines_async", A.I32, [A.cf_rrrw_view, A.P, A.P, C.c_int, A.P, A.P, A.SZ, A.P])
A.declare("cf_sparse_gather_fused_quads_async", A.I32,
          [A.cf_rrrw_view, A.U64, A.P, A.P, C.c_int, A.P, A.P, A.SZ, A.P])
A.declare("cf_fm_lines_bytes", A.U64, [A.cf_fm_view])
A.declare("cf_fm_lines_build_async", A.I32, [A.cf_fm_view, A.P, A.U64, A.P])
A.declare("cf_fm_count_lines_async", A.I32, [A.cf_fm_view, A.P, A.P, A.P, A.P, A.P, A.SZ, A.P])
A.declare("cf_fm_ranges_lines_async", A.I32, [A.cf_fm_view, A.P, A.P, A.P, A.P, A.P, A.P, A.SZ, A.P])
A.declare("cf_fm_locate_lines_async", A.I32, [A.cf_fm_view, A.P, A.P, A.P, A.SZ, A.P])
A.declare("cf_fm_build_aux", A.I32, [A.P, A.P, A.I32, A.I32, A.I32, A.P, A.P, A.P, A.P, A.P, C.POINTER(C.c_int32),
                                     A.P, A.U64, A.P])


def build_rrrw(tokens: torch.Tensor, bits: int, stream=None) -> tuple[RrrWaveletIndex, cf_rrrw_layout]:
    """RRR wavelet matrix of the device token array (int32 holding u32 values < 2^bits), built on the GPU."""
    n = tokens.numel()
    dev = tokens.device
    L = A.lib()
    wsb = int(L.cf_rrrw_build_workspace_bytes(n, bits))
    if wsb == 0:
        raise A.CfError(A.CF_ERR_UNSUPPORTED, "cf_rrrw_build_workspace_bytes")
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    lay = cf_rrrw_layout()
    s = stream_ptr(stream)
    A.check(L.cf_rrrw_build(_ptr(tokens), n, bits, _ptr(ws), wsb, C.byref(lay), s), "cf_rrrw_build")
    i32 = dict(dtype=torch.int32, device=dev)
    t = {"classes": torch.empty(bits * lay.cwords, **i32), "offsets": torch.empty(lay.owords, **i32),
         "rank_a": torch.empty(bits * lay.na, **i32), "rank_d": torch.empty(bits * (lay.nsb + 1), dtype=torch.int16,
                                                                            device=dev),
         "off_a": torch.empty(bits * lay.na, **i32), "off_d": torch.empty(bits * (lay.nsb + 1), dtype=torch.int16,
                                                                          device=dev),
         "offbase": torch.empty(bits, **i32), "zeros": torch.empty(bits, **i32)}
    arr = cf_rrrw_arrays(*[_ptr(t[k]) for k in ("classes", "offsets", "rank_a", "rank_d", "off_a", "off_d", "offbase",
                                                 "zeros")])
    A.check(L.cf_rrrw_build_copy(_ptr(ws), C.byref(lay), C.byref(arr), s), "cf_rrrw_build_copy")
    binom, width = rrr_tables()
    t["binom"] = _dev(binom, dev)
    t["width"] = _dev(width, dev)
    (stream if stream is not None else torch.cuda.current_stream(dev)).synchronize()  # copies done before ws goes
    return RrrWaveletIndex(bits, int(lay.cwords), int(lay.nsb), int(lay.na), t), lay


def build_fm(tokens: torch.Tensor, sa_sample: int, stream=None) -> tuple[FmIndex, dict]:
    """Full on-device FM-index build of a token array (int32 device tensor, values >= 0): text s = (tokens + 1) ++
    [0], GPU suffix array, BWT, RRR wavelet of the BWT, C / mark plane / msb / sampled SA. Returns the index and the
    intermediate device arrays (s, sa, bwt) and build timings."""
    import time
    dev = tokens.device
    t0 = time.perf_counter()
    s = torch.empty(tokens.numel() + 1, dtype=torch.int32, device=dev)
    s[:-1] = tokens + 1
    s[-1] = 0
    n = s.numel()
    sa = gpu_suffix_array(s, stream)
    torch.cuda.synchronize(dev)
    t_sa = time.perf_counter() - t0
    sigma = int(s.max().item()) + 1
    bits = max(1, (sigma - 1).bit_length())
    nw = (n + 31) // 32
    nb = (nw + 7) // 8
    bwt = torch.empty(n, dtype=torch.int32, device=dev)
    Ct = torch.empty(sigma, dtype=torch.int32, device=dev)
    mw = torch.empty(nw, dtype=torch.int32, device=dev)
    msb = torch.empty(nb + 1, dtype=torch.int32, device=dev)
    sval = torch.empty(n // sa_sample + 2, dtype=torch.int32, device=dev)
    cnt = C.c_int32(0)
    L = A.lib()
    wsb = int(L.cf_fm_build_workspace_bytes(n, sigma))
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    A.check(L.cf_fm_build_aux(_ptr(s), _ptr(sa), n, sigma, sa_sample, _ptr(bwt), _ptr(Ct), _ptr(mw), _ptr(msb),
                              _ptr(sval), C.byref(cnt), _ptr(ws), wsb, stream_ptr(stream)), "cf_fm_build_aux")
    w, lay = build_rrrw(bwt, bits, stream)
    torch.cuda.synchronize(dev)
    t_all = time.perf_counter() - t0
    fm = FmIndex(w, sigma, n, sa_sample, {"C": Ct, "mwords": mw, "msb": msb, "sval": sval[:cnt.value].clone()})
    return fm, {"s": s, "sa": sa, "bwt": bwt, "sa_s": t_sa, "build_s": t_all, "layout": lay}


# ------------------------------------------------------------------------------------------------ on-disk formats
class cf_rrrw_file_header(C.Structure):
    _fields_ = [("n", A.U64), ("rrr_bytes", A.U64), ("packed_bytes", A.U64), ("bits", A.U32), ("vocab", A.U32),
                ("nblocks", A.U32), ("nsb", A.U32), ("cwords", A.U32), ("na", A.U32), ("owords", A.U32),
                ("nq", A.U32), ("nr", A.U32), ("h0", A.F32)]


class cf_rrrw_file_queries(C.Structure):
    _fields_ = [("pos", A.P), ("access_golden", A.P), ("rank_c", A.P), ("rank_i", A.P), ("rank_golden", A.P)]


class cf_fm_file_header(C.Structure):
    _fields_ = [("n", A.U64), ("rrr_bytes", A.U64)] + [(k, A.U32) for k in (
        "bits", "vocab", "sigma", "nblocks", "nsb", "cwords", "na", "owords", "sa_sample", "mwords", "msb", "nsval",
        "npat", "patflat", "nloc", "reserved")]


class cf_fm_file_arrays(C.Structure):
    _fields_ = [(k, A.P) for k in ("C", "mwords", "msb", "sval", "pat", "pstart", "plen", "count_golden", "locoff",
                                   "locpos")]


for _name, _args in (("cf_rrrw_file_read_header", [C.c_char_p, A.P]), ("cf_rrrw_file_read", [C.c_char_p, A.P, A.P, A.P]),
                     ("cf_rrrw_file_write", [C.c_char_p, A.P, A.P, A.P]),
                     ("cf_fm_file_read_header", [C.c_char_p, A.P]), ("cf_fm_file_read", [C.c_char_p, A.P, A.P, A.P]),
                     ("cf_fm_file_write", [C.c_char_p, A.P, A.P, A.P])):
    A.declare(_name, A.I32, _args)

_WAVELET = (("classes", np.uint32, lambda h: h.bits * h.cwords), ("offsets", np.uint32, lambda h: h.owords),
            ("rank_a", np.int32, lambda h: h.bits * h.na), ("rank_d", np.uint16, lambda h: h.bits * (h.nsb + 1)),
            ("off_a", np.int32, lambda h: h.bits * h.na), ("off_d", np.uint16, lambda h: h.bits * (h.nsb + 1)),
            ("offbase", np.int32, lambda h: h.bits), ("zeros", np.int32, lambda h: h.bits))
_RRRW_QUERIES = (("pos", lambda h: h.nq), ("access_golden", lambda h: h.nq), ("rank_c", lambda h: h.nr),
                 ("rank_i", lambda h: h.nr), ("rank_golden", lambda h: h.nr))
_FM = (("C", np.int32, lambda h: h.sigma), ("mwords", np.uint32, lambda h: h.mwords), ("msb", np.int32, lambda h: h.msb),
       ("sval", np.int32, lambda h: h.nsval), ("pat", np.int32, lambda h: h.patflat),
       ("pstart", np.int32, lambda h: h.npat), ("plen", np.int32, lambda h: h.npat),
       ("count_golden", np.uint32, lambda h: h.npat), ("locoff", np.int32, lambda h: h.npat + 1),
       ("locpos", np.int32, lambda h: h.nloc))


def _host_ptr(a: np.ndarray | None):
    return None if a is None or a.size == 0 else a.ctypes.data_as(C.c_void_p)


def _wavelet_struct(d: dict) -> cf_rrrw_arrays:
    return cf_rrrw_arrays(*[_host_ptr(d[k]) for k, _, _ in _WAVELET])


def read_cfrw(path: str) -> dict:
    """Read a .cfrw v1 file with the library's reader (cf_rrrw_file_read): header fields + index arrays + query
    sections as host numpy arrays."""
    L = A.lib()
    h = cf_rrrw_file_header()
    A.check(L.cf_rrrw_file_read_header(path.encode(), C.byref(h)), "cf_rrrw_file_read_header")
    d = {k: getattr(h, k) for k, _ in h._fields_}
    for k, dt, cnt in _WAVELET:
        d[k] = np.zeros(cnt(h), dt)
    for k, cnt in _RRRW_QUERIES:
        d[k] = np.zeros(cnt(h), np.uint32)
    q = cf_rrrw_file_queries(*[_host_ptr(d[k]) for k, _ in _RRRW_QUERIES])
    A.check(L.cf_rrrw_file_read(path.encode(), C.byref(h), C.byref(_wavelet_struct(d)), C.byref(q)),
            "cf_rrrw_file_read")
    return d


def write_cfrw(path: str, d: dict) -> None:
    """Write a .cfrw v1 file (cf_rrrw_file_write) from the fields/arrays `read_cfrw` returns; the query sections
    may be absent (written empty)."""
    h = cf_rrrw_file_header()
    arrays = {k: np.ascontiguousarray(d[k], dt) for k, dt, _ in _WAVELET}
    queries = {k: np.ascontiguousarray(d.get(k, np.zeros(0)), np.uint32) for k, _ in _RRRW_QUERIES}
    for k, _ in h._fields_:
        if k in ("nq", "nr"):
            continue
        setattr(h, k, d[k])
    h.nq, h.nr = queries["pos"].size, queries["rank_c"].size
    q = cf_rrrw_file_queries(*[_host_ptr(queries[k]) for k, _ in _RRRW_QUERIES])
    A.check(A.lib().cf_rrrw_file_write(path.encode(), C.byref(h), C.byref(_wavelet_struct(arrays)), C.byref(q)),
            "cf_rrrw_file_write")


def read_cffm(path: str) -> dict:
    """Read a .cffm v1 file with the library's reader (cf_fm_file_read)."""
    L = A.lib()
    h = cf_fm_file_header()
    A.check(L.cf_fm_file_read_header(path.encode(), C.byref(h)), "cf_fm_file_read_header")
    d = {k: getattr(h, k) for k, _ in h._fields_}
    for k, dt, cnt in _WAVELET + _FM:
        d[k] = np.zeros(cnt(h), dt)
    fm = cf_fm_file_arrays(*[_host_ptr(d[k]) for k, _, _ in _FM])
    A.check(L.cf_fm_file_read(path.encode(), C.byref(h), C.byref(_wavelet_struct(d)), C.byref(fm)),
            "cf_fm_file_read")
    return d


def write_cffm(path: str, d: dict) -> None:
    """Write a .cffm v1 file (cf_fm_file_write); the pattern section may be absent (written empty)."""
    h = cf_fm_file_header()
    arrays = {k: np.ascontiguousarray(d[k], dt) for k, dt, _ in _WAVELET}
    extra = {k: np.ascontiguousarray(d.get(k, np.zeros(0)), dt) for k, dt, _ in _FM}
    if extra["locoff"].size == 0:
        extra["locoff"] = np.zeros(1, np.int32)
    for k, _ in h._fields_:
        if k in ("mwords", "msb", "nsval", "npat", "patflat", "nloc", "reserved"):
            continue
        setattr(h, k, d[k])
    h.mwords, h.msb, h.nsval = extra["mwords"].size, extra["msb"].size, extra["sval"].size
    h.npat, h.patflat, h.nloc = extra["pstart"].size, extra["pat"].size, extra["locpos"].size
    fm = cf_fm_file_arrays(*[_host_ptr(extra[k]) for k, _, _ in _FM])
    A.check(A.lib().cf_fm_file_write(path.encode(), C.byref(h), C.byref(_wavelet_struct(arrays)), C.byref(fm)),
            "cf_fm_file_write")


def _wavelet_file_fields(w: RrrWaveletIndex, lay: cf_rrrw_layout) -> dict:
    dt = {"classes": np.uint32, "offsets": np.uint32, "rank_a": np.int32, "rank_d": np.uint16, "off_a": np.int32,
          "off_d": np.uint16, "offbase": np.int32, "zeros": np.int32}
    d = {k: w.tensors[k].cpu().numpy().view(dt[k]) for k in dt}
    d.update(n=int(lay.n), bits=w.bits, nblocks=int(lay.nblocks), nsb=w.nsb, cwords=w.cwords, na=w.na,
             owords=int(lay.owords), rrr_bytes=int(lay.rrr_bytes))
    return d


def save_cfrw(path: str, w: RrrWaveletIndex, lay: cf_rrrw_layout, vocab: int, symbols: torch.Tensor,
              queries: dict | None = None) -> None:
    """Write a GPU-built RRR wavelet matrix as .cfrw v1, with the header figures the reference builder writes
    (tools/build_index.cpp:403-424): packed_bytes = the packed bit-plane wavelet's footprint, h0 = the empirical
    entropy of `symbols` (the sequence the matrix was built from) in bits per symbol. `queries` optionally carries
    pos / access_golden / rank_c / rank_i / rank_golden."""
    d = _wavelet_file_fields(w, lay)
    n, bits = d["n"], d["bits"]
    nwords = (n + 31) // 32
    d["packed_bytes"] = bits * nwords * 4 + bits * ((nwords + 7) // 8 + 1) * 4
    cnt = torch.bincount(symbols.reshape(-1).long()).cpu().numpy()
    h0 = 0.0
    for c in cnt:
        if c:
            p = float(c) / n
            h0 -= p * float(np.log2(p))
    d["h0"], d["vocab"] = h0, vocab
    d.update(queries or {})
    write_cfrw(path, d)


def save_cffm(path: str, fm: FmIndex, lay: cf_rrrw_layout, vocab: int, patterns: dict | None = None) -> None:
    """Write a GPU-built FM-index (build_fm's index and layout) as .cffm v1 (reference tools/build_index.cpp:496-526).
    `patterns` optionally carries pat / pstart / plen / count_golden / locoff / locpos."""
    d = _wavelet_file_fields(fm.w, lay)
    d.update(vocab=vocab, sigma=fm.sigma, sa_sample=fm.sa_sample)
    for k, dt in (("C", np.int32), ("mwords", np.uint32), ("msb", np.int32), ("sval", np.int32)):
        d[k] = fm.tensors[k].cpu().numpy().view(dt)
    d.update(patterns or {})
    write_cffm(path, d)
