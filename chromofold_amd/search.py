"""Host-side mirror of the compressed-domain search interface (RRR wavelet matrix, FM-index).

Mirrors the reference's C ABI `include/chromofold/chromofold_search.h` (cf_rrrw_access_async, cf_rrrw_rank_async,
cf_fm_count_async, cf_fm_ranges_async, cf_fm_locate_async): device-resident index arrays are held as torch tensors
(plumbing for HBM allocation and streams); every query runs through libchromofold.so. Errors surface as CfError
carrying the cf_status the C entry point returned.
"""
from __future__ import annotations

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

    def rank(self, symbols: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        out = torch.empty_like(positions, dtype=torch.int32)
        self.rank_into(symbols, positions, out)
        return out


def to_u32(t: torch.Tensor) -> np.ndarray:
    """Device int32 tensor holding u32 bits -> host uint32 array."""
    return t.cpu().numpy().view(np.uint32)


def u32_dev(a, device="cuda") -> torch.Tensor:
    return _dev(np.asarray(a, dtype=np.uint32), device)
