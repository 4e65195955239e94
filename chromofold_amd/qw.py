"""Host side of decode-in-matmul: the reference's single-stream fused matmul (cf_fused_matmul_async /
cf_dense_matmul_async, reference src/cuda/fused_matmul.cu:67-96) and the band-table int4 format cf_qw_matrix
(include/chromofold/chromofold_qw.h). Encoding runs in libchromofold's C++ host encoder; every product call runs the
gfx950 kernels. Torch tensors are only device-memory plumbing.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np
import torch

from . import _abi as A

QW_ABI_VERSION, QW_CODEC_HUFFMAN, QW_CODEC_RANS, QW_BAND_ROWS, QW_SEG_COLS = 3, 1, 2, 16, 64
QW_STRIPE_COLS, QW_CHUNK_STRIPES = 256, 16


class cf_qw_matrix(C.Structure):
    _fields_ = [("struct_size", A.U32), ("abi_version", A.U32), ("codec", A.U32), ("rows", A.U32),
                ("cols", A.U32), ("zero", A.I32), ("word_count", A.U64), ("words", A.P), ("offsets", A.P),
                ("tables", A.P), ("scales", A.P), ("states", A.P), ("chunk_words", A.U32), ("last_words", A.U32)]


A.declare("cf_qw_validate", A.I32, [C.POINTER(cf_qw_matrix)])
A.declare("cf_qw_matmul_async", A.I32, [C.POINTER(cf_qw_matrix), A.P, A.P, A.U32, A.P])
A.declare("cf_qw_quantize_int4", A.I32, [A.P, A.U32, A.U32, A.P, A.P])
A.declare("cf_qw_huffman_plan", A.U64, [A.P, A.U32, A.U32, A.P])
A.declare("cf_qw_huffman_encode", A.I32, [A.P, A.U32, A.U32, A.P, A.P, A.U64, A.P])
A.declare("cf_qw_rans_plan", A.I32, [A.P, A.U32, A.U32, C.c_uint8, A.P, A.P, A.P])
A.declare("cf_qw_rans_encode", A.I32, [A.P, A.U32, A.U32, C.c_uint8, A.P, A.U32, A.U32, A.P, A.U64, A.P, A.P])


def _np_ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


@dataclass
class QwHost:
    rows: int
    cols: int
    sym: np.ndarray           # [rows, cols] u8 (q + 8)
    scales: np.ndarray        # [rows, nseg] f32
    tables: np.ndarray        # HUFFMAN [bands * 16] u8 code lengths; RANS [bands * 256] u16 cumulative starts
    words: np.ndarray         # u32
    offsets: np.ndarray       # HUFFMAN [rows, nseg] bit offsets; RANS [bands * nstripes] slot offsets (u32)
    codec: int = QW_CODEC_HUFFMAN
    states: np.ndarray | None = None  # RANS [bands * nstripes * 64] u32
    chunk_words: int = 0              # RANS 16-bit words per full-chunk slot
    last_words: int = 0               # RANS 16-bit words of a band's last slot
    zero: int = 8

    @property
    def nbytes(self) -> int:
        """Resident bytes of the coded matrix: payload + offsets + scales + code tables (+ lane states)."""
        n = self.words.nbytes + self.offsets.nbytes + self.scales.nbytes + self.tables.nbytes
        return n + (self.states.nbytes if self.states is not None else 0)


def quantize_int4(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per (row, 64-column segment) absmax int4 quantisation with the library: (sym [rows, cols] u8, scales)."""
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    nseg = (cols + QW_SEG_COLS - 1) // QW_SEG_COLS
    sym = np.zeros((rows, cols), np.uint8)
    scales = np.zeros((rows, nseg), np.float32)
    L = A.lib()
    A.check(L.cf_qw_quantize_int4(_np_ptr(w), rows, cols, _np_ptr(sym), _np_ptr(scales)), "cf_qw_quantize_int4")
    return sym, scales


def encode_int4(w: np.ndarray, codec: int = QW_CODEC_HUFFMAN) -> QwHost:
    """Quantise (per row x 64-column absmax) and entropy-code a row-major f32 matrix with the library encoder."""
    sym, scales = quantize_int4(w)
    return encode_symbols(sym, scales, codec)


def encode_symbols(sym: np.ndarray, scales: np.ndarray, codec: int = QW_CODEC_HUFFMAN, zero: int = 8) -> QwHost:
    sym = np.ascontiguousarray(sym, np.uint8)
    if codec == QW_CODEC_RANS:
        return encode_symbols_rans(sym, scales, zero)
    rows, cols = sym.shape
    nseg = (cols + QW_SEG_COLS - 1) // QW_SEG_COLS
    bands = (rows + QW_BAND_ROWS - 1) // QW_BAND_ROWS
    lens = np.zeros(bands * 16, np.uint8)
    L = A.lib()
    nw = int(L.cf_qw_huffman_plan(_np_ptr(sym), rows, cols, _np_ptr(lens)))
    if nw == 0:
        raise A.CfError(A.CF_ERR_INVALID_ARGUMENT, "cf_qw_huffman_plan")
    words = np.zeros(nw, np.uint32)
    offs = np.zeros((rows, nseg), np.uint32)
    A.check(L.cf_qw_huffman_encode(_np_ptr(sym), rows, cols, _np_ptr(lens), _np_ptr(words), nw, _np_ptr(offs)),
            "cf_qw_huffman_encode")
    return QwHost(rows, cols, sym, np.ascontiguousarray(scales, np.float32), lens, words, offs, zero=zero)


def encode_symbols_rans(sym: np.ndarray, scales: np.ndarray, zero: int = 8) -> QwHost:
    sym = np.ascontiguousarray(sym, np.uint8)
    rows, cols = sym.shape
    bands = (rows + QW_BAND_ROWS - 1) // QW_BAND_ROWS
    nstripes = (cols + QW_STRIPE_COLS - 1) // QW_STRIPE_COLS
    nchunks = (nstripes + QW_CHUNK_STRIPES - 1) // QW_CHUNK_STRIPES
    cum = np.zeros(bands * 256, np.uint16)
    L = A.lib()
    cw, lw = C.c_uint32(0), C.c_uint32(0)
    A.check(L.cf_qw_rans_plan(_np_ptr(sym), rows, cols, zero, _np_ptr(cum), C.byref(cw), C.byref(lw)),
            "cf_qw_rans_plan")
    cw, lw = cw.value, lw.value
    nw = bands * ((nchunks - 1) * cw + lw) // 2
    words = np.zeros(nw, np.uint32)
    offs = np.zeros(bands * nstripes, np.uint32)
    states = np.zeros(bands * nstripes * 64, np.uint32)
    A.check(L.cf_qw_rans_encode(_np_ptr(sym), rows, cols, zero, _np_ptr(cum), cw, lw, _np_ptr(words), nw,
                                _np_ptr(offs), _np_ptr(states)), "cf_qw_rans_encode")
    return QwHost(rows, cols, sym, np.ascontiguousarray(scales, np.float32), cum, words, offs, QW_CODEC_RANS,
                  states, cw, lw, zero)


class QwMatrix:
    """Device-resident coded matrix; `matmul(x_bf16)` -> y f32 [batch, rows]."""

    def __init__(self, h: QwHost, device="cuda"):
        self.host = h
        dev = torch.device(device)
        self.t = {
            "words": torch.from_numpy(h.words.view(np.int32)).to(dev),
            "offs": torch.from_numpy(h.offsets.view(np.int32)).to(dev),
            "tables": torch.from_numpy(h.tables.view(np.uint8)).to(dev),
            "scales": torch.from_numpy(h.scales).to(dev),
        }
        if h.states is not None:
            self.t["states"] = torch.from_numpy(h.states.view(np.int32)).to(dev)
        t = self.t
        self.desc = cf_qw_matrix(C.sizeof(cf_qw_matrix), QW_ABI_VERSION, h.codec, h.rows, h.cols, h.zero,
                                 h.words.size, t["words"].data_ptr(), t["offs"].data_ptr(), t["tables"].data_ptr(),
                                 t["scales"].data_ptr(), t["states"].data_ptr() if "states" in t else None,
                                 h.chunk_words, h.last_words)

    def matmul_into(self, x: torch.Tensor, y: torch.Tensor, stream=None) -> None:
        assert x.dtype == torch.bfloat16 and x.is_contiguous() and x.shape[1] == self.host.cols
        assert y.dtype == torch.float32 and y.shape == (x.shape[0], self.host.rows)
        s = (stream if stream is not None else torch.cuda.current_stream()).cuda_stream
        A.check(A.lib().cf_qw_matmul_async(C.byref(self.desc), x.data_ptr(), y.data_ptr(), x.shape[0], s),
                "cf_qw_matmul_async")

    def matmul(self, x: torch.Tensor) -> torch.Tensor:
        y = torch.empty((x.shape[0], self.host.rows), dtype=torch.float32, device=x.device)
        self.matmul_into(x, y)
        return y


def fused_matmul(words, block_off, lut, maxlen: int, block: int, x: torch.Tensor, y: torch.Tensor, M: int, K: int,
                 scale: float, zero: int, stream=None) -> None:
    """cf_fused_matmul_async on device tensors (x f32 [B, K], y f32 [B, M])."""
    s = (stream if stream is not None else torch.cuda.current_stream()).cuda_stream
    A.check(A.lib().cf_fused_matmul_async(words.data_ptr(), block_off.data_ptr(), lut.data_ptr(), maxlen, block,
                                          x.data_ptr(), y.data_ptr(), x.shape[0], M, K, scale, zero, s),
            "cf_fused_matmul_async")


def dense_matmul(words, block_off, lut, maxlen: int, block: int, x: torch.Tensor, W: torch.Tensor, y: torch.Tensor,
                 M: int, K: int, scale: float, zero: int, stream=None) -> None:
    """cf_dense_matmul_async: decodes W [M, K] f32 into `W`, then y = x W^T."""
    s = (stream if stream is not None else torch.cuda.current_stream()).cuda_stream
    A.check(A.lib().cf_dense_matmul_async(words.data_ptr(), block_off.data_ptr(), lut.data_ptr(), maxlen, block,
                                          x.data_ptr(), W.data_ptr(), y.data_ptr(), x.shape[0], M, K, scale, zero, s),
            "cf_dense_matmul_async")
