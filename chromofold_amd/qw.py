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

QW_ABI_VERSION, QW_CODEC_HUFFMAN, QW_BAND_ROWS, QW_SEG_COLS = 2, 1, 16, 64


class cf_qw_matrix(C.Structure):
    _fields_ = [("struct_size", A.U32), ("abi_version", A.U32), ("codec", A.U32), ("rows", A.U32),
                ("cols", A.U32), ("zero", A.I32), ("word_count", A.U64), ("words", A.P), ("seg_offsets", A.P), ("code_lengths", A.P),
                ("scales", A.P)]


A.declare("cf_qw_validate", A.I32, [C.POINTER(cf_qw_matrix)])
A.declare("cf_qw_matmul_async", A.I32, [C.POINTER(cf_qw_matrix), A.P, A.P, A.U32, A.P])
A.declare("cf_qw_quantize_int4", A.I32, [A.P, A.U32, A.U32, A.P, A.P])
A.declare("cf_qw_huffman_plan", A.U64, [A.P, A.U32, A.U32, A.P])
A.declare("cf_qw_huffman_encode", A.I32, [A.P, A.U32, A.U32, A.P, A.P, A.U64, A.P])


def _np_ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


@dataclass
class QwHost:
    rows: int
    cols: int
    sym: np.ndarray           # [rows, cols] u8 (q + 8)
    scales: np.ndarray        # [rows, nseg] f32
    code_lengths: np.ndarray  # [bands * 16] u8
    words: np.ndarray         # u32
    seg_offsets: np.ndarray   # [rows, nseg] u32

    @property
    def nbytes(self) -> int:
        """Resident bytes of the coded matrix: payload + segment offsets + scales + code tables."""
        return self.words.nbytes + self.seg_offsets.nbytes + self.scales.nbytes + self.code_lengths.nbytes


def encode_int4(w: np.ndarray) -> QwHost:
    """Quantise (per row x 64-column absmax) and Huffman-code a row-major f32 matrix with the library encoder."""
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    nseg = (cols + QW_SEG_COLS - 1) // QW_SEG_COLS
    sym = np.zeros((rows, cols), np.uint8)
    scales = np.zeros((rows, nseg), np.float32)
    L = A.lib()
    A.check(L.cf_qw_quantize_int4(_np_ptr(w), rows, cols, _np_ptr(sym), _np_ptr(scales)), "cf_qw_quantize_int4")
    return encode_symbols(sym, scales)


def encode_symbols(sym: np.ndarray, scales: np.ndarray) -> QwHost:
    sym = np.ascontiguousarray(sym, np.uint8)
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
    return QwHost(rows, cols, sym, np.ascontiguousarray(scales, np.float32), lens, words, offs)


class QwMatrix:
    """Device-resident coded matrix; `matmul(x_bf16)` -> y f32 [batch, rows]."""

    def __init__(self, h: QwHost, device="cuda"):
        self.host = h
        dev = torch.device(device)
        self.t = {
            "words": torch.from_numpy(h.words.view(np.int32)).to(dev),
            "offs": torch.from_numpy(h.seg_offsets.view(np.int32)).to(dev),
            "lens": torch.from_numpy(h.code_lengths).to(dev),
            "scales": torch.from_numpy(h.scales).to(dev),
        }
        t = self.t
        self.desc = cf_qw_matrix(C.sizeof(cf_qw_matrix), QW_ABI_VERSION, QW_CODEC_HUFFMAN, h.rows, h.cols, 8,
                                 h.words.size, t["words"].data_ptr(), t["offs"].data_ptr(), t["lens"].data_ptr(),
                                 t["scales"].data_ptr())

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
