"""ctypes mirror of the chromoFold C ABI (include/chromofold/*.h) over libchromofold.so.

The structs below are field-for-field copies of the C headers (which themselves keep the reference's layouts:
reference include/chromofold/chromofold.h:38-46, chromofold_search.h:27-55, kv_cuda.h:21-75). Sizes are checked
against the C compiler's view in the CPU tests.

The library is the product path: there is no fallback. If libchromofold.so is missing, `lib()` raises.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libchromofold.so")

P = C.c_void_p
U32, I32, U64, I64, F32, SZ = C.c_uint32, C.c_int32, C.c_uint64, C.c_int64, C.c_float, C.c_size_t

CF_OK, CF_ERR_INVALID_ARGUMENT, CF_ERR_UNSUPPORTED, CF_ERR_CUDA = 0, 1, 2, 3
STATUS_NAMES = {0: "CF_OK", 1: "CF_ERR_INVALID_ARGUMENT", 2: "CF_ERR_UNSUPPORTED", 3: "CF_ERR_CUDA"}


class CfError(RuntimeError):
    def __init__(self, status: int, what: str):
        super().__init__(f"{what} -> {STATUS_NAMES.get(status, status)}")
        self.status = status


# ----------------------------------------------------------------------------------------------- structs
class cf_wavelet_view(C.Structure):
    _fields_ = [("bitplanes", P), ("superblocks", P), ("zero_counts", P), ("token_count", U64),
                ("levels", U32), ("nwords", U32), ("nblocks", U32)]


class cf_rrrw_view(C.Structure):
    _fields_ = [("classes", P), ("offsets", P), ("rank_a", P), ("rank_d", P), ("off_a", P), ("off_d", P),
                ("offbase", P), ("zeros", P), ("width", P), ("binom", P), ("bits", C.c_int),
                ("cwords", C.c_int), ("nsb", C.c_int), ("na", C.c_int)]


class cf_fm_view(C.Structure):
    _fields_ = [("w", cf_rrrw_view), ("C", P), ("mwords", P), ("msb", P), ("sval", P), ("sigma", C.c_int),
                ("n", C.c_int), ("sa_sample", C.c_int)]


class cf_kv_device_page(C.Structure):
    _fields_ = [("k_words", P), ("k_block_offsets", P), ("k_lut", P), ("k_scales", P),
                ("v_words", P), ("v_block_offsets", P), ("v_lut", P), ("v_scales", P),
                ("token_begin", U32), ("token_count", U32), ("head_dim", U32), ("block_size", U32),
                ("k_max_code_length", U32), ("v_max_code_length", U32), ("zero_point", U32), ("kv_head", U32),
                ("fixed_code_length", U32)]


class cf_kv_paged_attention_desc(C.Structure):
    _fields_ = [("struct_size", U32), ("abi_version", U32), ("pages", P), ("page_count", U32),
                ("kv_head_count", U32), ("query_head_count", U32), ("gqa_group_size", U32),
                ("active_k", P), ("active_v", P), ("active_token_begin", U32), ("active_token_count", U32),
                ("queries", P), ("output", P), ("query_token_begin", U32), ("query_count", U32),
                ("head_dim", U32), ("causal_window", U32), ("softmax_scale", F32)]


# ----------------------------------------------------------------------------------------------- signatures
_SIGS: dict[str, tuple] = {
    # chromofold.h
    "cf_access_async": (I32, [cf_wavelet_view, P, P, SZ, P]),
    "cf_rank_async": (I32, [cf_wavelet_view, P, P, P, SZ, P]),
    "cf_embedding_gather_async": (I32, [cf_wavelet_view, P, U32, P, P, SZ, P]),
    "cf_kv_attn_fused_async": (I32, [P, P, P, C.c_int, P, P, P, C.c_int, P, P, P, P, C.c_int, C.c_int, C.c_int,
                                     C.c_int, C.c_int, C.c_int, F32, P]),
    "cf_kv_attn_dense_async": (I32, [P, P, P, C.c_int, P, P, P, C.c_int, P, P, P, P, P, P, C.c_int, C.c_int,
                                     C.c_int, C.c_int, C.c_int, C.c_int, F32, P]),
    # chromofold_search.h
    "cf_rrrw_access_async": (I32, [cf_rrrw_view, P, P, SZ, P]),
    "cf_rrrw_rank_async": (I32, [cf_rrrw_view, P, P, P, SZ, P]),
    "cf_fm_count_async": (I32, [cf_fm_view, P, P, P, P, SZ, P]),
    "cf_fm_ranges_async": (I32, [cf_fm_view, P, P, P, P, P, SZ, P]),
    "cf_fm_locate_async": (I32, [cf_fm_view, P, P, SZ, P]),
    # chromofold_extra.h (the reference's benchmark-level entry points)
    "cf_rank2_async": (I32, [cf_wavelet_view, P, P, C.c_int, C.c_int, P, P, P, SZ, P]),
    "cf_embedding_gather_tpq_async": (I32, [cf_wavelet_view, P, U32, P, P, SZ, P]),
    "cf_rrr_rank_async": (I32, [P, P, P, P, P, P, P, P, SZ, P]),
    "cf_delta_fetch_async": (I32, [P, C.c_int, P, P, P, P, P, P, P, SZ, P]),
    "cf_sparse_gather_fused_async": (I32, [cf_rrrw_view, P, C.c_int, P, P, SZ, P]),
    "cf_sparse_decode_all_async": (I32, [cf_rrrw_view, P, SZ, P]),
    "cf_sparse_gather_async": (I32, [P, P, C.c_int, P, P, SZ, P]),
    "cf_rans_decode_async": (I32, [P, P, P, P, P, P, C.c_int, C.c_int, P, P]),
    "cf_fused_matmul_async": (I32, [P, P, P, C.c_int, C.c_int, P, P, C.c_int, C.c_int, C.c_int, F32, C.c_int, P]),
    "cf_dense_matmul_async": (I32, [P, P, P, C.c_int, C.c_int, P, P, P, C.c_int, C.c_int, C.c_int, F32, C.c_int,
                                    P]),
    # kv_cuda.h
    "cf_kv_validate_paged_attention_desc": (I32, [P]),
    "cf_kv_paged_attention_async": (I32, [P, P]),
}

_lib = None


def lib() -> C.CDLL:
    """Load libchromofold.so (after torch, so one HIP runtime serves both). Raises if it was never built."""
    global _lib
    if _lib is None:
        import torch  # noqa: F401  (torch's libamdhip64 must be the one the library binds to)
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"libchromofold.so not built: {LIB_PATH} (run __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name, None)
            if fn is not None:
                fn.restype = res
                fn.argtypes = args
        _lib = L
    return _lib


def declare(name: str, res, args) -> None:
    """Register a signature for an entry point declared in an additive header."""
    _SIGS[name] = (res, args)
    if _lib is not None:
        fn = getattr(_lib, name)
        fn.restype = res
        fn.argtypes = args


def check(status: int, what: str) -> None:
    if status != CF_OK:
        raise CfError(status, what)
