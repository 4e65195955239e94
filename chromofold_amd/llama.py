"""ctypes mirror of the llama.cpp paged-KV adapter (include/chromofold/chromofold_kv_adapter.h; reference
integrations/llama.cpp/chromofold_kv_adapter.h:1-89). `KvAdapter` wraps the handle; every method calls
libchromofold and raises CfAdapterError with cf_llama_kv_last_error() when the C call returns -1."""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _abi as A

BACKEND_DENSE, BACKEND_CHROMOFOLD = 0, 1


class cf_llama_kv_options(C.Structure):
    _fields_ = [("struct_size", A.U32), ("backend", C.c_int), ("layer_count", A.U32), ("kv_head_count", A.U32),
                ("query_head_count", A.U32), ("head_dim", A.U32), ("page_size", A.U32),
                ("gqa_group_size", A.U32), ("kv_bits", A.U32)]


class cf_llama_kv_stats(C.Structure):
    _fields_ = [(k, A.U64) for k in ("appended_tokens", "sealed_tokens", "sealed_pages", "active_tokens",
                                      "dense_active_bytes", "compressed_bytes", "descriptor_bytes")]


_H = A.P
A.declare("cf_llama_kv_options_validate", C.c_int, [C.POINTER(cf_llama_kv_options)])
A.declare("cf_llama_kv_create", _H, [C.POINTER(cf_llama_kv_options)])
A.declare("cf_llama_kv_destroy", None, [_H])
A.declare("cf_llama_kv_append", C.c_int, [_H, A.U32, A.U32, A.U32, A.P, A.P, A.U32, A.P])
A.declare("cf_llama_kv_attention", C.c_int, [_H, A.U32, A.P, A.P, A.U32, A.U32, A.U32, A.U32, A.F32, A.U32, A.P])
A.declare("cf_llama_kv_attention_host", C.c_int, [_H, A.U32, A.P, A.P, A.U32, A.U32, A.U32, A.U32, A.F32, A.U32,
                                                  A.P])
A.declare("cf_llama_kv_flush", C.c_int, [_H, A.P])
A.declare("cf_llama_kv_seq_rm", C.c_int, [_H, A.U64])
A.declare("cf_llama_kv_seq_cp", C.c_int, [_H, A.U64, A.U64])
A.declare("cf_llama_kv_seq_shift", C.c_int, [_H, A.U64, C.c_int32])
A.declare("cf_llama_kv_clear", C.c_int, [_H])
A.declare("cf_llama_kv_get_stats", C.c_int, [_H, C.POINTER(cf_llama_kv_stats)])
A.declare("cf_llama_kv_last_error", C.c_char_p, [_H])
A.declare("cf_kv_encode_fixed_page", A.I32, [A.U32, A.P, A.P, A.U32, A.U32, A.U32, A.P, A.P, A.P, A.P, A.P])


class CfAdapterError(RuntimeError):
    pass


def options(layer_count, kv_heads, query_heads, head_dim, page_size, gqa, kv_bits=0,
            backend=BACKEND_CHROMOFOLD) -> cf_llama_kv_options:
    return cf_llama_kv_options(C.sizeof(cf_llama_kv_options), backend, layer_count, kv_heads, query_heads, head_dim,
                               page_size, gqa, kv_bits)


def encode_fixed_page(bits: int, keys: np.ndarray, values: np.ndarray, block: int = 64):
    """cf_kv_encode_fixed_page -> (k_words, v_words, k_scales, v_scales, block_offsets)."""
    k = np.ascontiguousarray(keys, np.float32)
    v = np.ascontiguousarray(values, np.float32)
    T, D = k.shape
    n = T * D
    kw = np.zeros((n * bits + 31) // 32, np.uint32)
    vw = np.zeros_like(kw)
    ks = np.zeros(D, np.float32)
    vs = np.zeros(T, np.float32)
    bo = np.zeros((n + block - 1) // block, np.int32)
    p = lambda a: a.ctypes.data_as(C.c_void_p)
    A.check(A.lib().cf_kv_encode_fixed_page(bits, p(k), p(v), T, D, block, p(kw), p(vw), p(ks), p(vs), p(bo)),
            "cf_kv_encode_fixed_page")
    return kw, vw, ks, vs, bo


class KvAdapter:
    def __init__(self, opts: cf_llama_kv_options):
        self.L = A.lib()
        self.h = self.L.cf_llama_kv_create(C.byref(opts))
        if not self.h:
            raise CfAdapterError("cf_llama_kv_create returned NULL")
        self.head_dim = opts.head_dim

    def _ok(self, rc: int, what: str) -> None:
        if rc != 0:
            raise CfAdapterError(f"{what}: {self.last_error()}")

    def last_error(self) -> str:
        return self.L.cf_llama_kv_last_error(self.h).decode()

    def append(self, layer, head, token_begin, keys: np.ndarray, values: np.ndarray, stream=None):
        k = np.ascontiguousarray(keys, np.float32)
        v = np.ascontiguousarray(values, np.float32)
        self._ok(self.L.cf_llama_kv_append(self.h, layer, head, token_begin, k.ctypes.data_as(C.c_void_p),
                                           v.ctypes.data_as(C.c_void_p), k.shape[0], stream), "append")

    def attention(self, layer, q_dev, out_dev, query_count, query_heads, gqa, query_token_begin, scale, window=0,
                  stream=None):
        self._ok(self.L.cf_llama_kv_attention(self.h, layer, q_dev, out_dev, query_count, query_heads, gqa,
                                              query_token_begin, scale, window, stream), "attention")

    def attention_host(self, layer, q: np.ndarray, query_heads, gqa, query_token_begin, scale, window=0, stream=None):
        q = np.ascontiguousarray(q, np.float32)
        out = np.zeros_like(q)
        self._ok(self.L.cf_llama_kv_attention_host(self.h, layer, q.ctypes.data_as(C.c_void_p),
                                                   out.ctypes.data_as(C.c_void_p), q.shape[0], query_heads, gqa,
                                                   query_token_begin, scale, window, stream), "attention_host")
        return out

    def flush(self, stream=None):
        self._ok(self.L.cf_llama_kv_flush(self.h, stream), "flush")

    def stats(self) -> cf_llama_kv_stats:
        st = cf_llama_kv_stats()
        self._ok(self.L.cf_llama_kv_get_stats(self.h, C.byref(st)), "get_stats")
        return st

    def close(self):
        if self.h:
            self.L.cf_llama_kv_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
