"""Host-side mirror of the reference's single-sequence paged-KV seam (include/chromofold/kv_cuda.h) and of the
host runtime helpers (include/chromofold/kv_runtime.h).

`PagedKv` owns device copies of page arrays (words, block offsets, LUT, scales) and the device array of
cf_kv_device_page descriptors; `attention` fills a cf_kv_paged_attention_desc and calls
cf_kv_paged_attention_async exactly as the reference's llama.cpp adapter does
(reference integrations/llama.cpp/chromofold_kv_adapter.cpp:91-131).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _abi as A

CF_KV_CUDA_ABI_VERSION = 0
CF_KV_RUNTIME_ABI_VERSION = 0
CF_KV_PAGE_FLAG_SEALED = 1
CF_KV_PAGE_FLAG_DEVICE_RESIDENT = 2


class cf_kv_page_view(C.Structure):
    _fields_ = [("struct_size", A.U32), ("abi_version", A.U32), ("flags", A.U32), ("layer", A.U32),
                ("kv_head", A.U32), ("token_begin", A.U32), ("token_count", A.U32), ("head_dim", A.U32),
                ("block_size", A.U32), ("zero_point", A.U32),
                ("k_words", A.P), ("k_word_count", A.U64), ("k_block_offsets", A.P), ("k_block_count", A.U64),
                ("k_lut", A.P), ("k_lut_count", A.U64), ("k_scales", A.P), ("k_scale_count", A.U64),
                ("v_words", A.P), ("v_word_count", A.U64), ("v_block_offsets", A.P), ("v_block_count", A.U64),
                ("v_lut", A.P), ("v_lut_count", A.U64), ("v_scales", A.P), ("v_scale_count", A.U64)]


class cf_kv_cache_layout(C.Structure):
    _fields_ = [("struct_size", A.U32), ("abi_version", A.U32), ("layer_count", A.U32), ("kv_head_count", A.U32),
                ("head_dim", A.U32), ("page_capacity_tokens", A.U32), ("active_token_begin", A.U32),
                ("active_token_count", A.U32), ("active_element_bytes", A.U32), ("reserved", A.U32),
                ("pages", A.P), ("page_count", A.U64), ("active_k_bytes", A.U64), ("active_v_bytes", A.U64)]


class cf_kv_memory_stats(C.Structure):
    _fields_ = [("sealed_payload_bytes", A.U64), ("sealed_descriptor_bytes", A.U64),
                ("active_payload_bytes", A.U64), ("total_resident_bytes", A.U64), ("sealed_tokens", A.U64),
                ("active_tokens", A.U64), ("page_count", A.U64)]


class cf_online_softmax_state(C.Structure):
    _fields_ = [("max_score", C.c_double), ("exp_sum", C.c_double), ("weighted_values", A.P), ("dim", A.U32),
                ("initialized", A.U32)]


A.declare("cf_kv_validate_page", A.I32, [A.P])
A.declare("cf_kv_validate_layout", A.I32, [A.P])
A.declare("cf_kv_page_resident_bytes", A.I32, [A.P, A.P])
A.declare("cf_kv_cache_memory_stats", A.I32, [A.P, A.P])
A.declare("cf_online_softmax_init", A.I32, [A.P, A.P, A.U32])
A.declare("cf_online_softmax_accumulate", A.I32, [A.P, C.c_double, A.P])
A.declare("cf_online_softmax_merge", A.I32, [A.P, A.P])
A.declare("cf_online_softmax_finalize", A.I32, [A.P, A.P])


@dataclass
class HostPage:
    """One encoded page of one KV head (host arrays in the reference's EncodedKvPage shape)."""
    kv_head: int
    token_begin: int
    token_count: int
    head_dim: int
    k_words: np.ndarray
    k_block_offsets: np.ndarray
    k_lut: np.ndarray
    k_scales: np.ndarray
    v_words: np.ndarray
    v_block_offsets: np.ndarray
    v_lut: np.ndarray
    v_scales: np.ndarray
    block_size: int = 64
    k_max_code_length: int = 8
    v_max_code_length: int = 8
    zero_point: int = 128
    fixed_code_length: int = 8


def _dev(a, device, dtype):
    return torch.from_numpy(np.ascontiguousarray(a).view(dtype)).to(device)


@dataclass
class PagedKv:
    pages: list
    device: str = "cuda"
    _keep: list = field(default_factory=list)
    descs: torch.Tensor | None = None
    share_luts: bool = False  # pages whose k_lut / v_lut bytes are equal point at one device copy

    def __post_init__(self):
        arr = (A.cf_kv_device_page * max(1, len(self.pages)))()
        shared = {}

        def upload(k, a):
            dt = np.int32 if k != "k_scales" and k != "v_scales" else np.float32
            if not (self.share_luts and k in ("k_lut", "v_lut")):
                return _dev(a, self.device, dt)
            key = np.ascontiguousarray(a).tobytes()
            if key not in shared:
                shared[key] = _dev(a, self.device, dt)
            return shared[key]
        for i, p in enumerate(self.pages):
            t = {k: upload(k, getattr(p, k))
                 for k in ["k_words", "k_block_offsets", "k_lut", "k_scales", "v_words", "v_block_offsets", "v_lut",
                           "v_scales"]}
            self._keep.append(t)
            arr[i] = A.cf_kv_device_page(*[t[k].data_ptr() for k in ["k_words", "k_block_offsets", "k_lut",
                                                                      "k_scales", "v_words", "v_block_offsets",
                                                                      "v_lut", "v_scales"]],
                                         p.token_begin, p.token_count, p.head_dim, p.block_size,
                                         p.k_max_code_length, p.v_max_code_length, p.zero_point, p.kv_head,
                                         p.fixed_code_length)
        raw = np.frombuffer(bytes(arr), np.uint8).copy()
        self.descs = torch.from_numpy(raw).to(self.device)

    def desc(self, queries, output, kv_heads, gqa, query_token_begin, softmax_scale, causal_window=0,
             active=None, head_dim=None) -> A.cf_kv_paged_attention_desc:
        d = A.cf_kv_paged_attention_desc()
        d.struct_size = C.sizeof(A.cf_kv_paged_attention_desc)
        d.abi_version = CF_KV_CUDA_ABI_VERSION
        d.pages = self.descs.data_ptr() if self.pages else None
        d.page_count = len(self.pages)
        d.kv_head_count = kv_heads
        d.query_head_count = queries.shape[1]
        d.gqa_group_size = gqa
        if active is not None:
            tok0, ak, av = active
            d.active_k, d.active_v = ak.data_ptr(), av.data_ptr()
            d.active_token_begin, d.active_token_count = tok0, ak.shape[0]
        d.queries, d.output = queries.data_ptr(), output.data_ptr()
        d.query_token_begin = query_token_begin
        d.query_count = queries.shape[0]
        d.head_dim = head_dim if head_dim is not None else queries.shape[2]
        d.causal_window = causal_window
        d.softmax_scale = softmax_scale
        return d

    def attention(self, queries, kv_heads, gqa, query_token_begin, softmax_scale, causal_window=0, active=None,
                  stream=None):
        out = torch.full_like(queries, float("nan"))
        d = self.desc(queries, out, kv_heads, gqa, query_token_begin, softmax_scale, causal_window, active)
        s = (stream if stream is not None else torch.cuda.current_stream()).cuda_stream
        A.check(A.lib().cf_kv_paged_attention_async(C.byref(d), s), "cf_kv_paged_attention_async")
        return out
