"""Host mirror of the device seal engine, the device KV dataplane, the multi-sequence resolver and the batched
attention runtime.

ctypes structs and thin classes over libchromofold.so for include/chromofold/device_kv_dataplane.h,
device_kv_seal_attention.h, multisequence_cuda_resolver.h and production_attention.h (the reference's headers of
the same names: reference include/chromofold/device_kv_dataplane.h:11-89, device_kv_seal_attention.h:11-121,
multisequence_cuda_resolver.h:12-93, production_attention.h:11-105). Functions of those APIs return 0 / -1; the classes raise SealError with the
library's last-error message on -1. Device tensors are torch tensors on the GPU; no host fallback exists.
"""
from __future__ import annotations

import ctypes as C

import torch

from . import _abi as A

P, U32, U64, I32, I64, F32 = A.P, A.U32, A.U64, A.I32, A.I64, A.F32

CF_DEVICE_F16, CF_DEVICE_BF16, CF_DEVICE_F32 = 1, 2, 3
_TYPE = {torch.float16: CF_DEVICE_F16, torch.bfloat16: CF_DEVICE_BF16, torch.float32: CF_DEVICE_F32}

SEAL_STATES = ("ACTIVE_FILLING", "ACTIVE_FULL", "VALIDATING", "QUANTIZING", "PACKING", "PUBLISHING", "FAILED")
SEAL_FAULTS = ("NONE", "CANDIDATE_ALLOC", "FINITE_VALIDATION", "SCALE_ALLOC", "QUANTIZE_LAUNCH", "PAYLOAD_ALLOC",
               "PACK_LAUNCH", "DESCRIPTOR_VALIDATE", "PAGE_TABLE_GROW", "DESCRIPTOR_PUBLISH", "ACTIVE_REPLACEMENT")


class SealError(RuntimeError):
    pass


class cf_device_tensor_view(C.Structure):
    _fields_ = [("data", P), ("scalar_type", U32), ("token_count", U32), ("head_count", U32), ("head_dim", U32),
                ("token_stride_bytes", U64), ("head_stride_bytes", U64), ("element_stride_bytes", U64),
                ("device_ordinal", I32)]


class cf_device_page_descriptor(C.Structure):
    _fields_ = [("key_payload", P), ("value_payload", P), ("key_scales", P), ("value_scales", P),
                ("token_begin", U32), ("token_count", U32), ("kv_head_count", U32), ("head_dim", U32),
                ("block_size", U32), ("blocks_per_page", U32), ("key_payload_bytes", U64),
                ("value_payload_bytes", U64), ("resident_bytes", U64), ("generation", U64)]


class cf_device_seal_config(C.Structure):
    _fields_ = [(k, U32) for k in ("layer_count", "kv_head_count", "query_head_count", "head_dim", "page_size",
                                   "gqa_group_size", "block_size", "use_async_allocator")]


class cf_device_seal_counters(C.Structure):
    _fields_ = [(k, U64) for k in (
        "seal_attempts", "seal_successes", "seal_failures", "finite_validation_launches", "values_scanned",
        "nan_values", "inf_values", "invalid_pages_rejected", "quantization_launches", "values_quantized",
        "saturation_count", "packing_launches", "symbols_packed", "payload_bytes_written", "descriptor_validations",
        "descriptor_publications", "page_table_reallocations", "page_table_generation",
        "compressed_attention_launches", "sealed_pages_consumed", "sealed_values_consumed", "active_values_consumed",
        "query_conversion_launches", "output_conversion_launches", "cuda_errors", "compressed_bytes",
        "descriptor_bytes", "workspace_bytes", "peak_owned_bytes")]


class cf_device_kv_config(C.Structure):
    _fields_ = [(k, U32) for k in ("layer_count", "kv_head_count", "query_head_count", "head_dim", "page_size",
                                   "gqa_group_size", "use_async_allocator")]


class cf_device_kv_counters(C.Structure):
    _fields_ = [(k, U64) for k in (
        "device_append_calls", "device_values_appended", "fp16_values_converted", "bf16_values_converted",
        "fp32_values_copied", "quantization_launches", "huffman_pack_launches", "seal_attempts", "seal_successes",
        "seal_failures", "descriptor_publications", "compressed_attention_launches", "sealed_values_consumed",
        "active_values_consumed", "query_conversion_launches", "output_conversion_launches",
        "dense_fallback_launches", "cuda_errors", "active_bytes", "compressed_bytes", "descriptor_bytes",
        "workspace_bytes", "retired_pending_bytes", "peak_owned_bytes")]


class cf_ms_cuda_config(C.Structure):
    _fields_ = [(k, U32) for k in ("layer_count", "kv_head_count", "query_head_count", "head_dim", "page_size",
                                   "gqa_group_size", "use_async_allocator")]


class cf_ms_page_publication(C.Structure):
    _fields_ = [("sequence_id", I64), ("layer", U32), ("descriptor", cf_device_page_descriptor),
                ("resident_bytes", U64), ("seal_generation", U64)]


class cf_ms_batch_item(C.Structure):
    _fields_ = [("sequence_id", I64), ("layer", U32), ("query", cf_device_tensor_view), ("output", P),
                ("output_type", U32), ("output_token_stride_bytes", U64), ("output_head_stride_bytes", U64),
                ("output_element_stride_bytes", U64), ("query_token_begin", U32), ("softmax_scale", F32),
                ("causal_window", U32)]


class cf_ms_cuda_counters(C.Structure):
    _fields_ = [(k, U64) for k in (
        "pages_registered", "page_registration_failures", "descriptor_tables_built", "descriptor_table_rebuilds",
        "snapshots_acquired", "snapshots_released", "in_flight_page_references", "snapshot_release_events",
        "stale_snapshot_rejections", "server_batches_received", "compressed_batches_executed",
        "sequence_attention_launches", "prefill_items", "decode_items", "tokens_per_batch_peak",
        "copy_on_write_tail_copies", "cancellation_requests", "pages_retired", "pages_reclaimed",
        "pending_reclamation_bytes", "pending_reclamation_bytes_peak", "cross_sequence_contamination",
        "dense_fallback_launches", "cuda_errors")]


CF_ATTENTION_REFERENCE, CF_ATTENTION_OPTIMIZED = 0, 1


class cf_attention_tuning(C.Structure):
    _fields_ = [(k, U32) for k in ("threads_per_block", "warps_per_block", "heads_per_block", "pages_per_work_unit",
                                   "vector_width", "enable_cuda_graphs", "enable_async_sealing")]


class cf_attention_runtime_config(C.Structure):
    _fields_ = [(k, U32) for k in ("layer_count", "query_head_count", "kv_head_count", "head_dim", "page_size",
                                   "block_size", "gqa_group_size", "cuda_device", "use_async_allocator")] + \
               [("mode", C.c_int), ("tuning", cf_attention_tuning)]


class cf_attention_batch_item(C.Structure):
    _fields_ = [("sequence_id", I64), ("layer", U32), ("query", cf_device_tensor_view), ("output", P),
                ("output_type", U32), ("output_token_stride_bytes", U64), ("output_head_stride_bytes", U64),
                ("output_element_stride_bytes", U64), ("query_token_begin", U32), ("softmax_scale", F32),
                ("causal_window", U32), ("sealed_pages", P), ("sealed_page_count", U32), ("active_keys", P),
                ("active_values", P), ("active_token_begin", U32), ("active_token_count", U32)]


class cf_attention_counters(C.Structure):
    _fields_ = [(k, U64) for k in (
        "reference_launches", "optimized_launches", "decode_launches", "prefill_launches", "grouped_batches",
        "grouped_items", "kernel_launches_avoided", "graph_captures", "graph_replays", "graph_invalidations",
        "graph_replay_failures", "async_seal_submissions", "async_seal_overlaps", "descriptor_bytes_read",
        "compressed_payload_bytes_read", "scale_bytes_read", "allocation_count", "pool_hits", "pool_misses",
        "peak_reserved_bytes", "peak_live_bytes", "numerical_failures", "cross_sequence_contamination",
        "dense_fallback_launches", "cuda_errors")]


_SIGS = {
    "cf_device_tensor_validate": (C.c_int, [P]),
    "cf_device_seal_create": (P, [P]),
    "cf_device_seal_destroy": (None, [P, P]),
    "cf_device_seal_stage_active_page": (C.c_int, [P, U32, U32, P, P, U32, P]),
    "cf_device_seal_full_page_async": (C.c_int, [P, U32, P]),
    "cf_device_seal_attention_async": (C.c_int, [P, U32, P, P, U32, U64, U64, U64, U32, F32, U32, P]),
    "cf_device_seal_clear_async": (C.c_int, [P, P]),
    "cf_device_seal_set_fault": (C.c_int, [P, U32]),
    "cf_device_seal_get_state": (C.c_int, [P, U32, P]),
    "cf_device_seal_get_counters": (C.c_int, [P, P]),
    "cf_device_seal_last_error": (C.c_char_p, [P]),
    "cf_device_seal_get_pages": (C.c_int, [P, U32, P, U32, P]),
    "cf_device_kv_create": (P, [P]),
    "cf_device_kv_destroy": (None, [P, P]),
    "cf_device_kv_append_async": (C.c_int, [P, U32, U32, P, P, P]),
    "cf_device_kv_seal_full_pages_async": (C.c_int, [P, P]),
    "cf_device_kv_attention_async": (C.c_int, [P, U32, P, P, U32, U32, F32, U32, P]),
    "cf_device_kv_clear_async": (C.c_int, [P, P]),
    "cf_device_kv_get_counters": (C.c_int, [P, P]),
    "cf_device_kv_last_error": (C.c_char_p, [P]),
    "cf_ms_cuda_create": (P, [P]),
    "cf_ms_cuda_destroy": (None, [P, P]),
    "cf_ms_cuda_sequence_create": (C.c_int, [P, I64]),
    "cf_ms_cuda_sequence_remove_async": (C.c_int, [P, I64, P]),
    "cf_ms_cuda_publish_page_async": (C.c_int, [P, P, P]),
    "cf_ms_cuda_stage_active_async": (C.c_int, [P, I64, U32, U32, P, P, U32, P]),
    "cf_ms_cuda_copy_sequence_async": (C.c_int, [P, I64, I64, P]),
    "cf_ms_cuda_shift_sequence": (C.c_int, [P, I64, U32, U32, I32]),
    "cf_ms_cuda_execute_batch_async": (C.c_int, [P, P, U32, P]),
    "cf_ms_cuda_cancel_sequence_async": (C.c_int, [P, I64, P]),
    "cf_ms_cuda_reclaim_async": (C.c_int, [P, P]),
    "cf_ms_cuda_audit": (C.c_int, [P]),
    "cf_ms_cuda_get_counters": (C.c_int, [P, P]),
    "cf_ms_cuda_last_error": (C.c_char_p, [P]),
    "cf_attention_runtime_create": (P, [P]),
    "cf_attention_runtime_destroy": (None, [P, P]),
    "cf_attention_execute_async": (C.c_int, [P, P, U32, P]),
    "cf_attention_compare_async": (C.c_int, [P, P, U32, F32, F32, P]),
    "cf_attention_invalidate_graphs": (C.c_int, [P]),
    "cf_attention_get_counters": (C.c_int, [P, P]),
    "cf_attention_last_error": (C.c_char_p, [P]),
}
for _n, (_r, _a) in _SIGS.items():
    A.declare(_n, _r, _a)


def _stream(stream=None):
    if stream is None:
        return torch.cuda.current_stream().cuda_stream if torch.cuda.is_available() else None
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else stream


def tensor_view(t: torch.Tensor) -> cf_device_tensor_view:
    """View of a [tokens, heads, dim] tensor (any strides) of f16/bf16/f32."""
    if t.dim() != 3 or t.dtype not in _TYPE:
        raise ValueError("expected a 3-d f16/bf16/f32 tensor [tokens, heads, dim]")
    es = t.element_size()
    return cf_device_tensor_view(t.data_ptr(), _TYPE[t.dtype], t.shape[0], t.shape[1], t.shape[2], t.stride(0) * es,
                                 t.stride(1) * es, t.stride(2) * es, t.device.index or 0)


def _out_args(out: torch.Tensor):
    es = out.element_size()
    return out.data_ptr(), _TYPE[out.dtype], out.stride(0) * es, out.stride(1) * es, out.stride(2) * es


class SealEngine:
    """cf_device_seal_engine: stage fp32 active pages, seal them transactionally into int4 nibble pages, attend."""

    def __init__(self, layer_count, kv_heads, q_heads, head_dim, page_size, block_size, gqa=None):
        gqa = q_heads // kv_heads if gqa is None else gqa
        self.config = cf_device_seal_config(layer_count, kv_heads, q_heads, head_dim, page_size, gqa, block_size, 0)
        self.h = A.lib().cf_device_seal_create(C.byref(self.config))
        if not self.h:
            raise SealError("cf_device_seal_create rejected the config")

    def close(self, stream=None):
        if self.h:
            A.lib().cf_device_seal_destroy(self.h, _stream(stream))
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _rc(self, rc, what):
        if rc != 0:
            raise SealError(f"{what}: {A.lib().cf_device_seal_last_error(self.h).decode()}")

    def stage(self, layer, token_begin, k: torch.Tensor, v: torch.Tensor, stream=None):
        self._rc(A.lib().cf_device_seal_stage_active_page(self.h, layer, token_begin, k.data_ptr(), v.data_ptr(),
                                                          k.shape[0], _stream(stream)), "stage")

    def seal(self, layer, stream=None):
        self._rc(A.lib().cf_device_seal_full_page_async(self.h, layer, _stream(stream)), "seal")

    def attention(self, layer, q: torch.Tensor, out: torch.Tensor, query_begin, scale, window=0, stream=None):
        qv = tensor_view(q)
        op, ot, ots, ohs, oes = _out_args(out)
        self._rc(A.lib().cf_device_seal_attention_async(self.h, layer, C.byref(qv), op, ot, ots, ohs, oes, query_begin,
                                                        scale, window, _stream(stream)), "attention")

    def clear(self, stream=None):
        self._rc(A.lib().cf_device_seal_clear_async(self.h, _stream(stream)), "clear")

    def set_fault(self, fault: int) -> int:
        return A.lib().cf_device_seal_set_fault(self.h, fault)

    def state(self, layer) -> int:
        s = C.c_uint32(99)
        self._rc(A.lib().cf_device_seal_get_state(self.h, layer, C.byref(s)), "state")
        return s.value

    def counters(self) -> dict:
        c = cf_device_seal_counters()
        self._rc(A.lib().cf_device_seal_get_counters(self.h, C.byref(c)), "counters")
        return {k: getattr(c, k) for k, _ in c._fields_}

    def pages(self, layer) -> list:
        n = C.c_uint32(0)
        self._rc(A.lib().cf_device_seal_get_pages(self.h, layer, None, 0, C.byref(n)), "pages")
        arr = (cf_device_page_descriptor * max(1, n.value))()
        self._rc(A.lib().cf_device_seal_get_pages(self.h, layer, arr, n.value, C.byref(n)), "pages")
        return [arr[i] for i in range(n.value)]

    def last_error(self) -> str:
        return A.lib().cf_device_seal_last_error(self.h).decode()


class DeviceKv:
    """cf_device_kv_dataplane: append strided f16/bf16/f32 K/V, seal full pages, attend (fp32 query/output)."""

    def __init__(self, layer_count, kv_heads, q_heads, head_dim, page_size, gqa=None):
        gqa = q_heads // kv_heads if gqa is None else gqa
        self.config = cf_device_kv_config(layer_count, kv_heads, q_heads, head_dim, page_size, gqa, 0)
        self.h = A.lib().cf_device_kv_create(C.byref(self.config))
        if not self.h:
            raise SealError("cf_device_kv_create rejected the config")

    def close(self, stream=None):
        if self.h:
            A.lib().cf_device_kv_destroy(self.h, _stream(stream))
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _rc(self, rc, what):
        if rc != 0:
            raise SealError(f"{what}: {A.lib().cf_device_kv_last_error(self.h).decode()}")

    def append(self, layer, token_begin, k: torch.Tensor, v: torch.Tensor, stream=None):
        kv, vv = tensor_view(k), tensor_view(v)
        self._rc(A.lib().cf_device_kv_append_async(self.h, layer, token_begin, C.byref(kv), C.byref(vv),
                                                   _stream(stream)), "append")

    def seal_full_pages(self, stream=None):
        self._rc(A.lib().cf_device_kv_seal_full_pages_async(self.h, _stream(stream)), "seal")

    def attention(self, layer, q: torch.Tensor, out: torch.Tensor, query_begin, scale, window=0, stream=None):
        self._rc(A.lib().cf_device_kv_attention_async(self.h, layer, q.data_ptr(), out.data_ptr(), q.shape[0],
                                                      query_begin, scale, window, _stream(stream)), "attention")

    def clear(self, stream=None):
        self._rc(A.lib().cf_device_kv_clear_async(self.h, _stream(stream)), "clear")

    def counters(self) -> dict:
        c = cf_device_kv_counters()
        self._rc(A.lib().cf_device_kv_get_counters(self.h, C.byref(c)), "counters")
        return {k: getattr(c, k) for k, _ in c._fields_}


class MsResolver:
    """cf_ms_cuda_resolver: sequences over shared, refcounted sealed pages; batched attention."""

    def __init__(self, layer_count, kv_heads, q_heads, head_dim, page_size, gqa=None):
        gqa = q_heads // kv_heads if gqa is None else gqa
        self.config = cf_ms_cuda_config(layer_count, kv_heads, q_heads, head_dim, page_size, gqa, 0)
        self.h = A.lib().cf_ms_cuda_create(C.byref(self.config))
        if not self.h:
            raise SealError("cf_ms_cuda_create rejected the config")

    def close(self, stream=None):
        if self.h:
            A.lib().cf_ms_cuda_destroy(self.h, _stream(stream))
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _rc(self, rc, what):
        if rc != 0:
            raise SealError(f"{what}: {A.lib().cf_ms_cuda_last_error(self.h).decode()}")

    def create(self, seq):
        self._rc(A.lib().cf_ms_cuda_sequence_create(self.h, seq), "sequence_create")

    def remove(self, seq, stream=None):
        self._rc(A.lib().cf_ms_cuda_sequence_remove_async(self.h, seq, _stream(stream)), "sequence_remove")

    def publish(self, seq, layer, desc: cf_device_page_descriptor, seal_generation=0, stream=None):
        pub = cf_ms_page_publication(seq, layer, desc, desc.resident_bytes, seal_generation)
        self._rc(A.lib().cf_ms_cuda_publish_page_async(self.h, C.byref(pub), _stream(stream)), "publish")

    def stage_active(self, seq, layer, token_begin, k: torch.Tensor, v: torch.Tensor, stream=None):
        self._rc(A.lib().cf_ms_cuda_stage_active_async(self.h, seq, layer, token_begin, k.data_ptr(), v.data_ptr(),
                                                       k.shape[0], _stream(stream)), "stage_active")

    def copy(self, src, dst, stream=None):
        self._rc(A.lib().cf_ms_cuda_copy_sequence_async(self.h, src, dst, _stream(stream)), "copy")

    def shift(self, seq, begin, end, delta):
        self._rc(A.lib().cf_ms_cuda_shift_sequence(self.h, seq, begin, end, delta), "shift")

    def execute(self, items: list, stream=None):
        """items: (sequence_id, layer, q [tokens, q_heads, dim], out tensor, query_begin, scale, window)."""
        arr = (cf_ms_batch_item * len(items))()
        for i, (seq, layer, q, out, qb, scale, window) in enumerate(items):
            op, ot, ots, ohs, oes = _out_args(out)
            arr[i] = cf_ms_batch_item(seq, layer, tensor_view(q), op, ot, ots, ohs, oes, qb, scale, window)
        self._rc(A.lib().cf_ms_cuda_execute_batch_async(self.h, arr, len(items), _stream(stream)), "execute_batch")

    def cancel(self, seq, stream=None):
        self._rc(A.lib().cf_ms_cuda_cancel_sequence_async(self.h, seq, _stream(stream)), "cancel")

    def reclaim(self, stream=None):
        self._rc(A.lib().cf_ms_cuda_reclaim_async(self.h, _stream(stream)), "reclaim")

    def audit(self) -> int:
        return A.lib().cf_ms_cuda_audit(self.h)

    def counters(self) -> dict:
        c = cf_ms_cuda_counters()
        self._rc(A.lib().cf_ms_cuda_get_counters(self.h, C.byref(c)), "counters")
        return {k: getattr(c, k) for k, _ in c._fields_}


class AttentionRuntime:
    """cf_attention_runtime: batched decode attention over caller-held two's-complement int4 nibble pages."""

    def __init__(self, layer_count, kv_heads, q_heads, head_dim, gqa=None, page_size=0, block_size=0,
                 mode=CF_ATTENTION_OPTIMIZED):
        gqa = q_heads // kv_heads if gqa is None else gqa
        self.config = cf_attention_runtime_config(layer_count, q_heads, kv_heads, head_dim, page_size, block_size,
                                                  gqa, 0, 0, mode, cf_attention_tuning())
        self.h = A.lib().cf_attention_runtime_create(C.byref(self.config))
        if not self.h:
            raise SealError("cf_attention_runtime_create rejected the config")

    def close(self, stream=None):
        if self.h:
            A.lib().cf_attention_runtime_destroy(self.h, _stream(stream))
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def last_error(self) -> str:
        return A.lib().cf_attention_last_error(self.h).decode()

    def execute_items(self, items, stream=None) -> int:
        """items: a ctypes array of cf_attention_batch_item; returns the library's status (0 / -1)."""
        return A.lib().cf_attention_execute_async(self.h, items, len(items), _stream(stream))

    def execute(self, items, stream=None):
        if self.execute_items(items, stream) != 0:
            raise SealError(f"execute: {self.last_error()}")

    def counters(self) -> dict:
        c = cf_attention_counters()
        if A.lib().cf_attention_get_counters(self.h, C.byref(c)) != 0:
            raise SealError("counters")
        return {k: getattr(c, k) for k, _ in c._fields_}
