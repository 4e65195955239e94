"""CPU tests of the host-side KV runtime (kv_runtime.h) and of the seam's host validation (kv_cuda.h), mirroring
the reference's tests/kv_runtime_test.cpp:49-140 and tests/paged_kv_cuda_seam.cu (fake device pointers: these
entry points must never dereference device memory)."""
import ctypes as C
import math

import numpy as np
import pytest

from chromofold_amd import _abi as A
from chromofold_amd import legacy as Lg

FAKE = 0x1000


def _page(begin, count, layer=0, head=0):
    p = Lg.cf_kv_page_view()
    p.struct_size = C.sizeof(Lg.cf_kv_page_view)
    p.abi_version = Lg.CF_KV_RUNTIME_ABI_VERSION
    p.flags = Lg.CF_KV_PAGE_FLAG_SEALED | Lg.CF_KV_PAGE_FLAG_DEVICE_RESIDENT
    p.layer, p.kv_head, p.token_begin, p.token_count, p.head_dim, p.block_size = layer, head, begin, count, 4, 4
    p.k_words, p.k_word_count, p.k_block_offsets, p.k_block_count = FAKE, 3, FAKE, count
    p.k_lut, p.k_lut_count, p.k_scales, p.k_scale_count = FAKE, 8, FAKE, 4
    p.v_words, p.v_word_count, p.v_block_offsets, p.v_block_count = FAKE, 4, FAKE, count
    p.v_lut, p.v_lut_count, p.v_scales, p.v_scale_count = FAKE, 8, FAKE, count
    return p


def test_struct_sizes_match_reference_abi():
    # measured with gcc x86-64 on the reference headers (cf_kv_device_page 104, desc 96, page view 168, layout 72,
    # wavelet view 48, rrrw view 96, fm view 144)
    assert C.sizeof(A.cf_kv_device_page) == 104 and A.cf_kv_device_page.fixed_code_length.offset == 96
    assert C.sizeof(A.cf_kv_paged_attention_desc) == 96
    assert C.sizeof(Lg.cf_kv_page_view) == 168 and C.sizeof(Lg.cf_kv_cache_layout) == 72
    assert C.sizeof(A.cf_wavelet_view) == 48 and C.sizeof(A.cf_rrrw_view) == 96 and C.sizeof(A.cf_fm_view) == 144


def test_page_validation_and_accounting():
    L = A.lib()
    p = _page(0, 4)
    assert L.cf_kv_validate_page(C.byref(p)) == A.CF_OK
    b = C.c_uint64()
    assert L.cf_kv_page_resident_bytes(C.byref(p), C.byref(b)) == A.CF_OK
    assert b.value == (3 + 4) * 4 + (4 + 4 + 8 + 8) * 4 + (4 + 4) * 4
    for field, val in [("v_scale_count", 3), ("flags", 0), ("head_dim", 129), ("block_size", 0),
                       ("k_block_count", 3), ("struct_size", 8), ("abi_version", 1), ("k_words", None)]:
        q = _page(0, 4)
        setattr(q, field, val)
        if field == "head_dim":
            q.k_scale_count = 129
        assert L.cf_kv_validate_page(C.byref(q)) == A.CF_ERR_INVALID_ARGUMENT, field
    q = _page(0xFFFFFFFE, 4)  # token range overflows u32
    assert L.cf_kv_validate_page(C.byref(q)) == A.CF_ERR_INVALID_ARGUMENT
    assert L.cf_kv_page_resident_bytes(C.byref(p), None) == A.CF_ERR_INVALID_ARGUMENT


def test_layout_and_overlap_detection():
    L = A.lib()
    pages = (Lg.cf_kv_page_view * 2)(_page(0, 4), _page(4, 4))
    ly = Lg.cf_kv_cache_layout()
    ly.struct_size, ly.abi_version = C.sizeof(ly), 0
    ly.layer_count, ly.kv_head_count, ly.head_dim, ly.page_capacity_tokens = 1, 1, 4, 4
    ly.active_token_begin, ly.active_token_count, ly.active_element_bytes = 8, 2, 2
    ly.pages, ly.page_count = C.addressof(pages), 2
    ly.active_k_bytes = ly.active_v_bytes = 2 * 1 * 1 * 4 * 2
    assert L.cf_kv_validate_layout(C.byref(ly)) == A.CF_OK
    st = Lg.cf_kv_memory_stats()
    assert L.cf_kv_cache_memory_stats(C.byref(ly), C.byref(st)) == A.CF_OK
    assert (st.page_count, st.sealed_tokens, st.active_tokens) == (2, 8, 2)
    assert st.active_payload_bytes == ly.active_k_bytes + ly.active_v_bytes
    assert st.total_resident_bytes == st.sealed_payload_bytes + st.sealed_descriptor_bytes + st.active_payload_bytes
    assert st.sealed_descriptor_bytes == 2 * C.sizeof(Lg.cf_kv_page_view)
    pages[1].token_begin = 3  # overlap
    assert L.cf_kv_validate_layout(C.byref(ly)) == A.CF_ERR_INVALID_ARGUMENT
    pages[1].token_begin = 4
    ly.active_k_bytes = 1
    assert L.cf_kv_validate_layout(C.byref(ly)) == A.CF_ERR_INVALID_ARGUMENT
    ly.active_k_bytes = 16
    pages[1].kv_head = 1  # head out of range
    assert L.cf_kv_validate_layout(C.byref(ly)) == A.CF_ERR_INVALID_ARGUMENT


def test_online_softmax_page_merge():
    """Two partial states (pages) merged == one state over all scores == dense fp64 softmax, including extreme
    scores (-1000 / 900) that overflow a naive exp (reference kv_runtime_test.cpp:97-140)."""
    L = A.lib()
    scores = [-1000.0, -2.0, 3.0, 2.5, 900.0, 899.0]
    values = [[1, 0, 0, 0], [0, 1, 0, 0], [0, 0, 1, 0], [0, 0, 0, 1], [1, 2, 3, 4], [4, 3, 2, 1]]
    bufs = [(C.c_double * 4)() for _ in range(3)]
    states = [Lg.cf_online_softmax_state() for _ in range(3)]
    for s, b in zip(states, bufs):
        assert L.cf_online_softmax_init(C.byref(s), b, 4) == A.CF_OK
    vals = [(C.c_float * 4)(*v) for v in values]
    for i in range(6):
        assert L.cf_online_softmax_accumulate(C.byref(states[0 if i < 3 else 1]), scores[i], vals[i]) == A.CF_OK
        assert L.cf_online_softmax_accumulate(C.byref(states[2]), scores[i], vals[i]) == A.CF_OK
    assert L.cf_online_softmax_merge(C.byref(states[0]), C.byref(states[1])) == A.CF_OK
    m = max(scores)
    w = np.array([math.exp(s - m) for s in scores])
    dense = (w[:, None] * np.array(values, float)).sum(0) / w.sum()
    for s in (states[0], states[2]):
        out = (C.c_float * 4)()
        assert L.cf_online_softmax_finalize(C.byref(s), out) == A.CF_OK
        assert np.allclose(np.array(out[:]), dense, rtol=1e-6, atol=1e-7)
    empty = Lg.cf_online_softmax_state()
    eb = (C.c_double * 4)()
    assert L.cf_online_softmax_init(C.byref(empty), eb, 4) == A.CF_OK
    out = (C.c_float * 4)()
    assert L.cf_online_softmax_finalize(C.byref(empty), out) == A.CF_ERR_INVALID_ARGUMENT  # nothing accumulated
    assert L.cf_online_softmax_merge(C.byref(states[0]), C.byref(empty)) == A.CF_OK       # empty src: no-op
    assert L.cf_online_softmax_accumulate(C.byref(empty), float("inf"), vals[0]) == A.CF_ERR_INVALID_ARGUMENT
    assert L.cf_online_softmax_init(C.byref(empty), eb, 129) == A.CF_ERR_INVALID_ARGUMENT


def _desc():
    d = A.cf_kv_paged_attention_desc()
    d.struct_size, d.abi_version = C.sizeof(d), 0
    d.pages, d.page_count = FAKE, 3
    d.kv_head_count, d.query_head_count, d.gqa_group_size = 2, 14, 7
    d.queries, d.output = FAKE, FAKE
    d.query_token_begin, d.query_count, d.head_dim, d.softmax_scale = 10, 1, 64, 0.125
    return d


def test_seam_validation_rules():
    """cf_kv_validate_paged_attention_desc rules (reference paged_kv_attention.cu:280-299); the async entry point
    must reject the same descriptors before any device call (fake pointers, no GPU needed)."""
    L = A.lib()
    assert L.cf_kv_validate_paged_attention_desc(C.byref(_desc())) == A.CF_OK
    assert L.cf_kv_validate_paged_attention_desc(None) == A.CF_ERR_INVALID_ARGUMENT
    bad = [("struct_size", 95), ("abi_version", 1), ("queries", None), ("output", None), ("query_count", 0),
           ("query_head_count", 0), ("kv_head_count", 0), ("gqa_group_size", 0), ("head_dim", 0), ("head_dim", 129),
           ("softmax_scale", float("nan")), ("softmax_scale", float("inf")), ("query_head_count", 13),
           ("page_count", 4097), ("pages", None), ("active_token_count", 3), ("query_token_begin", 0xFFFFFFFF)]
    for field, val in bad:
        d = _desc()
        setattr(d, field, val)
        assert L.cf_kv_validate_paged_attention_desc(C.byref(d)) == A.CF_ERR_INVALID_ARGUMENT, (field, val)
        assert L.cf_kv_paged_attention_async(C.byref(d), None) == A.CF_ERR_INVALID_ARGUMENT, (field, val)
    d = _desc()
    d.page_count, d.pages = 0, None  # no pages at all is valid (tail-only attention)
    assert L.cf_kv_validate_paged_attention_desc(C.byref(d)) == A.CF_OK
    d = _desc()
    d.active_token_count, d.active_k, d.active_v, d.active_token_begin = 2, FAKE, FAKE, 0xFFFFFFFE
    assert L.cf_kv_validate_paged_attention_desc(C.byref(d)) == A.CF_ERR_INVALID_ARGUMENT
