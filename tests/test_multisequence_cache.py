"""Host bookkeeping cache cf_multisequence_* (CPU only: it holds no KV data).

The first two tests replay the reference's own contract tests call for call (tests/m10_multisequence_contract.cpp,
tests/m10_multisequence_host_contract.cpp). The rest pin the semantics of reference src/multisequence_cache.cpp:
contiguous appends inside one active page, suffix-only removal of the active range, shifts, speculative commit /
rollback against the baseline, ranged copy of the active range, and the refusal of attention (no dense fallback).
The active range is observed through the append contiguity rule (an append must start at begin + count).
Rejected removals / shifts / commits must leave the sequence unchanged (validated over all layers first).
"""
import ctypes as C

import pytest

from chromofold_amd import sealkv as S

L = S.A.lib()


def _cache(**kw):
    c = S.MultiSequenceCache(kw.get("layers", 2), 2, 4, 64, kw.get("page", 64))
    return c, c.h


def _view(tokens, heads=2, dim=64, data=0x1000):
    return S.cf_device_tensor_view(data, S.CF_DEVICE_F16, tokens, heads, dim, heads * dim * 2, dim * 2, 2, 0)


def _append(h, seq, layer, begin, n):
    k = _view(n)
    return L.cf_sequence_append_async(h, seq, layer, begin, C.byref(k), C.byref(k), None)


def test_reference_contract_m10():
    c, h = _cache()
    assert L.cf_sequence_create(h, 10) == 0
    assert L.cf_sequence_create(h, 11) == 0
    assert L.cf_sequence_create(h, 10) != 0
    assert L.cf_multisequence_audit(h) == 0
    spec = L.cf_sequence_speculation_begin(h, 10)
    assert spec != 0
    assert L.cf_sequence_speculation_rollback(h, 10, spec, None) == 0
    assert L.cf_sequence_shift_async(h, 10, 0, 0, 0, None) == 0
    assert L.cf_sequence_copy_async(h, 10, 12, 0, 0, None) == 0
    assert L.cf_multisequence_audit(h) == 0
    assert L.cf_sequence_remove_async(h, 11, -1, -1, None) == 0
    assert L.cf_multisequence_reclaim_async(h, None) == 0
    assert L.cf_multisequence_audit(h) == 0
    n = c.counters()
    assert n["sequences_created"] == 2 and n["sequences_copied"] == 1
    assert n["speculative_transactions_started"] == 1 and n["speculative_transactions_rolled_back"] == 1
    assert n["dense_fallback_launches"] == 0 and n["invariant_failures"] == 0
    c.close()


def test_reference_host_contract_m10():
    c, h = _cache()
    assert L.cf_sequence_create(h, 10) == 0 and L.cf_sequence_create(h, 11) == 0
    assert L.cf_sequence_create(h, 10) != 0
    t = L.cf_sequence_speculation_begin(h, 10)
    assert t != 0
    assert L.cf_sequence_speculation_rollback(h, 10, t, None) == 0
    assert L.cf_sequence_copy_async(h, 10, 12, 0, 0, None) == 0
    assert L.cf_sequence_remove_async(h, 11, -1, -1, None) == 0
    assert L.cf_multisequence_reclaim_async(h, None) == 0
    assert L.cf_multisequence_audit(h) == 0
    n = c.counters()
    assert (n["sequences_created"], n["sequences_copied"]) == (2, 1)
    assert n["active_sequences"] == 2 and n["active_sequences_peak"] == 3
    c.close()


def test_config_and_null_checks():
    with pytest.raises(S.SealError):
        S.MultiSequenceCache(1, 2, 5, 64, 64, gqa=2)
    with pytest.raises(S.SealError):
        S.MultiSequenceCache(0, 2, 4, 64, 64)
    assert not L.cf_multisequence_create(None)
    assert L.cf_sequence_create(None, 1) == -1
    assert L.cf_sequence_speculation_begin(None, 1) == 0
    assert L.cf_multisequence_audit(None) == -1
    assert L.cf_multisequence_last_error(None) == b"null multisequence cache"
    c, h = _cache()
    assert L.cf_sequence_copy_async(h, 1, 1, 0, 10, None) == -1  # same id
    assert L.cf_sequence_copy_async(h, 1, 2, 10, 0, None) == -1  # end < begin
    assert L.cf_sequence_copy_async(h, 1, 2, 0, 10, None) == -1
    assert c.last_error() == "source sequence does not exist"
    assert L.cf_sequence_remove_async(h, 1, 5, 4, None) == -1
    c.close()


def test_appends_fill_one_active_page_contiguously():
    c, h = _cache(page=16)
    assert L.cf_sequence_create(h, 1) == 0
    assert _append(h, 1, 0, 100, 10) == 0
    assert _append(h, 1, 0, 111, 1) == -1 and c.last_error() == "non-contiguous sequence append"
    assert _append(h, 1, 0, 110, 7) == -1 and c.last_error() == "append crosses sequence active-page boundary"
    assert _append(h, 1, 0, 110, 6) == 0  # fills the page (16 tokens)
    assert _append(h, 1, 1, 5, 3) == 0  # layers are independent
    bad = _view(2, heads=3)
    assert L.cf_sequence_append_async(h, 1, 0, 116, C.byref(bad), C.byref(bad), None) == -1
    assert c.last_error() == "append tensor topology mismatch"
    assert _append(h, 1, 2, 0, 1) == -1  # layer out of range
    null = _view(1, data=0)
    assert L.cf_sequence_append_async(h, 1, 0, 116, C.byref(null), C.byref(null), None) == -1
    assert _append(h, 9, 0, 0, 1) == -1 and c.last_error() == "sequence does not exist"
    assert L.cf_multisequence_audit(h) == 0
    c.close()


def test_remove_active_suffix_and_reject_non_suffix_without_change():
    c, h = _cache()
    assert L.cf_sequence_create(h, 1) == 0
    assert _append(h, 1, 0, 100, 10) == 0 and _append(h, 1, 1, 100, 10) == 0
    assert L.cf_sequence_remove_async(h, 1, 105, 200, None) == 0  # suffix [105, 110) of both layers
    assert _append(h, 1, 0, 110, 1) == -1
    assert _append(h, 1, 0, 105, 1) == 0  # layer 0 now [100, 106)
    before = c.counters()["unsupported_operations"]
    assert L.cf_sequence_remove_async(h, 1, 0, 103, None) == -1
    assert c.last_error() == "non-suffix active-tail removal is not supported"
    assert c.counters()["unsupported_operations"] == before + 1
    assert _append(h, 1, 1, 105, 1) == 0  # layer 1 unchanged: still [100, 105)
    assert L.cf_sequence_remove_async(h, 1, -5, 1000, None) == 0  # begin < 0 -> 0: everything
    assert _append(h, 1, 0, 7, 1) == 0  # empty active range: any start
    assert L.cf_sequence_remove_async(h, 1, -1, -1, None) == 0
    assert L.cf_sequence_remove_async(h, 1, -1, -1, None) == -1
    n = c.counters()
    assert n["sequences_removed"] == 3 and n["active_sequences"] == 0
    c.close()


def test_shift_moves_the_active_range_and_rejects_negative_positions_atomically():
    c, h = _cache()
    assert L.cf_sequence_create(h, 1) == 0
    assert _append(h, 1, 0, 100, 5) == 0 and _append(h, 1, 1, 10, 5) == 0
    assert L.cf_sequence_shift_async(h, 1, 100, 200, -50, None) == 0  # layer 0 only (layer 1 outside)
    assert _append(h, 1, 0, 55, 1) == 0 and _append(h, 1, 1, 15, 1) == 0
    # layer 1's range [10, 16) would go negative: nothing moves, not even layer 0's [50, 56)
    assert L.cf_sequence_shift_async(h, 1, 0, 100, -20, None) == -1
    assert c.last_error() == "context shift produces negative active position"
    assert _append(h, 1, 0, 56, 1) == 0 and _append(h, 1, 1, 16, 1) == 0
    assert c.counters()["sequences_shifted"] == 1
    assert L.cf_sequence_shift_async(h, 2, 0, 1, 1, None) == -1
    assert L.cf_sequence_shift_async(h, 1, 5, 4, 1, None) == -1
    c.close()


def test_speculation_commit_and_rollback():
    c, h = _cache()
    assert L.cf_sequence_create(h, 1) == 0
    assert _append(h, 1, 0, 0, 5) == 0 and _append(h, 1, 1, 0, 5) == 0
    s = L.cf_sequence_speculation_begin(h, 1)  # baseline 5
    assert s != 0 and L.cf_sequence_speculation_begin(h, 1) == 0
    assert c.last_error() == "speculation already active"
    assert _append(h, 1, 0, 5, 4) == 0 and _append(h, 1, 1, 5, 3) == 0  # provisional 4 and 3
    assert L.cf_sequence_speculation_commit(h, 1, s, 4, None) == -1  # layer 1 has only 3
    assert c.last_error() == "accepted token count exceeds provisional tail"
    assert L.cf_sequence_speculation_commit(h, 1, s + 1, 1, None) == -1
    assert c.last_error() == "invalid speculative transaction"
    assert L.cf_sequence_speculation_commit(h, 1, s, 2, None) == 0  # both layers -> 7 tokens
    assert _append(h, 1, 0, 7, 1) == 0 and _append(h, 1, 1, 7, 1) == 0
    s2 = L.cf_sequence_speculation_begin(h, 1)  # baseline 8
    assert _append(h, 1, 0, 8, 2) == 0
    assert L.cf_sequence_speculation_rollback(h, 1, s2, None) == 0
    assert _append(h, 1, 0, 8, 1) == 0  # back to 8 tokens
    assert L.cf_sequence_speculation_rollback(h, 1, s2, None) == -1
    n = c.counters()
    assert (n["speculative_transactions_started"], n["speculative_transactions_committed"],
            n["speculative_transactions_rolled_back"]) == (2, 1, 1)
    c.close()


def test_ranged_copy_takes_the_active_range_only_when_inside():
    c, h = _cache()
    assert L.cf_sequence_create(h, 1) == 0
    assert _append(h, 1, 0, 50, 7) == 0
    assert L.cf_sequence_copy_async(h, 1, 2, 0, 100, None) == 0
    assert _append(h, 2, 0, 57, 1) == 0 and _append(h, 2, 0, 0, 1) == -1
    assert L.cf_sequence_copy_async(h, 1, 3, 0, 52, None) == 0  # active [50, 57) not inside [0, 52)
    assert _append(h, 3, 0, 0, 1) == 0
    assert L.cf_sequence_copy_async(h, 1, 3, 0, 100, None) == 0  # replaces 3
    assert _append(h, 3, 0, 57, 1) == 0
    assert c.counters()["sequences_copied"] == 3 and L.cf_multisequence_audit(h) == 0
    c.close()


def test_attention_validates_then_refuses_without_dense_fallback():
    c, h = _cache()
    assert L.cf_sequence_create(h, 1) == 0
    item = S.cf_sequence_attention_item(1, 0, _view(1, heads=4), 0x2000, S.CF_DEVICE_F32, 1024, 256, 4, 0, 0.1, 0)
    assert L.cf_multisequence_attention_async(h, C.byref(item), 1, None) == -1
    assert "cf_ms_cuda_execute_batch_async" in c.last_error()
    bad = S.cf_sequence_attention_item(7, 0, _view(1, heads=4), 0x2000, S.CF_DEVICE_F32, 1024, 256, 4, 0, 0.1, 0)
    assert L.cf_multisequence_attention_async(h, C.byref(bad), 1, None) == -1
    assert c.last_error() == "attention item references unknown sequence"
    item.output = None
    assert L.cf_multisequence_attention_async(h, C.byref(item), 1, None) == -1
    assert c.last_error() == "invalid sequence attention item"
    assert L.cf_multisequence_attention_async(h, C.byref(item), 0, None) == -1
    n = c.counters()
    assert n["batches_dispatched"] == 1 and n["sequences_per_batch_peak"] == 1 and n["dense_fallback_launches"] == 0
    c.close()
