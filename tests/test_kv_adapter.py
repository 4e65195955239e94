"""llama.cpp adapter on the CPU (no device work happens before a page is sealed), mirroring reference
tests/llama_kv_adapter_seam.cpp:7-44, and the fixed-width page encoder the adapter seals with, bit-identical to the
oracle's restatement of the reference fixture encoder (and to the reference's own code where oracle/_ref is built)."""
import ctypes as C

import numpy as np
import pytest

import oracle as O


def test_adapter_seam_contract():
    from chromofold_amd import llama as Lm
    L = Lm.A.lib()
    dense = Lm.options(0, 0, 0, 0, 0, 0, backend=Lm.BACKEND_DENSE)
    assert L.cf_llama_kv_options_validate(C.byref(dense)) == 0
    assert not L.cf_llama_kv_create(C.byref(dense))
    o = Lm.options(2, 2, 8, 64, 128, 4)
    assert L.cf_llama_kv_options_validate(C.byref(o)) == 0
    a = Lm.KvAdapter(o)
    st = a.stats()
    assert st.appended_tokens == 0 and st.sealed_pages == 0
    assert L.cf_llama_kv_seq_shift(a.h, 0, 0) == 0
    assert L.cf_llama_kv_seq_cp(a.h, 0, 1) != 0
    assert "shared-page" in a.last_error()
    assert L.cf_llama_kv_clear(a.h) == 0
    assert L.cf_llama_kv_seq_rm(a.h, 0) == 0
    assert L.cf_llama_kv_seq_rm(a.h, 3) != 0
    assert L.cf_llama_kv_seq_shift(a.h, 0, 2) != 0
    a.close()
    o.query_head_count = 7
    assert L.cf_llama_kv_options_validate(C.byref(o)) != 0
    bad = Lm.options(1, 1, 1, 64, 16, 1)
    bad.struct_size = 8
    assert L.cf_llama_kv_options_validate(C.byref(bad)) != 0
    assert L.cf_llama_kv_get_stats(None, None) == -1
    assert L.cf_llama_kv_last_error(None) == b"invalid ChromoFold KV adapter"


def test_adapter_append_contract_on_host():
    """Tail bookkeeping before any page seals: contiguity, ranges, stats (no device needed)."""
    from chromofold_amd import llama as Lm
    a = Lm.KvAdapter(Lm.options(1, 2, 4, 32, 16, 2))
    x = np.ones((3, 32), np.float32)
    a.append(0, 0, 5, x, x)
    with pytest.raises(Lm.CfAdapterError, match="contiguous"):
        a.append(0, 0, 9, x, x)
    with pytest.raises(Lm.CfAdapterError, match="out of range"):
        a.append(1, 0, 0, x, x)
    a.append(0, 0, 8, x, x)
    st = a.stats()
    assert st.appended_tokens == 6 and st.active_tokens == 6 and st.sealed_pages == 0
    assert st.dense_active_bytes == 2 * 6 * 32 * 4


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("T,D", [(16, 64), (32, 128), (5, 96), (70, 32)])
def test_fixed_page_encoder_matches_oracle_and_reference(bits, T, D):
    from chromofold_amd import llama as Lm
    rng = np.random.default_rng(bits + T + D)
    k = (rng.standard_normal((T, D)) * 2).astype(np.float32)
    v = rng.standard_normal((T, D)).astype(np.float32)
    k[:, 3] = 0.0
    v[1] = 0.0
    kw, vw, ks, vs, bo = Lm.encode_fixed_page(bits, k, v)
    ksym, vsym, oks, ovs, _, _ = O.kv_fixture_quantize(k, v, bits)
    assert np.array_equal(ks, oks) and np.array_equal(vs, ovs)
    assert np.array_equal(kw, O.pack_fixed(ksym, bits)) and np.array_equal(vw, O.pack_fixed(vsym, bits))
    assert np.array_equal(bo, (np.arange(0, T * D, 64) * bits).astype(np.int32))
    if O.ref_lib() is not None:
        ref = O.ref_fixture_page(bits, k, v)
        assert np.array_equal(kw, ref["kw"]) and np.array_equal(vw, ref["vw"]) and np.array_equal(bo, ref["kboff"])


def test_fixed_page_encoder_rejects_non_finite():
    from chromofold_amd import llama as Lm
    k = np.ones((4, 8), np.float32)
    k[1, 1] = np.inf
    with pytest.raises(Lm.A.CfError):
        Lm.encode_fixed_page(4, k, np.ones((4, 8), np.float32))
