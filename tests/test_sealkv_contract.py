"""Host-side contracts of the device seal engine, dataplane and multi-sequence resolver (no device work), and the
pinning of the CPU oracle for the int4 nibble-page format.

The contract cases restate the reference's own contract tests: tests/m9_device_seal_contract.cpp (config checks,
initial state, every fault point settable and one past the last refused, zeroed counters) and
tests/m10_cuda_sequence_resolver_contract.cpp (create, duplicate rejected, empty shift, cancel, audit, counters).

The oracle (oracle/oracle_seal.cpp) is pinned by a hand-computed page, by closed-form properties of the
quantiser (scale = absmax / 7 exactly, the block maximum maps to +-7, error <= scale / 2, the nibble order) and by
comparing its attention with an independent dense softmax over the dequantised values (numpy matrix form, not the
oracle's loop), with causal, window and GQA masks.
"""
import numpy as np
import pytest

import oracle as O
from chromofold_amd import sealkv as S


# ------------------------------------------------------------------------------------------------ seal engine
def test_seal_engine_contract_matches_reference_contract_test():
    e = S.SealEngine(layer_count=2, kv_heads=4, q_heads=8, head_dim=64, page_size=64, block_size=32)
    assert e.state(0) == 0  # CF_SEAL_ACTIVE_FILLING
    for fault in range(11):
        assert e.set_fault(fault) == 0
    assert e.set_fault(11) != 0
    c = e.counters()
    assert c["seal_attempts"] == 0 and c["seal_successes"] == 0
    assert c["descriptor_publications"] == 0 and c["compressed_attention_launches"] == 0
    assert e.pages(0) == [] and e.pages(1) == []
    with pytest.raises(S.SealError):
        e.state(2)
    e.close()


@pytest.mark.parametrize("field,value", [("query_head_count", 7), ("block_size", 0), ("layer_count", 0),
                                         ("page_size", 0), ("head_dim", 12), ("head_dim", 264)])
def test_seal_engine_rejects_bad_configs(field, value):
    import ctypes as C
    from chromofold_amd import _abi as A
    cfg = S.cf_device_seal_config(2, 4, 8, 64, 64, 2, 32, 1)
    setattr(cfg, field, value)
    assert not A.lib().cf_device_seal_create(C.byref(cfg))


def test_seal_on_non_full_page_fails_without_device_work():
    e = S.SealEngine(1, 2, 4, 32, 16, 16)
    with pytest.raises(S.SealError, match="full active page"):
        e.seal(0)
    c = e.counters()
    assert c["seal_attempts"] == 1 and c["seal_failures"] == 1
    e.close()


def test_dataplane_and_resolver_config_checks():
    with pytest.raises(S.SealError):
        S.DeviceKv(1, 4, 7, 64, 64, gqa=2)
    with pytest.raises(S.SealError):
        S.MsResolver(1, 4, 8, 60, 64)  # head_dim not a multiple of 8
    dp = S.DeviceKv(2, 2, 4, 64, 32)
    assert dp.counters()["seal_attempts"] == 0
    dp.close()


def test_tensor_view_validation_rules():
    """reference src/cuda/device_kv_dataplane.cu:111-120"""
    import ctypes as C
    from chromofold_amd import _abi as A
    L = A.lib()

    def view(**kw):
        base = dict(data=0x1000, scalar_type=3, token_count=2, head_count=3, head_dim=8, token_stride_bytes=96,
                    head_stride_bytes=32, element_stride_bytes=4, device_ordinal=0)
        base.update(kw)
        return S.cf_device_tensor_view(**base)

    ok = lambda v: L.cf_device_tensor_validate(C.byref(v))
    assert ok(view()) == 0
    assert ok(view(data=0)) == -1
    assert ok(view(token_count=0)) == -1
    assert ok(view(scalar_type=4)) == -1
    assert ok(view(element_stride_bytes=2)) == -1
    assert ok(view(head_stride_bytes=31)) == -1
    assert ok(view(token_stride_bytes=95)) == -1
    assert ok(view(scalar_type=1, element_stride_bytes=2, head_stride_bytes=16, token_stride_bytes=48)) == 0
    assert L.cf_device_tensor_validate(None) == -1


# ------------------------------------------------------------------------------------------------ resolver
def test_resolver_contract_matches_reference_contract_test():
    r = S.MsResolver(layer_count=2, kv_heads=2, q_heads=4, head_dim=64, page_size=64)
    r.create(101)
    r.create(202)
    with pytest.raises(S.SealError, match="already exists"):
        r.create(101)
    r.shift(101, 0, 0, 0)
    r.cancel(202)
    assert r.audit() == 0
    c = r.counters()
    assert c["cancellation_requests"] == 1
    assert c["dense_fallback_launches"] == 0 and c["cross_sequence_contamination"] == 0
    with pytest.raises(S.SealError):
        r.copy(101, 101)
    with pytest.raises(S.SealError, match="missing"):
        r.copy(999, 5)
    r.close()


def test_resolver_rejects_bad_publications_on_host():
    r = S.MsResolver(1, 2, 4, 64, 64)
    r.create(1)
    d = S.cf_device_page_descriptor()
    with pytest.raises(S.SealError, match="invalid"):
        r.publish(2, 0, d)
    with pytest.raises(S.SealError, match="incomplete"):
        r.publish(1, 0, d)
    d.key_payload = d.value_payload = d.key_scales = d.value_scales = 0x1000
    d.kv_head_count, d.head_dim, d.block_size, d.token_count = 3, 64, 32, 64
    with pytest.raises(S.SealError, match="topology"):
        r.publish(1, 0, d)
    d.kv_head_count = 2
    d.key_payload = 0x1001
    with pytest.raises(S.SealError, match="aligned"):
        r.publish(1, 0, d)
    c = r.counters()
    assert c["page_registration_failures"] == 4 and c["pages_registered"] == 0
    assert r.audit() == 0
    r.close()


# ------------------------------------------------------------------------------------------------ oracle pinning
def test_oracle_seal_hand_computed_page():
    x = np.array([0.7, -1.4, 0.35, 0.0, 2, 2, 2, -2, 0, 0, 0, 0], np.float32)
    payload, scales, sat = O.nib_seal(x, 4)
    # block 0: absmax 1.4 -> scale 0.2; 0.7/0.2 -> 4 (round half to even), -1.4/0.2 = -7, 0.35/0.2 -> 2, 0 -> 0
    # block 1: scale 2/7: +-7; block 2: all zero -> scale 1.0, symbols 8
    assert scales.tolist() == [np.float32(1.4) / np.float32(7), np.float32(2) / np.float32(7), 1.0]
    sym = [4 + 8, -7 + 8, 2 + 8, 8, 15, 15, 15, 1, 8, 8, 8, 8]
    assert payload.tolist() == [sym[2 * i] | (sym[2 * i + 1] << 4) for i in range(6)]
    assert sat == 0


@pytest.mark.parametrize("bs", [1, 5, 16, 32, 33, 128])
def test_oracle_seal_properties(bs):
    rng = np.random.default_rng(bs)
    x = (rng.standard_normal(4096) * rng.choice([1e-3, 1.0, 50.0], 4096)).astype(np.float32)
    x[100:100 + bs] = 0.0  # an all-zero stretch
    payload, scales, sat = O.nib_seal(x, bs)
    nb = (x.size + bs - 1) // bs
    for b in range(nb):
        blk = x[b * bs:(b + 1) * bs]
        amax = np.float32(np.abs(blk).max())
        assert scales[b] == (amax / np.float32(7) if amax > 0 else np.float32(1.0))
    deq = O.nib_dequant(payload, scales, x.size, bs)
    s = scales[np.arange(x.size) // bs].astype(np.float64)
    assert np.all(np.abs(deq - x) <= s / 2 * (1 + 1e-6))
    # the element of largest magnitude of each block decodes to +-7 * scale
    for b in range(nb):
        blk = x[b * bs:(b + 1) * bs]
        i = b * bs + int(np.abs(blk).argmax())
        if blk.any():
            assert abs(deq[i]) == 7 * float(scales[b])
    assert sat == 0


def test_oracle_seal_rejects_non_finite():
    x = np.ones(64, np.float32)
    x[3] = np.nan
    x[9] = np.inf
    with pytest.raises(ValueError, match="1 NaN, 1 Inf"):
        O.nib_seal(x, 32)


def _dense_reference(pages, bs, q, qbegin, kvh, gqa, scale, window, ak=None, av=None, abegin=0):
    """Matrix-form softmax attention over the dequantised keys (independent of the oracle's loops)."""
    qt, qh, D = q.shape
    Ks, Vs, pos = [], [], []
    for p in pages:
        n = p.token_count * kvh * D
        Ks.append(O.nib_dequant(p.k_payload, p.k_scales, n, bs).reshape(p.token_count, kvh, D))
        Vs.append(O.nib_dequant(p.v_payload, p.v_scales, n, bs).reshape(p.token_count, kvh, D))
        pos.append(p.token_begin + np.arange(p.token_count))
    if ak is not None:
        Ks.append(ak.astype(np.float64))
        Vs.append(av.astype(np.float64))
        pos.append(abegin + np.arange(ak.shape[0]))
    K, V, pos = np.concatenate(Ks), np.concatenate(Vs), np.concatenate(pos)
    out = np.zeros((qt, qh, D))
    for t in range(qt):
        P = qbegin + t
        vis = (pos <= P) & ((window == 0) | (pos + window > P))
        for h in range(qh):
            if not vis.any():
                continue
            kk, vv = K[vis, h // gqa], V[vis, h // gqa]
            s = kk @ q[t, h].astype(np.float64) * scale
            w = np.exp(s - s.max())
            out[t, h] = w @ vv / w.sum()
    return out


@pytest.mark.parametrize("kvh,gqa,D,bs,window", [(2, 2, 16, 8, 0), (1, 3, 8, 5, 0), (3, 1, 24, 24, 7),
                                                 (2, 4, 32, 32, 40)])
def test_oracle_attention_equals_dense_softmax(kvh, gqa, D, bs, window):
    rng = np.random.default_rng(D + bs)
    pages = []
    for i, (tb, tc) in enumerate([(0, 16), (16, 16), (40, 9)]):
        k = rng.standard_normal((tc, kvh, D)).astype(np.float32)
        v = rng.standard_normal((tc, kvh, D)).astype(np.float32)
        pages.append(O.nib_seal_page(k, v, tb, bs))
    ak = rng.standard_normal((5, kvh, D)).astype(np.float32)
    av = rng.standard_normal((5, kvh, D)).astype(np.float32)
    q = rng.standard_normal((6, kvh * gqa, D)).astype(np.float32)
    for qbegin in (0, 20, 47):
        got = O.nib_attention(pages, bs, q, qbegin, kvh, gqa, 0.3, window, ak, av, 49)
        exp = _dense_reference(pages, bs, q, qbegin, kvh, gqa, 0.3, window, ak, av, 49)
        np.testing.assert_allclose(got, exp, rtol=1e-5, atol=1e-6)
    # nothing visible (queries before every key) -> zeros
    got = O.nib_attention(pages[2:], bs, q, 0, kvh, gqa, 0.3, window)
    assert not got.any()
