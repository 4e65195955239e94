"""GPU parity of the int4 nibble-page path: the device seal engine (cf_device_seal_*), the device KV dataplane
(cf_device_kv_*) and the multi-sequence resolver (cf_ms_cuda_*), all through the C ABI.

- sealed pages: payload and scale bytes bit-exact against the oracle's quantiser (oracle/oracle_seal.cpp, which
  restates reference src/cuda/device_kv_seal_attention.cu:72-113);
- attention: against the oracle's float64 attention over the same pages (reference :116-187 semantics: causal,
  window, GQA, active page), tolerance rtol 1e-3 / atol 1e-4 for an fp32 output (fp32 accumulation on the GPU),
  widened only by the output dtype's own rounding for f16 / bf16 outputs;
- the transaction: every fault point rolls the layer back to ACTIVE_FULL with nothing published, a NaN/Inf page
  is rejected, a later seal succeeds with the same bytes;
- resolver: shared pages after copy, per-sequence active pages, one batched launch over decode and prefill items
  of several sequences, shift, cancel, remove/reclaim and audit.
"""
import ctypes as C

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

_hip = None


def _d2h(ptr: int, nbytes: int) -> np.ndarray:
    global _hip
    if _hip is None:
        _hip = C.CDLL("libamdhip64.so")
        _hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        _hip.hipMemcpy.restype = C.c_int
    out = np.empty(nbytes, np.uint8)
    assert _hip.hipMemcpy(out.ctypes.data, ptr, nbytes, 2) == 0  # hipMemcpyDeviceToHost
    return out


@pytest.fixture(scope="module")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _t(a, dev, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t if dtype is None else t.to(dtype)


def _page_bytes(desc, values, bs):
    nb = (values + bs - 1) // bs
    kp = _d2h(desc.key_payload, (values + 1) // 2)
    vp = _d2h(desc.value_payload, (values + 1) // 2)
    ks = _d2h(desc.key_scales, nb * 4).view(np.float32)
    vs = _d2h(desc.value_scales, nb * 4).view(np.float32)
    return kp, vp, ks, vs


def _tol(dtype):
    import torch
    return {torch.float32: (1e-3, 1e-4), torch.float16: (2e-3, 1e-3), torch.bfloat16: (1e-2, 8e-3)}[dtype]


def _run_engine_case(dev, kvh, gqa, D, page, bs, seed):
    import torch
    from chromofold_amd.sealkv import SealEngine
    rng = np.random.default_rng(seed)
    e = SealEngine(2, kvh, kvh * gqa, D, page, bs)
    ref_pages = []
    layer = 1
    for p in range(3):
        k = (rng.standard_normal((page, kvh, D)) * rng.choice([0.5, 2.0, 30.0])).astype(np.float32)
        v = rng.standard_normal((page, kvh, D)).astype(np.float32)
        e.stage(layer, p * page, _t(k, dev), _t(v, dev))
        assert e.state(layer) == 1
        e.seal(layer)
        assert e.state(layer) == 0
        ref_pages.append(O.nib_seal_page(k, v, p * page, bs))
    torch.cuda.synchronize()
    descs = e.pages(layer)
    assert len(descs) == 3 and e.pages(0) == []
    values = page * kvh * D
    for d, r in zip(descs, ref_pages):
        kp, vp, ks, vs = _page_bytes(d, values, bs)
        assert np.array_equal(kp, r.k_payload) and np.array_equal(vp, r.v_payload)
        assert np.array_equal(ks, r.k_scales) and np.array_equal(vs, r.v_scales)
        assert (d.token_begin, d.token_count, d.kv_head_count, d.head_dim, d.block_size) == (
            r.token_begin, page, kvh, D, bs)
    # a partial active page after the sealed ones
    na = page // 2 + 1
    ak = rng.standard_normal((na, kvh, D)).astype(np.float32)
    av = rng.standard_normal((na, kvh, D)).astype(np.float32)
    e.stage(layer, 3 * page, _t(ak, dev), _t(av, dev))
    last = 3 * page + na - 1
    return e, ref_pages, ak, av, last, rng


@pytest.mark.parametrize("kvh,gqa,D,page,bs", [(4, 2, 64, 64, 32), (2, 7, 128, 16, 128), (1, 1, 32, 8, 12),
                                               (8, 4, 128, 32, 64), (2, 8, 256, 16, 32), (3, 3, 96, 8, 24),
                                               (2, 4, 16, 32, 5), (1, 16, 64, 16, 64),
                                               # head_dim 128 with block 32 / 64 / 128k: the MFMA kernel reads the
                                               # pages (partial 16-token chunks, pages across tiles, several tiles
                                               # per page, a block spanning two rows)
                                               (4, 4, 128, 8, 32), (2, 4, 128, 48, 64), (1, 2, 128, 128, 256),
                                               (8, 1, 128, 64, 128), (2, 3, 128, 16, 32)])
def test_seal_engine_bytes_and_attention(dev, kvh, gqa, D, page, bs):
    import torch
    print(f"case kvh={kvh} gqa={gqa} D={D} page={page} bs={bs}", flush=True)
    e, pages, ak, av, last, rng = _run_engine_case(dev, kvh, gqa, D, page, bs, seed=D * 7 + bs)
    qh = kvh * gqa
    scale = 1.0 / np.sqrt(D)
    cases = [(1, last, 0, torch.float32), (5, last - 4, 0, torch.float32), (3, 2 * page + 1, 0, torch.float16),
             (2, last - 1, page // 2 + 3, torch.bfloat16), (1, page - 1, 0, torch.float32)]
    for qt, qbegin, window, dt in cases:
        q = rng.standard_normal((qt, qh, D)).astype(np.float32)
        qd = _t(q, dev, dt)
        out = torch.full((qt, qh, D), float("nan"), dtype=dt, device=dev)
        e.attention(1, qd, out, qbegin, scale, window)
        torch.cuda.synchronize()
        ref = O.nib_attention(pages, bs, qd.float().cpu().numpy(), qbegin, kvh, gqa, scale, window, ak, av, 3 * page)
        rtol, atol = _tol(dt)
        np.testing.assert_allclose(out.float().cpu().numpy(), ref, rtol=rtol, atol=atol,
                                   err_msg=f"qt={qt} qbegin={qbegin} window={window} {dt}")
    c = e.counters()
    assert c["seal_successes"] == 3 and c["compressed_attention_launches"] == len(cases)
    assert c["finite_validation_launches"] == 3 and c["quantization_launches"] == 3
    e.close()


@pytest.mark.parametrize("bs,gqa", [(32, 4), (128, 8)])
def test_seal_engine_long_context_many_splits(dev, bs, gqa):
    """96 pages x 64 tokens: many tiles per wavefront, several context splits, decode and a short prefill."""
    import torch
    from chromofold_amd.sealkv import SealEngine
    kvh, D, page = 2, 128, 64
    rng = np.random.default_rng(bs + gqa)
    e = SealEngine(1, kvh, kvh * gqa, D, page, bs)
    pages = []
    for p in range(96):
        k = rng.standard_normal((page, kvh, D)).astype(np.float32)
        v = rng.standard_normal((page, kvh, D)).astype(np.float32)
        e.stage(0, p * page, _t(k, dev), _t(v, dev))
        e.seal(0)
        pages.append(O.nib_seal_page(k, v, p * page, bs))
    total = 96 * page
    for qt, qbegin, window in [(1, total - 1, 0), (3, total - 3, 0), (1, total - 1, 1000), (2, 4000, 0)]:
        q = rng.standard_normal((qt, kvh * gqa, D)).astype(np.float32)
        out = torch.full((qt, kvh * gqa, D), float("nan"), device=dev)
        e.attention(0, _t(q, dev), out, qbegin, 1 / np.sqrt(D), window)
        torch.cuda.synchronize()
        ref = O.nib_attention(pages, bs, q, qbegin, kvh, gqa, 1 / np.sqrt(D), window)
        np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=1e-3, atol=1e-4, err_msg=f"{qt} {qbegin} {window}")
    e.close()


def test_seal_engine_strided_query_and_output(dev):
    """Query and output as non-contiguous views (padded rows, strided elements)."""
    import torch
    e, pages, ak, av, last, rng = _run_engine_case(dev, 2, 4, 64, 16, 32, seed=5)
    qh, D, qt = 8, 64, 3
    qbuf = _t(rng.standard_normal((qt, qh + 1, D * 2)).astype(np.float32), dev)
    q = qbuf[:, 1:, ::2]  # [qt, qh, D], element stride 8 B, padded head and token strides
    obuf = torch.zeros((qt, qh, D + 24), dtype=torch.float16, device=dev)
    out = obuf[:, :, 5:5 + D]
    e.attention(1, q, out, last - 2, 0.125)
    torch.cuda.synchronize()
    ref = O.nib_attention(pages, 32, q.cpu().numpy(), last - 2, 2, 4, 0.125, 0, ak, av, 48)
    np.testing.assert_allclose(out.float().cpu().numpy(), ref, rtol=2e-3, atol=1e-3)
    e.close()


def test_seal_engine_no_visible_key_gives_zero_and_empty_layer(dev):
    import torch
    from chromofold_amd.sealkv import SealEngine
    e = SealEngine(1, 2, 4, 32, 8, 16)
    q = torch.randn(2, 4, 32, device=dev)
    out = torch.full((2, 4, 32), 7.0, device=dev)
    e.attention(0, q, out, 0, 0.2)  # nothing sealed, no active page
    torch.cuda.synchronize()
    assert not out.any()
    k = torch.randn(8, 2, 32, device=dev)
    e.stage(0, 100, k, k)
    e.attention(0, q, out, 50, 0.2)  # queries before every key
    torch.cuda.synchronize()
    assert not out.any()
    e.close()


def test_seal_faults_roll_back_and_nan_pages_are_rejected(dev):
    import torch
    from chromofold_amd.sealkv import SealEngine, SealError
    e = SealEngine(1, 2, 4, 64, 16, 32)
    rng = np.random.default_rng(3)
    k = rng.standard_normal((16, 2, 64)).astype(np.float32)
    v = rng.standard_normal((16, 2, 64)).astype(np.float32)
    e.stage(0, 0, _t(k, dev), _t(v, dev))
    for fault in range(1, 11):
        assert e.set_fault(fault) == 0
        with pytest.raises(SealError, match="injected"):
            e.seal(0)
        assert e.state(0) == 1 and e.pages(0) == []
    assert e.set_fault(0) == 0
    bad = k.copy()
    bad[3, 1, 7] = np.nan
    bad[9, 0, 0] = -np.inf
    e.stage(0, 0, _t(bad, dev), _t(v, dev))
    with pytest.raises(SealError, match="NaN or Inf"):
        e.seal(0)
    assert e.state(0) == 1 and e.pages(0) == []
    e.stage(0, 0, _t(k, dev), _t(v, dev))
    e.seal(0)
    torch.cuda.synchronize()
    (d,) = e.pages(0)
    r = O.nib_seal_page(k, v, 0, 32)
    kp, vp, ks, vs = _page_bytes(d, 16 * 2 * 64, 32)
    assert np.array_equal(kp, r.k_payload) and np.array_equal(vp, r.v_payload)
    assert np.array_equal(ks, r.k_scales) and np.array_equal(vs, r.v_scales)
    c = e.counters()
    assert c["seal_failures"] == 11 and c["seal_successes"] == 1
    assert c["nan_values"] == 1 and c["inf_values"] == 1 and c["invalid_pages_rejected"] == 1
    # clear returns the layer to an empty state; sealing again works
    e.clear()
    assert e.pages(0) == [] and e.state(0) == 0
    e.stage(0, 0, _t(k, dev), _t(v, dev))
    e.seal(0)
    torch.cuda.synchronize()
    (d2,) = e.pages(0)
    kp2, _, _, _ = _page_bytes(d2, 16 * 2 * 64, 32)
    assert np.array_equal(kp2, r.k_payload)
    e.close()


def test_dataplane_append_seal_attend(dev):
    import torch
    from chromofold_amd.sealkv import DeviceKv, SealError
    kvh, gqa, D, page = 2, 3, 64, 16
    dp = DeviceKv(2, kvh, kvh * gqa, D, page)
    rng = np.random.default_rng(11)
    total = 2 * page + 5
    K = rng.standard_normal((total, kvh, D)).astype(np.float32)
    V = rng.standard_normal((total, kvh, D)).astype(np.float32)
    # appends in chunks, as bf16 through a padded (non-contiguous) view, then f16, then f32
    t = 0
    for n, dt in [(6, torch.bfloat16), (10, torch.float16), (16, torch.float32), (5, torch.bfloat16)]:
        pad = np.zeros((n, kvh, D + 8), np.float32)
        pad[:, :, 3:3 + D] = K[t:t + n]
        kk = _t(pad, dev, dt)[:, :, 3:3 + D]
        vv = _t(V[t:t + n], dev, dt)
        dp.append(0, t, kk, vv)
        K[t:t + n] = kk.float().cpu().numpy()
        V[t:t + n] = vv.float().cpu().numpy()
        t += n
        if t % page == 0:
            with pytest.raises(SealError, match="crosses"):
                dp.append(0, t, kk[:1], vv[:1])
            dp.seal_full_pages()
    with pytest.raises(SealError, match="non-contiguous"):
        dp.append(0, t + 1, kk[:1], vv[:1])
    q = rng.standard_normal((4, kvh * gqa, D)).astype(np.float32)
    out = torch.zeros((4, kvh * gqa, D), device=dev)
    dp.attention(0, _t(q, dev), out, total - 4, 0.1)
    torch.cuda.synchronize()
    pages = [O.nib_seal_page(K[p * page:(p + 1) * page], V[p * page:(p + 1) * page], p * page, 32) for p in range(2)]
    ref = O.nib_attention(pages, 32, q, total - 4, kvh, gqa, 0.1, 0, K[2 * page:], V[2 * page:], 2 * page)
    np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=1e-3, atol=1e-4)
    c = dp.counters()
    assert c["seal_successes"] == 2 and c["device_append_calls"] == 4
    # K and V are counted separately, as in reference src/cuda/device_kv_dataplane.cu:163-180
    assert c["bf16_values_converted"] == 2 * 11 * kvh * D and c["fp16_values_converted"] == 2 * 10 * kvh * D
    dp.clear()
    dp.close()


def test_resolver_shared_pages_batched_attention(dev):
    import torch
    from chromofold_amd.sealkv import MsResolver, SealEngine, SealError
    kvh, gqa, D, page, bs = 2, 4, 128, 16, 32
    qh = kvh * gqa
    rng = np.random.default_rng(21)
    eng = SealEngine(1, kvh, qh, D, page, bs)
    ref_pages = []
    for p in range(4):
        k = rng.standard_normal((page, kvh, D)).astype(np.float32)
        v = rng.standard_normal((page, kvh, D)).astype(np.float32)
        eng.stage(0, p * page, _t(k, dev), _t(v, dev))
        eng.seal(0)
        ref_pages.append(O.nib_seal_page(k, v, p * page, bs))
    descs = eng.pages(0)
    r = MsResolver(1, kvh, qh, D, page)
    r.create(1)
    for d in descs[:3]:
        r.publish(1, 0, d)
    tail1 = rng.standard_normal((2, 5, kvh, D)).astype(np.float32)
    r.stage_active(1, 0, 3 * page, _t(tail1[0], dev), _t(tail1[1], dev))
    r.copy(1, 2)  # shares the three pages, copies the tail
    tail2 = rng.standard_normal((2, 7, kvh, D)).astype(np.float32)
    r.stage_active(2, 0, 3 * page, _t(tail2[0], dev), _t(tail2[1], dev))  # seq 2 diverges
    r.create(3)
    r.publish(3, 0, descs[3])  # a page sealed at position 3 * page, seen alone by sequence 3
    assert r.audit() == 0
    # one batch: decode items of 1 and 2, a prefill item of 3, a windowed decode of 1
    specs = [(1, 3 * page + 4, 1, 0, torch.float32), (2, 3 * page + 6, 1, 0, torch.float16),
             (3, 4 * page - 4, 4, 0, torch.float32), (1, 3 * page + 4, 1, 9, torch.bfloat16)]
    items, refs = [], []
    for seq, qbegin, qt, window, dt in specs:
        q = _t(rng.standard_normal((qt, qh, D)).astype(np.float32), dev, dt)
        out = torch.full((qt, qh, D), float("nan"), dtype=dt, device=dev)
        items.append((seq, 0, q, out, qbegin, 0.09, window))
        qn = q.float().cpu().numpy()
        if seq == 1:
            ref = O.nib_attention(ref_pages[:3], bs, qn, qbegin, kvh, gqa, 0.09, window, tail1[0], tail1[1], 3 * page)
        elif seq == 2:
            ref = O.nib_attention(ref_pages[:3], bs, qn, qbegin, kvh, gqa, 0.09, window, tail2[0], tail2[1], 3 * page)
        else:
            ref = O.nib_attention(ref_pages[3:], bs, qn, qbegin, kvh, gqa, 0.09, window)
        refs.append((out, ref, dt))
    r.execute(items)
    torch.cuda.synchronize()
    for (out, ref, dt), spec in zip(refs, specs):
        rtol, atol = _tol(dt)
        np.testing.assert_allclose(out.float().cpu().numpy(), ref, rtol=rtol, atol=atol, err_msg=str(spec))
    c = r.counters()
    assert c["sequence_attention_launches"] == 1 and c["decode_items"] == 3 and c["prefill_items"] == 1
    assert c["copy_on_write_tail_copies"] == 1 and c["pages_registered"] == 4
    assert c["in_flight_page_references"] == 3 + 3 + 1 + 3
    r.reclaim()
    assert r.counters()["in_flight_page_references"] == 0
    # shift sequence 3's page by -2 * page: positions move, attention follows
    r.shift(3, 3 * page, 4 * page, -2 * page)
    q = _t(rng.standard_normal((1, qh, D)).astype(np.float32), dev)
    out = torch.zeros((1, qh, D), device=dev)
    r.execute([(3, 0, q, out, 2 * page - 1, 0.09, 0)])
    torch.cuda.synchronize()
    moved = O.NibPage(ref_pages[3].k_payload, ref_pages[3].v_payload, ref_pages[3].k_scales, ref_pages[3].v_scales,
                      page, page)
    ref = O.nib_attention([moved], bs, q.cpu().numpy(), 2 * page - 1, kvh, gqa, 0.09)
    np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=1e-3, atol=1e-4)
    with pytest.raises(SealError, match="immutable"):
        r.shift(3, page + 1, 2 * page, 1)
    with pytest.raises(SealError, match="negative"):
        r.shift(3, 0, 4 * page, -5 * page)
    # cancel: no more dispatch
    r.cancel(3)
    with pytest.raises(SealError, match="unavailable"):
        r.execute([(3, 0, q, out, 2 * page - 1, 0.09, 0)])
    # remove 1: its pages stay (shared with 2); remove 2: they retire; reclaim frees them
    r.remove(1)
    assert r.counters()["pages_retired"] == 0
    r.remove(2)
    c = r.counters()
    assert c["pages_retired"] == 3 and c["pending_reclamation_bytes"] == 3 * descs[0].resident_bytes
    torch.cuda.synchronize()
    r.reclaim()
    c = r.counters()
    assert c["pages_reclaimed"] == 3 and c["pending_reclamation_bytes"] == 0
    assert r.audit() == 0
    r.close()
    eng.close()


def test_resolver_copy_onto_existing_destination_releases_old_references(dev):
    from chromofold_amd.sealkv import MsResolver, SealEngine
    import torch
    eng = SealEngine(1, 1, 2, 32, 8, 16)
    k = torch.randn(8, 1, 32, device=dev)
    for p in range(2):
        eng.stage(0, 8 * p, k, k)
        eng.seal(0)
    d = eng.pages(0)
    r = MsResolver(1, 1, 2, 32, 8)
    r.create(1)
    r.create(2)
    r.publish(1, 0, d[0])
    r.publish(2, 0, d[1])
    r.copy(1, 2)  # sequence 2's own page loses its only reference
    c = r.counters()
    assert c["pages_retired"] == 1
    assert r.audit() == 0
    torch.cuda.synchronize()
    r.reclaim()
    assert r.counters()["pages_reclaimed"] == 1
    r.close()
    eng.close()
