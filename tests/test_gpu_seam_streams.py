"""The reference seam cf_kv_paged_attention_async called from several streams at once, and under graph capture.

The reference seam keeps no state across calls, so its callers may overlap calls on different streams with no
ordering of their own (reference include/chromofold/kv_cuda.h:82-83: the caller owns only its own buffers' stream
dependencies). This build's seam splits long contexts and keeps the split partials in library-owned device regions;
these tests check that calls overlapping on different streams never see each other's partials: two different
descriptors (different head_dim, page codecs and query positions) alternate over six non-blocking streams, more
streams than the library has regions (so the last streams first run unsplit, then take regions over behind event
waits), with no host synchronisation between the calls; and two host threads each launch on their own per-thread
default stream (the same handle, hipStreamPerThread, for two different streams). Every output must match the same
descriptor's output from a serial run within 1e-5 absolute (a call that runs unsplit sums in another order, a few
ulps away; partials mixed in from the other descriptor would be off by ~1e-2), and the float64 oracle within the
reference tests' 2e-4 absolute bar. A call captured into a HIP graph runs unsplit (a capture cannot wait for an event recorded outside
it); its replays, with other seam calls between them, must match the oracle too."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from legacy_helpers import fixed_page, huffman_page, rans_page

pytestmark = pytest.mark.gpu
ABS_TOL = 2e-4
SERIAL_TOL = 1e-5


@pytest.fixture(scope="module")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _context(rng, hd, T, kinds, kvh=2, P=32):
    pages, deq = [], []
    for p0 in range(0, T, P):
        for h in range(kvh):
            k = rng.standard_normal((P, hd)).astype(np.float32)
            v = rng.standard_normal((P, hd)).astype(np.float32)
            kind = kinds[(p0 // P + h) % len(kinds)]
            if kind == "rans":
                page, kd, vd = rans_page(k, v, h, p0)
            elif kind == "huff":
                page, kd, vd = huffman_page(k, v, h, p0)
            else:
                page, kd, vd = fixed_page(k, v, h, p0, kind)
            pages.append(page)
            deq.append((h, p0, kd, vd))
    return pages, deq


class _Case:
    """One seam descriptor (64 query rows x GQA 7 over 2 KV heads: 14 (tile, head) units, so the context is split
    over many workgroups) with its float64 reference."""

    def __init__(self, dev, seed, hd, T, kinds, qtok0):
        import torch
        from chromofold_amd.legacy import PagedKv
        rng = np.random.default_rng(seed)
        self.kvh, self.gqa, self.hd, self.qtok0 = 2, 7, hd, qtok0
        pages, deq = _context(rng, hd, T, kinds)
        self.pk = PagedKv(pages, str(dev))
        self.q_host = rng.standard_normal((64, self.kvh * self.gqa, hd)).astype(np.float32)
        self.q = torch.from_numpy(self.q_host).to(dev)
        self.scale = 1 / np.sqrt(hd)
        self.ref = np.zeros_like(self.q_host)
        for r in range(self.q_host.shape[0]):
            self.ref[r], _ = O.paged_attention_f64(self.q_host[r], self.q_host.shape[1], self.kvh, hd, self.gqa,
                                                   qtok0 + r, 0, self.scale, deq, None)

    def launch(self, out, stream_handle):
        from chromofold_amd import _abi as A
        d = self.pk.desc(self.q, out, self.kvh, self.gqa, self.qtok0, self.scale)
        A.check(A.lib().cf_kv_paged_attention_async(C.byref(d), stream_handle), "cf_kv_paged_attention_async")


def test_overlapping_calls_on_six_streams(dev):
    import torch
    a = _Case(dev, 11, 128, 4096, (4, "rans", 8, "huff"), 4096 - 64)
    b = _Case(dev, 12, 64, 3072, (8, 4, "huff"), 3072 - 80)
    # serial outputs on the current stream
    serial = {}
    for name, c in (("a", a), ("b", b)):
        out = torch.full_like(c.q, float("nan"))
        c.launch(out, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        serial[name] = out.cpu().numpy()
        assert np.isfinite(serial[name]).all()
        assert np.abs(serial[name] - c.ref).max() <= ABS_TOL
    streams = [torch.cuda.Stream(device=dev) for _ in range(6)]
    n = 36  # six rounds over the six streams
    outs = [torch.full_like(a.q if i % 2 == 0 else b.q, float("nan")) for i in range(n)]
    torch.cuda.synchronize()  # outputs filled; nothing below synchronises until every call is queued
    for i in range(n):
        (a if i % 2 == 0 else b).launch(outs[i], streams[i % 6].cuda_stream)
    torch.cuda.synchronize()
    for i, out in enumerate(outs):
        c, name = (a, "a") if i % 2 == 0 else (b, "b")
        got = out.cpu().numpy()
        assert np.abs(got - serial[name]).max() <= SERIAL_TOL, f"call {i} (descriptor {name}) vs the serial run"
        assert np.abs(got - c.ref).max() <= ABS_TOL


def test_graph_captured_call_runs_unsplit(dev):
    import torch
    a = _Case(dev, 21, 128, 2048, (4, "rans"), 2048 - 64)
    b = _Case(dev, 22, 64, 2048, (8,), 2048 - 64)
    out = torch.full_like(a.q, float("nan"))
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        a.launch(out, torch.cuda.current_stream().cuda_stream)
    other = torch.full_like(b.q, float("nan"))
    for rep in range(3):
        out.fill_(float("nan"))
        g.replay()
        b.launch(other, torch.cuda.current_stream().cuda_stream)  # eager split call between the replays
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        assert np.isfinite(got).all(), f"replay {rep}"
        assert np.abs(got - a.ref).max() <= ABS_TOL, f"replay {rep}"
        assert np.abs(other.cpu().numpy() - b.ref).max() <= ABS_TOL, f"replay {rep}"


def test_per_thread_default_streams_from_two_threads(dev):
    """hipStreamPerThread ((hipStream_t)2) names a different stream in each host thread: two threads launching on
    it at once (ctypes releases the GIL during the call) must not share split partials."""
    import threading
    import torch
    a = _Case(dev, 31, 128, 4096, (4, 8), 4096 - 64)
    b = _Case(dev, 32, 64, 4096, ("rans", 4), 4096 - 64)
    serial = {}
    for name, c in (("a", a), ("b", b)):
        out = torch.full_like(c.q, float("nan"))
        c.launch(out, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        serial[name] = out.cpu().numpy()
    outs = {"a": [torch.full_like(a.q, float("nan")) for _ in range(8)],
            "b": [torch.full_like(b.q, float("nan")) for _ in range(8)]}
    torch.cuda.synchronize()
    errors = []

    def work(c, lst):
        try:
            torch.cuda.set_device(dev)
            for o in lst:
                c.launch(o, 2)  # hipStreamPerThread
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(e)

    ts = [threading.Thread(target=work, args=(a, outs["a"])), threading.Thread(target=work, args=(b, outs["b"]))]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    torch.cuda.synchronize()  # device-wide: both threads' per-thread streams
    assert not errors, errors
    for name, c in (("a", a), ("b", b)):
        for i, o in enumerate(outs[name]):
            got = o.cpu().numpy()
            assert np.abs(got - serial[name]).max() <= SERIAL_TOL, f"{name} call {i} vs the serial run"
            assert np.abs(got - c.ref).max() <= ABS_TOL
