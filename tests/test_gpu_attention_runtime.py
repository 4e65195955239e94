"""GPU parity of the batched attention runtime (cf_attention_execute_async, reference
include/chromofold/production_attention.h, src/cuda/production_attention.cu:59-139) against its float64 CPU
oracle (oracle.rt_attention_f64, pinned in test_attention_runtime.py), through the C ABI.

Pages are two's-complement int4 nibble pages with per-(token, KV head) row blocks written by the oracle's fixture
quantiser; several items per call, each with its own device page table, active fp32 tail, query position, window
(future positions are attended: the contract has no causal bound) and NULL pages. Bars, per (item, query head)
row, max |err| / max |ref|: 2e-5 for fp32 outputs (fp32 accumulation on the VALU), 1e-3 for f16 and 8e-3 for bf16
outputs (their rounding); rows with nothing attended must be exactly zero.
"""

import numpy as np
import pytest

import oracle as O
from kv_helpers import head_err

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _pages(rng, kvh, D, bs, n_pages, page, begin=0, gap=0, amp=1.0):
    out = []
    for p in range(n_pages):
        K = (rng.standard_normal((page, kvh, D)) * amp).astype(np.float32)
        V = (rng.standard_normal((page, kvh, D)) * amp).astype(np.float32)
        kp, ks = O.rt_quantize(K, bs)
        vp, vs = O.rt_quantize(V, bs)
        out.append(O.RtPage(kp, vp, ks, vs, begin + p * (page + gap), page, D, bs))
    return out


class _Dev:
    """Device copies of host pages, page tables and tails; keeps every tensor alive until the call is done."""

    def __init__(self, dev, kvh, shifted=()):
        self.dev, self.kvh, self.keep, self.shifted = dev, kvh, [], set(shifted)

    def tensor(self, a, shift=0):
        """Device copy of `a`; shift = 4 places it 4 bytes into its allocation (4-byte but not 16-byte aligned)."""
        import torch
        if a is None:
            return 0
        a = np.ascontiguousarray(a)
        if a.dtype == np.uint8 and a.size % 4:  # whole 32-bit words for the kernel's loads
            a = np.concatenate([a, np.zeros(4 - a.size % 4, np.uint8)])
        if shift:
            a = np.concatenate([np.zeros(shift, np.uint8), a.view(np.uint8).reshape(-1)])
        t = torch.from_numpy(a).to(self.dev)
        self.keep.append(t)
        return t.data_ptr() + shift

    def table(self, pages):
        import torch
        from chromofold_amd import sealkv as S
        if not pages:
            return 0
        descs = (S.cf_device_page_descriptor * len(pages))()
        for i, p in enumerate(pages):
            d = descs[i]
            sh = 4 if i in self.shifted else 0
            d.key_payload, d.value_payload = self.tensor(p.k_payload, sh), self.tensor(p.v_payload, sh)
            d.key_scales, d.value_scales = self.tensor(p.k_scales), self.tensor(p.v_scales)
            d.token_begin, d.token_count, d.kv_head_count = p.token_begin, p.token_count, self.kvh
            d.head_dim, d.block_size = p.head_dim, p.block_size
        t = torch.frombuffer(bytearray(descs), dtype=torch.uint8).to(self.dev)
        self.keep.append(t)
        return t.data_ptr()


def _item(D_, i, q, out, qpos, scale, window, pages, ak=None, av=None, abegin=0):
    from chromofold_amd import sealkv as S
    it = S.cf_attention_batch_item()
    it.sequence_id, it.layer = 100 + i, 0
    qes = q.element_size()
    it.query = S.cf_device_tensor_view(q.data_ptr(), S._TYPE[q.dtype], 1, q.shape[0], q.shape[1], 0,
                                       q.stride(0) * qes, q.stride(1) * qes, 0)
    oes = out.element_size()
    it.output, it.output_type = out.data_ptr(), S._TYPE[out.dtype]
    it.output_token_stride_bytes, it.output_head_stride_bytes = 0, out.stride(0) * oes
    it.output_element_stride_bytes = out.stride(1) * oes
    it.query_token_begin, it.softmax_scale, it.causal_window = qpos, scale, window
    it.sealed_pages, it.sealed_page_count = D_.table(pages), len(pages)
    if ak is not None:
        it.active_keys, it.active_values = D_.tensor(ak), D_.tensor(av)
        it.active_token_begin, it.active_token_count = abegin, ak.shape[0]
    return it


def _run(dev, kvh, gqa, D, specs, q_dtype=None, out_dtype=None, layout="contiguous", shifted=()):
    """specs: list of (pages, qpos, window, active_k, active_v, active_begin). Returns (got [items, qh, D],
    ref [items, qh, D]) with got in float64."""
    import torch
    from chromofold_amd import sealkv as S
    q_dtype = q_dtype or torch.float32
    out_dtype = out_dtype or torch.float32
    qh = kvh * gqa
    rt = S.AttentionRuntime(1, kvh, qh, D, gqa=gqa, page_size=32, block_size=32)
    D_ = _Dev(dev, kvh, shifted)
    rng = np.random.default_rng(D * 7 + len(specs))
    items = (S.cf_attention_batch_item * len(specs))()
    outs, refs = [], []
    for i, (pages, qpos, window, ak, av, abegin) in enumerate(specs):
        qf = rng.standard_normal((qh, D)).astype(np.float32)
        if layout == "contiguous":
            q = torch.from_numpy(qf).to(dev).to(q_dtype)
            out = torch.full((qh, D), float("nan"), device=dev, dtype=out_dtype)
        else:  # [D, qh] storage read through transposed strides
            q = torch.from_numpy(np.ascontiguousarray(qf.T)).to(dev).to(q_dtype).t()
            out = torch.full((D, qh), float("nan"), device=dev, dtype=out_dtype).t()
        outs.append(out)
        D_.keep.append(q)
        items[i] = _item(D_, i, q, out, qpos, 0.125 if D >= 64 else 0.25, window, pages, ak, av, abegin)
        qv = q.float().cpu().numpy()  # the values the kernel reads
        refs.append(O.rt_attention_f64(qv, kvh, gqa, qpos, window, items[i].softmax_scale, pages, ak, av, abegin))
    rt.execute(items)
    torch.cuda.synchronize()
    got = np.stack([o.double().cpu().numpy() for o in outs])
    counters = rt.counters()
    rt.close()
    return got, np.stack(refs), counters


def test_batch_of_items_matches_oracle(dev):
    kvh, gqa, D, bs = 2, 4, 64, 32
    rng = np.random.default_rng(5)
    pa = _pages(rng, kvh, D, bs, 6, 16)
    pb = _pages(rng, kvh, D, bs, 3, 32, begin=40, gap=8, amp=3.0)
    ak = rng.standard_normal((7, kvh, D)).astype(np.float32)
    av = rng.standard_normal((7, kvh, D)).astype(np.float32)
    holed = list(pa)
    holed[2] = O.RtPage(None, pa[2].v_payload, pa[2].k_scales, pa[2].v_scales, pa[2].token_begin, 16, D, bs)
    specs = [
        (pa, 200, 0, ak, av, 96),       # every page and the tail
        (pa, 40, 0, ak, av, 96),        # query inside the pages: later positions attended too
        (pa, 60, 17, None, None, 0),    # window bound p + 17 >= 60 falls inside a page
        (holed, 90, 0, ak, av, 96),     # a page with a NULL payload is skipped
        (pb, 500, 3, None, None, 0),    # nothing within the window (every p + 3 < 500): zeros
        ([], 5, 0, ak, av, 0),          # the tail only
        ([], 5, 0, None, None, 0),      # nothing at all: zeros
        (pb + pa, 150, 64, ak, av, 120),
    ]
    got, ref, c = _run(dev, kvh, gqa, D, specs)
    assert np.isfinite(got).all()
    assert not got[4].any() and not got[6].any()
    assert head_err(got, ref) <= 2e-5
    assert c["optimized_launches"] == 1 and c["grouped_items"] == len(specs) and c["cuda_errors"] == 0


@pytest.mark.parametrize("D,bs", [(40, 16), (64, 24), (64, 7), (128, 64), (32, 8)])
def test_row_blocks_and_block_sizes(dev, D, bs):
    """Blocks that do not divide head_dim (per-row block index differs from the flat one), block sizes that are
    not a multiple of 8 (value-by-value path) and ones that are (whole-word path)."""
    kvh, gqa = 3, 2
    rng = np.random.default_rng(D * bs)
    pages = _pages(rng, kvh, D, bs, 5, 24)
    specs = [(pages, 119, 0, None, None, 0), (pages, 50, 30, None, None, 0)]
    got, ref, _ = _run(dev, kvh, gqa, D, specs)
    assert head_err(got, ref) <= 2e-5


@pytest.mark.parametrize("q_dtype,out_dtype,tol", [("float16", "float32", 2e-5), ("bfloat16", "bfloat16", 8e-3),
                                                   ("float32", "float16", 1e-3)])
def test_dtypes_and_strided_views(dev, q_dtype, out_dtype, tol):
    import torch
    kvh, gqa, D, bs = 2, 2, 128, 32
    rng = np.random.default_rng(17)
    pages = _pages(rng, kvh, D, bs, 4, 32)
    ak = rng.standard_normal((5, kvh, D)).astype(np.float32)
    av = rng.standard_normal((5, kvh, D)).astype(np.float32)
    specs = [(pages, 130, 0, ak, av, 128), (pages, 64, 40, ak, av, 128)]
    got, ref, _ = _run(dev, kvh, gqa, D, specs, getattr(torch, q_dtype), getattr(torch, out_dtype), "transposed")
    assert head_err(got, ref) <= tol


def test_long_context_gqa8_with_splits(dev):
    """One KV head serving 8 query heads (two groups of 4 per lane) over 96 pages: the call splits the pages."""
    kvh, gqa, D, bs = 1, 8, 128, 64
    rng = np.random.default_rng(23)
    pages = _pages(rng, kvh, D, bs, 96, 32)
    ak = rng.standard_normal((11, kvh, D)).astype(np.float32)
    av = rng.standard_normal((11, kvh, D)).astype(np.float32)
    specs = [(pages, 3083, 0, ak, av, 3072), (pages, 1500, 700, ak, av, 3072), (pages[:10], 319, 0, None, None, 0)]
    got, ref, _ = _run(dev, kvh, gqa, D, specs)
    assert head_err(got, ref) <= 2e-5


def test_invalid_item_fails_the_call_before_any_launch(dev):
    import torch
    from chromofold_amd import sealkv as S
    kvh, gqa, D = 2, 2, 64
    rt = S.AttentionRuntime(1, kvh, kvh * gqa, D)
    D_ = _Dev(dev, kvh)
    q = torch.zeros((kvh * gqa, D), device=dev)
    out = torch.full_like(q, 7.0)
    items = (S.cf_attention_batch_item * 2)()
    items[0] = _item(D_, 0, q, out, 0, 1.0, 0, [])
    items[1] = _item(D_, 1, q, out, 0, 1.0, 0, [])
    items[1].sealed_page_count = 3  # pages counted but no table
    assert rt.execute_items(items) == -1 and "page table" in rt.last_error()
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())  # nothing ran
    c = rt.counters()
    assert c["optimized_launches"] == 0 and c["cuda_errors"] == 0
    items[1].sealed_page_count = 0
    rt.execute(items)
    torch.cuda.synchronize()
    assert not out.any()  # nothing attended: zeros
    assert rt.counters()["optimized_launches"] == 1
    rt.close()


def test_matrix_core_and_valu_pages_in_one_request(dev):
    """head_dim 128 requests run on the matrix-core kernel for every page whose block size is a multiple of 32,
    whose payloads are 16-byte aligned and which holds at most the runtime's page size (32 tokens); the VALU kernel
    takes the others (block sizes 16 and 48, a 40-token page, a payload 4 bytes off 16-byte alignment, NULL
    pages) out of the same page table. Every page must count exactly once: one request over all of them, others
    over subsets, windows cutting through both kinds, against the float64 oracle."""
    kvh, gqa, D = 2, 4, 128
    rng = np.random.default_rng(31)
    pages, begin = [], 0
    for bs, n, tok in ((32, 3, 32), (16, 2, 32), (64, 2, 24), (48, 2, 32), (128, 2, 32), (256, 1, 16), (32, 1, 40),
                       (96, 2, 32)):
        pages += _pages(rng, kvh, D, bs, n, tok, begin=begin)
        begin += n * tok
    p0 = pages[0]
    null_page = O.RtPage(p0.k_payload, p0.v_payload, None, p0.v_scales, begin, 32, D, 32)
    pages.append(null_page)
    shifted = [1, 6]  # page 1 (block size 32) and page 6 (block size 128) start 4 bytes into their allocations
    ak = rng.standard_normal((6, kvh, D)).astype(np.float32)
    av = rng.standard_normal((6, kvh, D)).astype(np.float32)
    specs = [
        (pages, begin + 40, 0, ak, av, begin + 32),
        (pages, 200, 90, None, None, 0),          # window from position 110: both kinds on either side
        (pages[::-1], 400, 0, ak, av, begin + 32),  # table order does not matter
        (pages[3:9], 150, 0, None, None, 0),
    ]
    got, ref, c = _run(dev, kvh, gqa, D, specs, shifted=shifted)
    assert np.isfinite(got).all()
    assert head_err(got, ref) <= 2e-5
    assert c["optimized_launches"] == 1 and c["cuda_errors"] == 0


@pytest.mark.parametrize("kvh", [5, 6])
def test_refused_pages_reach_every_wave(dev, kvh):
    """With 5 or 6 KV heads of 16 lanes each (head_dim 128) the VALU kernel's workgroup is 80 or 96 threads: its
    second wave has 16 or 32 lanes, fewer than the 64 pages one split tests. Pages the matrix cores refuse
    (block sizes 16 and 48) sit at table indices 16 and above, so the second wave's KV heads must learn of them
    from the first wave's test, not from their own lanes."""
    gqa, D = 2, 128
    rng = np.random.default_rng(40 + kvh)
    pages, begin = [], 0
    for bs, n in ((32, 16), (16, 3), (32, 10), (48, 4), (64, 8), (16, 2)):
        pages += _pages(rng, kvh, D, bs, n, 32, begin=begin)
        begin += n * 32
    assert len(pages) == 43
    specs = [(pages, begin + 5, 0, None, None, 0), (pages[::-1], 900, 300, None, None, 0)]
    got, ref, c = _run(dev, kvh, gqa, D, specs)
    assert np.isfinite(got).all()
    assert head_err(got, ref) <= 2e-5
    assert c["optimized_launches"] == 1 and c["cuda_errors"] == 0
