"""GPU parity of the reference seam cf_kv_paged_attention_async on reference-format pages.

Mirrors the reference's GPU tests: tests/paged_kv_cuda_correctness.cu (single int4 page, smooth data, max abs
error <= 2e-4 against a CPU attention over the encoder's dequantised values), tests/adapter_attention_test.cu
(head_dim {32, 64, 96, 128} x {int4, int8}, 2 KV heads, 14 query heads, 70 tokens = sealed pages + dense active
tail, seed 9001) and tests/kv_reference_test.cpp (page-order invariance, GQA + tail, empty visible set -> 0).
Huffman-coded pages (variable-length codes, rows starting mid-block) exercise the LUT decoder the reference's
warp kernel cannot take. Reference = fp64 oracle over the same dequantised values."""
import numpy as np
import pytest

import oracle as O
from legacy_helpers import fixed_page, huffman_page

pytestmark = pytest.mark.gpu
ABS_TOL = 2e-4


@pytest.fixture(scope="module")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _run(dev, pages_deq, host_pages, q, kv_heads, gqa, qtok0, scale, window=0, tail=None):
    import torch
    from chromofold_amd.legacy import PagedKv
    pk = PagedKv(host_pages, str(dev))
    dq = torch.from_numpy(q).to(dev)
    active = None
    if tail is not None:
        active = (tail[0], torch.from_numpy(tail[1]).to(dev), torch.from_numpy(tail[2]).to(dev))
    got = pk.attention(dq, kv_heads, gqa, qtok0, scale, window, active).cpu().numpy()
    ref = np.zeros_like(q)
    for r in range(q.shape[0]):
        ref[r], _ = O.paged_attention_f64(q[r], q.shape[1], kv_heads, q.shape[2], gqa, qtok0 + r, window, scale,
                                          pages_deq, tail)
    return got, ref


def test_single_int4_page_smooth_data(dev):
    """reference tests/paged_kv_cuda_correctness.cu: 128 tokens x 64 dims, one page, int4."""
    T, D = 128, 64
    t = np.arange(T, dtype=np.float32)[:, None]
    d = np.arange(D, dtype=np.float32)[None, :]
    k = (np.sin(0.03 * t + 0.11 * d) + 0.25 * np.cos(0.07 * d)).astype(np.float32)
    v = (np.cos(0.05 * t - 0.13 * d) * 0.8).astype(np.float32)
    page, kd, vd = fixed_page(k, v, 0, 0, 4)
    q = np.random.default_rng(1).standard_normal((4, 1, D)).astype(np.float32)
    got, ref = _run(dev, [(0, 0, kd, vd)], [page], q, 1, 1, T - 4, 1 / np.sqrt(D))
    assert np.abs(got - ref).max() <= ABS_TOL


@pytest.mark.parametrize("hd", [32, 64, 96, 128])
@pytest.mark.parametrize("bits", [4, 8])
def test_adapter_matrix_pages_plus_tail(dev, hd, bits):
    """reference tests/adapter_attention_test.cu:22-111: kvh 2, qh 14 (gqa 7), 70 tokens -> 2 sealed 32-token
    pages per head + a 6-token dense fp32 tail, several query rows."""
    rng = np.random.default_rng(9001)
    kvh, gqa, N, P = 2, 7, 70, 32
    K = rng.standard_normal((kvh, N, hd)).astype(np.float32)
    V = rng.standard_normal((kvh, N, hd)).astype(np.float32)
    pages, deq = [], []
    for h in range(kvh):
        for p0 in range(0, (N // P) * P, P):
            page, kd, vd = fixed_page(K[h, p0:p0 + P], V[h, p0:p0 + P], h, p0, bits)
            pages.append(page)
            deq.append((h, p0, kd, vd))
    t0 = (N // P) * P
    tail = (t0, np.ascontiguousarray(K[:, t0:].transpose(1, 0, 2)), np.ascontiguousarray(V[:, t0:].transpose(1, 0, 2)))
    q = rng.standard_normal((3, kvh * gqa, hd)).astype(np.float32)
    got, ref = _run(dev, deq, pages, q, kvh, gqa, N - 3, 1 / np.sqrt(hd), tail=tail)
    assert np.abs(got - ref).max() <= ABS_TOL, np.abs(got - ref).max()


@pytest.mark.parametrize("hd,maxlen", [(96, 12), (128, 16), (64, 9)])
def test_huffman_pages_mid_block_rows(dev, hd, maxlen):
    """Variable-length (canonical Huffman) pages: rows of 96 dims start mid-way through 64-symbol blocks, so the
    decoder must skip-decode from the block offsets; maxlen 16 exercises the LUT-in-HBM path."""
    rng = np.random.default_rng(hd + maxlen)
    kvh, gqa, T = 2, 4, 96
    pages, deq = [], []
    for h in range(kvh):
        for p0 in (0, 40):
            n = 40 if p0 == 0 else 56
            k = (rng.standard_normal((n, hd)) ** 3).astype(np.float32)  # peaky -> short codes for small values
            v = rng.standard_normal((n, hd)).astype(np.float32)
            page, kd, vd = huffman_page(k, v, h, p0, 8, maxlen)
            pages.append(page)
            deq.append((h, p0, kd, vd))
    q = rng.standard_normal((2, kvh * gqa, hd)).astype(np.float32)
    got, ref = _run(dev, deq, pages, q, kvh, gqa, T - 2, 1 / np.sqrt(hd))
    assert np.abs(got - ref).max() <= ABS_TOL


def test_page_order_window_and_empty(dev):
    """Shuffled page order gives the same result; a causal window; a query with no visible token -> zeros
    (the GPU convention; the CPU reference throws, reference kv_reference.cpp:235)."""
    import torch
    from chromofold_amd.legacy import PagedKv
    rng = np.random.default_rng(5)
    hd, kvh, gqa = 64, 2, 2
    pages, deq = [], []
    for h in range(kvh):
        for p0 in range(0, 128, 16):
            k = rng.standard_normal((16, hd)).astype(np.float32)
            v = rng.standard_normal((16, hd)).astype(np.float32)
            page, kd, vd = fixed_page(k, v, h, 100 + p0, 8)
            pages.append(page)
            deq.append((h, 100 + p0, kd, vd))
    order = rng.permutation(len(pages))
    q = rng.standard_normal((2, kvh * gqa, hd)).astype(np.float32)
    a, ref = _run(dev, deq, pages, q, kvh, gqa, 200, 0.125, window=37)
    b, _ = _run(dev, [deq[i] for i in order], [pages[i] for i in order], q, kvh, gqa, 200, 0.125, window=37)
    assert np.abs(a - ref).max() <= ABS_TOL and np.abs(b - ref).max() <= ABS_TOL
    # query token before every page: nothing visible -> zeros
    pk = PagedKv(pages, str(dev))
    out = pk.attention(torch.from_numpy(q).to(dev), kvh, gqa, 10, 0.125).cpu().numpy()
    assert (out == 0).all()


@pytest.mark.parametrize("hd", [32, 64, 96, 128])
def test_rans_pages_with_fixed_huffman_and_tail(dev, hd):
    """The rANS page tag of the seam (kv_cuda.h: fixed_code_length == 0, k_max_code_length == 0): kv_codec_ext.h
    groups coded on their own (full and partial, RANS_HYBRID and the INT8 raw fallback of a group holding -128)
    mixed with fixed-width and Huffman pages of the same heads, a dense tail, GQA 7, a causal window; against the
    fp64 oracle over the values the oracle decodes from each page."""
    from legacy_helpers import rans_page
    rng = np.random.default_rng(900 + hd)
    kvh, gqa = 2, 7
    pages, deq = [], []
    for h in range(kvh):
        tok = 0
        for kind, n in (("rans", 64), ("fixed", 32), ("rans", 40), ("huff", 48), ("int8", 64), ("rans", 7)):
            k = rng.standard_normal((n, hd)).astype(np.float32)
            v = (rng.standard_normal((n, hd)) * 0.3).astype(np.float32)
            if kind == "fixed":
                page, kd, vd = fixed_page(k, v, h, tok, 8)
            elif kind == "huff":
                page, kd, vd = huffman_page(k, v, h, tok)
            else:
                if kind == "int8":
                    k[3, 5] = np.nan  # quantises to -128 (lrint semantics): the encoder stores the group as INT8
                page, kd, vd = rans_page(k, v, h, tok)
            pages.append(page)
            deq.append((h, tok, kd, vd))
            tok += n
    T = tok
    tail_k = rng.standard_normal((5, kvh, hd)).astype(np.float32)
    tail_v = rng.standard_normal((5, kvh, hd)).astype(np.float32)
    q = rng.standard_normal((3, kvh * gqa, hd)).astype(np.float32)
    got, ref = _run(dev, deq, pages, q, kvh, gqa, T + 2, 1 / np.sqrt(hd), tail=(T, tail_k, tail_v))
    assert np.isfinite(got).all()
    assert np.abs(got - ref).max() <= ABS_TOL
    got, ref = _run(dev, deq, pages, q, kvh, gqa, T - 30, 1 / np.sqrt(hd), window=90)
    assert np.abs(got - ref).max() <= ABS_TOL


def test_rans_pages_refused_as_nan(dev):
    """Pages the seam cannot decode on their own give NaN for their (row, KV head) and leave the other head
    untouched: a group that continues a chain (its states live in the group before it), a descriptor whose
    token_count disagrees with the blob, and one whose head_dim disagrees."""
    from legacy_helpers import rans_page
    rng = np.random.default_rng(77)
    hd, kvh, gqa = 64, 2, 2
    k0, v0 = rng.standard_normal((64, hd)).astype(np.float32), rng.standard_normal((64, hd)).astype(np.float32)
    k1, v1 = rng.standard_normal((64, hd)).astype(np.float32), rng.standard_normal((64, hd)).astype(np.float32)
    good, kd, vd = rans_page(k1, v1, 1, 0)
    q = rng.standard_normal((1, kvh * gqa, hd)).astype(np.float32)
    cont, _, _ = rans_page(k1, v1, 0, 0, continues=True, second=(k0, v0))
    wrong_count, _, _ = rans_page(k0, v0, 0, 0)
    wrong_count.token_count = 60
    wrong_dim, _, _ = rans_page(k0, v0, 0, 0)
    wrong_dim.head_dim = 32
    for bad in (cont, wrong_count, wrong_dim):
        got, ref = _run(dev, [(1, 0, kd, vd)], [bad, good], q, kvh, gqa, 63, 0.125)
        assert np.isnan(got[:, :gqa]).all()                       # KV head 0: the refused page
        assert np.abs(got[:, gqa:] - ref[:, gqa:]).max() <= ABS_TOL  # KV head 1: decoded normally


@pytest.mark.parametrize("hd", [64, 128])
def test_many_rows_long_context_splits(dev, hd):
    """The launch shapes small tests never reach: 64 query rows x GQA 7 (448 query vectors = 7 tiles per KV head),
    2 KV heads, 4096 context tokens in 128 pages per head (fixed-width int4, rANS and Huffman pages interleaved across
    heads in the descriptor array), a 20-token dense tail: the context is split over many workgroups whose partials
    are merged by a second kernel. Causal rows (each row sees its own prefix), then a 300-token window."""
    from legacy_helpers import rans_page
    rng = np.random.default_rng(4000 + hd)
    kvh, gqa, T, P = 2, 7, 4096, 32
    pages, deq = [], []
    for p0 in range(0, T, P):
        for h in range(kvh):
            k = rng.standard_normal((P, hd)).astype(np.float32)
            v = rng.standard_normal((P, hd)).astype(np.float32)
            kind = (p0 // P + h) % 5
            if kind == 3:
                page, kd, vd = rans_page(k, v, h, p0)
            elif kind == 4:
                page, kd, vd = huffman_page(k, v, h, p0)
            else:
                page, kd, vd = fixed_page(k, v, h, p0, 4)
            pages.append(page)
            deq.append((h, p0, kd, vd))
    tail_k = rng.standard_normal((20, kvh, hd)).astype(np.float32)
    tail_v = rng.standard_normal((20, kvh, hd)).astype(np.float32)
    q = rng.standard_normal((64, kvh * gqa, hd)).astype(np.float32)
    got, ref = _run(dev, deq, pages, q, kvh, gqa, T + 20 - 64, 1 / np.sqrt(hd), tail=(T, tail_k, tail_v))
    assert np.isfinite(got).all()
    assert np.abs(got - ref).max() <= ABS_TOL
    got, ref = _run(dev, deq, pages, q, kvh, gqa, T - 100, 1 / np.sqrt(hd), window=300, tail=(T, tail_k, tail_v))
    assert np.abs(got - ref).max() <= ABS_TOL


def _zp_page(k, v, kv_head, token_begin, zp):
    """An int4 fixed-width page whose codes sit around zero point `zp` instead of 8: the fixture's symbols (q + 8,
    q in [-7, 7]) moved by zp - 8, so the page dequantises to the same values."""
    ks, vs, ksc, vsc, kd, vd = O.kv_fixture_quantize(k, v, 4)
    assert ks.min() >= 8 - zp and vs.min() >= 8 - zp and ks.max() <= 23 - zp
    page, _, _ = fixed_page(k, v, kv_head, token_begin, 4)
    page.k_words = O.pack_fixed((ks.astype(np.int64) - (8 - zp)).astype(ks.dtype), 4)
    page.v_words = O.pack_fixed((vs.astype(np.int64) - (8 - zp)).astype(vs.dtype), 4)
    page.zero_point = zp
    for words, sym in ((page.k_words, ks), (page.v_words, vs)):
        got = O.huffman_decode(words, page.k_lut, 4, 0, sym.size).astype(np.int64)
        assert np.array_equal(got - zp, sym.reshape(-1).astype(np.int64) - 8)  # same signed codes, other offset
    return page, kd, vd


def test_fixed_pages_paired_with_their_own_zero_points(dev):
    """Consecutive fixed-width pages of 32 tokens or fewer share one 64-token chunk of the seam kernel (two halves,
    each with its page's zero point, K scales and positions); pages of more than 32 tokens fill both halves
    themselves. Pages of 16 tokens alternating zero points 8 and 7, a 5-token page, a 40-token page and a 23-token
    page, 2 KV heads, GQA 7, many query rows; bar 2e-6 (fp32-grade, the values are exact)."""
    rng = np.random.default_rng(515)
    kvh, gqa, D = 2, 7, 64
    pages, deq = [], []
    for h in range(kvh):
        tok = 0
        for i, n in enumerate((16, 16, 16, 5, 16, 40, 16, 23, 16)):
            k = rng.standard_normal((n, D)).astype(np.float32)
            v = rng.standard_normal((n, D)).astype(np.float32)
            page, kd, vd = _zp_page(k, v, h, tok, 8 if i % 2 == 0 else 7)
            pages.append(page)
            deq.append((h, tok, kd, vd))
            tok += n
    T = tok
    q = rng.standard_normal((24, kvh * gqa, D)).astype(np.float32)
    got, ref = _run(dev, deq, pages, q, kvh, gqa, T - 24, 1 / np.sqrt(D))
    assert np.isfinite(got).all()
    assert np.abs(got - ref).max() <= 2e-6
    got, ref = _run(dev, deq, pages, q, kvh, gqa, T - 24, 1 / np.sqrt(D), window=50)
    assert np.abs(got - ref).max() <= 2e-6


@pytest.mark.parametrize("hd", [40, 80])
@pytest.mark.parametrize("bits", [4, 8])
def test_scalar_route_head_dims(dev, hd, bits):
    """head_dim not a multiple of 32 (80 is a real model head size): the reference sends these to its scalar kernel
    (src/cuda/paged_kv_attention.cu:306-324). The adapter matrix's shape (2 KV heads, GQA 7, 32-token sealed pages
    + a dense fp32 tail) with fixed-width pages, then Huffman pages whose rows start mid-way through 64-symbol
    blocks, mixed with fixed-width ones, and a causal window."""
    rng = np.random.default_rng(7000 + hd + bits)
    kvh, gqa, N, P = 2, 7, 70, 32
    K = rng.standard_normal((kvh, N, hd)).astype(np.float32)
    V = rng.standard_normal((kvh, N, hd)).astype(np.float32)
    pages, deq = [], []
    for h in range(kvh):
        for p0 in range(0, (N // P) * P, P):
            page, kd, vd = fixed_page(K[h, p0:p0 + P], V[h, p0:p0 + P], h, p0, bits)
            pages.append(page)
            deq.append((h, p0, kd, vd))
    t0 = (N // P) * P
    tail = (t0, np.ascontiguousarray(K[:, t0:].transpose(1, 0, 2)), np.ascontiguousarray(V[:, t0:].transpose(1, 0, 2)))
    q = rng.standard_normal((3, kvh * gqa, hd)).astype(np.float32)
    got, ref = _run(dev, deq, pages, q, kvh, gqa, N - 3, 1 / np.sqrt(hd), tail=tail)
    assert np.abs(got - ref).max() <= ABS_TOL
    # Huffman pages (40 and 56 tokens: rows cross code blocks) after fixed-width ones
    pages, deq = [], []
    for h in range(kvh):
        tok = 0
        for kind, n in (("fixed", 32), ("huff", 40), ("huff", 56), ("fixed", 16)):
            k = (rng.standard_normal((n, hd)) ** 3).astype(np.float32)
            v = rng.standard_normal((n, hd)).astype(np.float32)
            if kind == "huff":
                page, kd, vd = huffman_page(k, v, h, tok, 8, 12)
            else:
                page, kd, vd = fixed_page(k, v, h, tok, bits)
            pages.append(page)
            deq.append((h, tok, kd, vd))
            tok += n
    q = rng.standard_normal((2, kvh * gqa, hd)).astype(np.float32)
    got, ref = _run(dev, deq, pages, q, kvh, gqa, tok - 2, 1 / np.sqrt(hd))
    assert np.abs(got - ref).max() <= ABS_TOL
    got, ref = _run(dev, deq, pages, q, kvh, gqa, tok - 40, 1 / np.sqrt(hd), window=60)
    assert np.abs(got - ref).max() <= ABS_TOL


def test_scalar_route_head_dim_80_long_context_splits(dev):
    """head_dim 80 at the split shapes: 64 query rows x GQA 7, 2 KV heads, 4096 tokens of int4 and Huffman pages
    and a dense tail: the context is split over many workgroups and merged."""
    rng = np.random.default_rng(8080)
    kvh, gqa, T, P, hd = 2, 7, 4096, 32, 80
    pages, deq = [], []
    for p0 in range(0, T, P):
        for h in range(kvh):
            k = rng.standard_normal((P, hd)).astype(np.float32)
            v = rng.standard_normal((P, hd)).astype(np.float32)
            if (p0 // P + h) % 4 == 3:
                page, kd, vd = huffman_page(k, v, h, p0)
            else:
                page, kd, vd = fixed_page(k, v, h, p0, 4 if (p0 // P) % 2 else 8)
            pages.append(page)
            deq.append((h, p0, kd, vd))
    tail_k = rng.standard_normal((9, kvh, hd)).astype(np.float32)
    tail_v = rng.standard_normal((9, kvh, hd)).astype(np.float32)
    q = rng.standard_normal((64, kvh * gqa, hd)).astype(np.float32)
    got, ref = _run(dev, deq, pages, q, kvh, gqa, T + 9 - 64, 1 / np.sqrt(hd), tail=(T, tail_k, tail_v))
    assert np.isfinite(got).all()
    assert np.abs(got - ref).max() <= ABS_TOL


def _route_case(rng, kvh, hd, T, int8_at=None):
    """rANS pages of 64 tokens (the last one ragged) for every KV head, one table pair per head shared by all its
    pages, in shuffled descriptor order."""
    from chromofold_amd import kv
    from legacy_helpers import rans_page
    pages, deq = [], []
    for h in range(kvh):
        K = rng.standard_normal((T, hd)).astype(np.float32)
        V = (rng.standard_normal((T, hd)) * (0.5 + h)).astype(np.float32)
        n = min(T, 1024)
        tables = np.concatenate([kv.build_table(K[:n - n % 16].reshape(-1, 16, hd)),
                                 kv.build_table(V[:n - n % 16].reshape(-1, 16, hd))])
        for p0 in range(0, T, 64):
            k, v = K[p0:p0 + 64].copy(), V[p0:p0 + 64].copy()
            if int8_at is not None and (h, p0) == int8_at:
                k[1, 2] = np.nan  # -128 after quantisation: the encoder stores this group as INT8
            page, kd, vd = rans_page(k, v, h, p0, tables=tables)
            pages.append(page)
            deq.append((h, p0, kd, vd))
    order = rng.permutation(len(pages))
    return [pages[i] for i in order], [deq[i] for i in order]


def _run_shared(dev, deq, pages, q, kvh, gqa, qtok, scale, window=0):
    import torch
    from chromofold_amd.legacy import PagedKv
    pk = PagedKv(pages, str(dev), share_luts=True)
    got = pk.attention(torch.from_numpy(q).to(dev), kvh, gqa, qtok, scale, window).cpu().numpy()
    ref = np.zeros_like(q)
    ref[0], _ = O.paged_attention_f64(q[0], q.shape[1], kvh, q.shape[2], gqa, qtok, window, scale, deq, None)
    return got, ref


@pytest.mark.parametrize("hd,gqa,kvh,T", [(128, 4, 8, 4000), (64, 1, 3, 2500), (128, 3, 2, 700), (64, 4, 1, 64)])
def test_decode_route_rans_pages(dev, hd, gqa, kvh, T):
    """A decode call (one query row, at most 4 query heads per KV head) over rANS pages whose KV heads each share one
    table pair: the seam's decode-shape route (a page list per head, whole pages per wavefront through the batched
    decode's group body, the seam's merge). Against the fp64 oracle at the seam's 2e-4 bar: the query at the end of
    the context, in the middle of it (later pages wholly invisible, one page partly visible), and with a causal
    window; a group stored as INT8 (it holds -128) among the rANS groups."""
    rng = np.random.default_rng(7000 + hd + T)
    pages, deq = _route_case(rng, kvh, hd, T, int8_at=(0, 64) if T > 64 else None)
    q = rng.standard_normal((1, kvh * gqa, hd)).astype(np.float32)
    sc = 1 / np.sqrt(hd)
    for qtok, window in ((T - 1, 0), (T // 2 + 5, 0), (T - 1, 300), (T // 3, 100)):
        got, ref = _run_shared(dev, deq, pages, q, kvh, gqa, qtok, sc, window)
        assert np.isfinite(got).all(), (qtok, window)
        assert np.abs(got - ref).max() <= ABS_TOL, (qtok, window, float(np.abs(got - ref).max()))


def test_decode_route_mixed_heads(dev):
    """One decode call where the route takes KV head 0 (rANS pages, one table pair) and leaves KV head 1 to the seam
    kernel (a fixed-width page among its rANS pages) and KV head 2 too (its rANS pages carry two different table
    pairs): every head against the fp64 oracle."""
    from chromofold_amd import kv
    from legacy_helpers import rans_page
    rng = np.random.default_rng(7100)
    hd, gqa, kvh, T = 128, 4, 3, 640
    pages, deq = _route_case(rng, 1, hd, T)
    for h in (1, 2):
        K = rng.standard_normal((T, hd)).astype(np.float32)
        V = rng.standard_normal((T, hd)).astype(np.float32)
        tabs = [np.concatenate([kv.build_table(K[:256].reshape(-1, 16, hd)), kv.build_table(V[:256].reshape(-1, 16, hd))]),
                np.concatenate([kv.build_table(K[256:512].reshape(-1, 16, hd)),
                                kv.build_table(V[256:512].reshape(-1, 16, hd))])]
        for p0 in range(0, T, 64):
            if h == 1 and p0 == 128:
                page, kd, vd = fixed_page(K[p0:p0 + 64], V[p0:p0 + 64], h, p0, 8)
            else:
                page, kd, vd = rans_page(K[p0:p0 + 64], V[p0:p0 + 64], h, p0,
                                         tables=tabs[(p0 // 64) % 2 if h == 2 else 0])
            pages.append(page)
            deq.append((h, p0, kd, vd))
    q = rng.standard_normal((1, kvh * gqa, hd)).astype(np.float32)
    got, ref = _run_shared(dev, deq, pages, q, kvh, gqa, T - 1, 1 / np.sqrt(hd))
    assert np.isfinite(got).all()
    assert np.abs(got - ref).max() <= ABS_TOL


def test_decode_route_refused_pages_nan(dev):
    """Pages the route refuses make their KV head's outputs NaN, as the seam kernel does, and leave the other heads
    untouched: a group that continues a chain, a descriptor whose token_count disagrees with its blob, and a blob
    whose word stream was altered (the chain no longer ends where the encoder started)."""
    from legacy_helpers import rans_page
    rng = np.random.default_rng(7200)
    hd, gqa, kvh, T = 64, 2, 2, 256
    pages, deq = _route_case(rng, kvh, hd, T)
    q = rng.standard_normal((1, kvh * gqa, hd)).astype(np.float32)
    h0 = [i for i, p in enumerate(pages) if p.kv_head == 0]
    k0 = rng.standard_normal((64, hd)).astype(np.float32)
    v0 = rng.standard_normal((64, hd)).astype(np.float32)
    for how in ("continues", "count", "stream"):
        bad = list(pages)
        i = h0[1]
        p = pages[i]
        if how == "continues":
            cont, _, _ = rans_page(k0, v0, 0, p.token_begin, continues=True, second=(k0, v0), tables=None)
            cont.k_lut, cont.v_lut = p.k_lut, p.v_lut  # the head's table pair, so that the route still takes the head
            bad[i] = cont
        elif how == "count":
            q2, _, _ = rans_page(k0, v0, 0, p.token_begin)
            q2.k_lut, q2.v_lut = p.k_lut, p.v_lut
            q2.token_count = 60
            bad[i] = q2
        else:
            q2, _, _ = rans_page(k0, v0, 0, p.token_begin, tables=np.concatenate([p.k_lut, p.v_lut]))
            blob = q2.k_words.copy()
            blob[-20] ^= 0x5A  # a byte of the word streams
            q2.k_words = blob
            bad[i] = q2
        got, ref = _run_shared(dev, deq, bad, q, kvh, gqa, T - 1, 0.125)
        assert np.isnan(got[:, :gqa]).all(), how                      # KV head 0: the refused page
        assert np.abs(got[:, gqa:] - ref[:, gqa:]).max() <= ABS_TOL, how  # KV head 1: decoded normally


def test_decode_route_many_heads_full_page_list(dev):
    """The route at its limits: 64 KV heads (the most it serves) x 64 rANS pages = 4096 descriptors (the seam's
    per-launch limit), so every one of the 16 list workgroups sees all 64 heads and every head's pages span all 16
    chunk records; plus a descriptor whose kv_head lies past the call's KV heads, which the route and the seam
    kernel both leave out. Against the fp64 oracle, which only ever reads pages of the call's heads."""
    import copy
    rng = np.random.default_rng(7300)
    hd, gqa, kvh, T = 64, 1, 64, 4096
    pages, deq = _route_case(rng, kvh, hd, T)
    assert len(pages) == 4096
    q = rng.standard_normal((1, kvh * gqa, hd)).astype(np.float32)
    got, ref = _run_shared(dev, deq, pages, q, kvh, gqa, T - 1, 0.125)
    assert np.isfinite(got).all()
    assert np.abs(got - ref).max() <= ABS_TOL
    stray = copy.copy(pages[5])
    stray.kv_head = kvh  # not a KV head of this call
    more = pages[:100] + [stray] + pages[100:-1]  # 4096 descriptors again; the dropped page's head loses a page
    kept = [d for d in deq if not (d[0] == pages[-1].kv_head and d[1] == pages[-1].token_begin)]
    got2, ref2 = _run_shared(dev, kept, more, q, kvh, gqa, T - 1, 0.125)
    assert np.isfinite(got2).all()
    assert np.abs(got2 - ref2).max() <= ABS_TOL


def test_decode_route_unaligned_tables_fall_back(dev):
    """Table pointers off 16-byte alignment: the route leaves the head to the seam kernel (which reads tables at
    any 4-byte alignment), with the same results within the bar."""
    import torch
    from chromofold_amd.legacy import PagedKv
    rng = np.random.default_rng(7400)
    hd, gqa, kvh, T = 128, 4, 2, 512
    pages, deq = _route_case(rng, kvh, hd, T)
    q = rng.standard_normal((1, kvh * gqa, hd)).astype(np.float32)
    got, ref = _run_shared(dev, deq, pages, q, kvh, gqa, T - 1, 0.125)
    assert np.abs(got - ref).max() <= ABS_TOL
    import ctypes as C
    from chromofold_amd import _abi as A
    pk = PagedKv(pages, str(dev), share_luts=True)
    arr = (A.cf_kv_device_page * len(pages)).from_buffer_copy(pk.descs.cpu().numpy().tobytes())
    copies = {}
    for i, p in enumerate(pages):  # every table re-pointed 4 bytes into a copy of the same contents
        for f in ("k_lut", "v_lut"):
            a = np.ascontiguousarray(getattr(p, f)).view(np.int32)
            key = a.tobytes()
            if key not in copies:
                copies[key] = torch.from_numpy(np.concatenate([[0], a]).astype(np.int32)).to(dev)
            setattr(arr[i], f, copies[key].data_ptr() + 4)
            assert getattr(arr[i], f) % 16 == 4
    pk.descs = torch.from_numpy(np.frombuffer(bytes(arr), np.uint8).copy()).to(dev)
    got2 = pk.attention(torch.from_numpy(q).to(dev), kvh, gqa, T - 1, 0.125).cpu().numpy()
    assert np.abs(got2 - ref).max() <= ABS_TOL
