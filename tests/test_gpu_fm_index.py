"""GPU parity of the FM-index entry points (cf_fm_count/ranges/locate_async) and the GPU suffix-array build.

Anchors: the reference fixture tiny.cffm (528 count goldens and their located positions, compared as sorted sets
like reference benchmarks/fm_search.cu:150-186), the naive substring search the reference itself uses as ground
truth (tools/build_index.cpp:322-333), and the CPU suffix array (unique for a sentinel-terminated text, so the
GPU build must match it bit for bit, reference benchmarks/suffix_array.cu:186-197). Bit-exact throughout.
"""
import numpy as np
import pytest

import cf_fixtures as F
import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _i32(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev)


def _check_locate(idx, lo, hi, expected_sets, dev):
    rows = np.concatenate([np.arange(a, b, dtype=np.int32) for a, b in zip(lo, hi)] or [np.zeros(0, np.int32)])
    if rows.size == 0:
        return
    pos = idx.locate(_i32(rows, dev)).cpu().numpy()
    at = 0
    for t, (a, b) in enumerate(zip(lo, hi)):
        got = np.sort(pos[at:at + (b - a)])
        at += b - a
        assert np.array_equal(got, expected_sets(t)), t


def test_tiny_cffm_fixture(dev):
    from chromofold_amd.search import FmIndex
    d = F.load_cffm()
    idx = FmIndex.from_host(d, dev)
    pat, ps, pl = _i32(d["pat"], dev), _i32(d["pstart"], dev), _i32(d["plen"], dev)
    cnt = idx.count(pat, ps, pl).cpu().numpy().view(np.uint32)
    assert np.array_equal(cnt, d["count_golden"])
    lo, hi = (x.cpu().numpy() for x in idx.ranges(pat, ps, pl))
    assert np.array_equal((hi - lo).astype(np.uint32), d["count_golden"])
    _check_locate(idx, lo, hi, lambda t: d["locpos"][d["locoff"][t]:d["locoff"][t + 1]], dev)


@pytest.mark.parametrize("n,vocab,sample,seed", [(5000, 3, 4, 1), (20000, 64, 16, 2), (200000, 32000, 32, 3)])
def test_random_text_vs_naive(dev, n, vocab, sample, seed):
    import torch
    from chromofold_amd import synth
    from chromofold_amd.search import FmIndex, gpu_suffix_array
    rng = np.random.default_rng(seed)
    tok = synth.zipf_tokens(n, vocab, 1.1, seed) if vocab > 100 else rng.integers(0, vocab, n).astype(np.uint32)
    s = O.fm_text(tok)
    sa_cpu = O.suffix_array(s)
    sa_gpu = gpu_suffix_array(_i32(s, dev)).cpu().numpy()
    assert np.array_equal(sa_gpu, sa_cpu)
    f, bwt = O.fm_build(tok, sample, sa=sa_cpu)
    idx = FmIndex.from_host(f, dev)
    # patterns: windows of the text (length 1..32), random patterns, out-of-alphabet symbols, empty pattern
    pats, starts, lens = [], [], []
    at = 0
    for k in range(600):
        L = int(rng.integers(1, 33))
        if k % 10 == 9:
            p = rng.integers(0, vocab, L) + 1
        else:
            o = int(rng.integers(0, max(1, n - L)))
            p = tok[o:o + L].astype(np.int64) + 1
        if k == 7:
            p = np.array([f.sigma + 5, 1, 2])       # symbol past the alphabet -> empty range
        if k == 11:
            p = np.array([-3, 1])                   # negative symbol -> empty range
        if k == 13:
            p = np.zeros(0, np.int64)               # empty pattern -> the whole BWT
        pats.append(p)
        starts.append(at)
        lens.append(len(p))
        at += len(p)
    pat = np.concatenate(pats).astype(np.int32)
    ps, pl = np.array(starts, np.int32), np.array(lens, np.int32)
    cnt = idx.count(_i32(pat, dev), _i32(ps, dev), _i32(pl, dev)).cpu().numpy()
    assert np.array_equal(cnt.view(np.uint32), O.fm_count(f, pat, ps, pl))
    seq = tok.astype(np.int32)
    for t in range(0, len(pats), 5):
        p = pats[t]
        if len(p) and (p.min() < 1 or p.max() >= f.sigma):
            assert cnt[t] == 0
        elif len(p):
            assert cnt[t] == O.naive_count(seq, (p - 1).astype(np.int32)), t
        else:
            assert cnt[t] == f.n
    lo, hi = (x.cpu().numpy() for x in idx.ranges(_i32(pat, dev), _i32(ps, dev), _i32(pl, dev)))
    sel = [t for t in range(len(pats)) if 0 < lens[t] and hi[t] - lo[t] <= 2000][:200]
    _check_locate(idx, lo[sel], hi[sel],
                  lambda j: np.sort(O.naive_positions(seq, (pats[sel[j]] - 1).astype(np.int32))), dev)


def test_locate_every_row(dev):
    """locate of every SA row returns the suffix array itself (SA[r] == locate(r))."""
    from chromofold_amd.search import FmIndex
    rng = np.random.default_rng(9)
    tok = rng.integers(0, 40, 30000).astype(np.uint32)
    s = O.fm_text(tok)
    sa = O.suffix_array(s)
    for sample in (1, 7, 32):
        f, _ = O.fm_build(tok, sample, sa=sa)
        idx = FmIndex.from_host(f, dev)
        got = idx.locate(_i32(np.arange(s.size), dev)).cpu().numpy()
        assert np.array_equal(got, sa), sample


@pytest.mark.parametrize("n,vocab", [(1, 1), (2, 1), (17, 2), (1000, 1), (4096, 2), (100000, 5), (300000, 32000)])
def test_gpu_suffix_array_shapes(dev, n, vocab):
    from chromofold_amd.search import gpu_suffix_array
    rng = np.random.default_rng(n)
    tok = rng.integers(0, vocab, n).astype(np.uint32)
    s = O.fm_text(tok)
    assert np.array_equal(gpu_suffix_array(_i32(s, dev)).cpu().numpy(), O.suffix_array(s))


def _fm_oracle_view(fm):
    from chromofold_amd.search import to_u32
    w = O.RrrwArrays(fm.w.bits, fm.w.cwords, fm.w.nsb, fm.w.na,
                     *[fm.w.tensors[k].cpu().numpy().view(dt) for k, dt in
                       (("classes", np.uint32), ("offsets", np.uint32), ("rank_a", np.int32),
                        ("rank_d", np.uint16), ("off_a", np.int32), ("off_d", np.uint16),
                        ("offbase", np.int32), ("zeros", np.int32))])
    return O.FmArrays(w, fm.tensors["C"].cpu().numpy(), to_u32(fm.tensors["mwords"]), fm.tensors["msb"].cpu().numpy(),
                      fm.tensors["sval"].cpu().numpy(), fm.sigma, fm.n, fm.sa_sample)


@pytest.mark.parametrize("n", [200_000, 2_000_000])
def test_staged_kernels_vs_oracle(dev, n):
    """Batches of >= 256 x 1024 items take the persistent kernels that stage the wavelet's tables in LDS: all of them
    for the 200K-token index, the anchors and the unrank table only for the 2M-token one (its per-superblock deltas
    exceed the LDS budget). Count, ranges and locate against the oracle, bit for bit."""
    import torch
    from chromofold_amd import synth
    from chromofold_amd.search import build_fm
    vocab = 32000
    tok = synth.zipf_tokens(n, vocab, 1.1, 40 + n % 7)
    fm, _ = build_fm(torch.from_numpy(tok.view(np.int32)).to(dev), 32)
    w = fm.w
    deltas = 2 * 2 * w.bits * (w.nsb + 1)
    assert (deltas < 90_000) == (n < 1_000_000)  # which staged variant each case exercises
    flat, pstart, plen = synth.fm_patterns(tok, 270_000, 30_000, vocab, 41, 4, 12)
    dpat, dps, dpl = (_i32(a, dev) for a in (flat, pstart, plen))
    cnt = fm.count(dpat, dps, dpl).cpu().numpy().view(np.uint32)
    lo, hi = (x.cpu().numpy() for x in fm.ranges(dpat, dps, dpl))
    f = _fm_oracle_view(fm)
    assert np.array_equal(cnt, O.fm_count(f, flat, pstart, plen))
    rlo, rhi = O.fm_ranges(f, flat, pstart, plen)
    assert np.array_equal(lo, rlo) and np.array_equal(hi, rhi)
    rows = np.concatenate([np.arange(a, b, dtype=np.int32) for a, b in zip(lo, hi) if b > a])[:270_000]
    assert rows.size >= 256 * 1024
    pos = torch.empty(rows.size, dtype=torch.int32, device=dev)
    fm.locate(_i32(rows, dev), pos)
    assert np.array_equal(pos.cpu().numpy(), O.fm_locate(f, rows))


def test_staged_kernels_many_items_per_lane(dev):
    """The staged kernels hand items to lanes from a per-workgroup queue. Here each lane takes several items of very
    different cost: 1.2M patterns of length 0-40 (the empty pattern matches every row) and up to 1.2M occurrences,
    whose LF walks take 0-31 steps. Count, ranges and locate against the oracle, bit for bit."""
    import torch
    from chromofold_amd import synth
    from chromofold_amd.search import build_fm
    vocab = 32000
    tok = synth.zipf_tokens(200_000, vocab, 1.1, 43)
    fm, _ = build_fm(torch.from_numpy(tok.view(np.int32)).to(dev), 32)
    flat, pstart, plen = synth.fm_patterns(tok, 1_000_000, 200_000, vocab, 44, 0, 40)
    assert (plen == 0).any() and pstart.size >= 4 * 256 * 1024
    dpat, dps, dpl = (_i32(a, dev) for a in (flat, pstart, plen))
    cnt = fm.count(dpat, dps, dpl).cpu().numpy().view(np.uint32)
    lo, hi = (x.cpu().numpy() for x in fm.ranges(dpat, dps, dpl))
    f = _fm_oracle_view(fm)
    assert np.array_equal(cnt, O.fm_count(f, flat, pstart, plen))
    assert (cnt[plen == 0] == fm.n).all()
    rlo, rhi = O.fm_ranges(f, flat, pstart, plen)
    assert np.array_equal(lo, rlo) and np.array_equal(hi, rhi)
    keep = (hi > lo) & (hi - lo < 64)
    rows = np.concatenate([np.arange(a, b, dtype=np.int32) for a, b in zip(lo[keep], hi[keep])])[:1_200_000]
    assert rows.size >= 4 * 256 * 1024
    pos = torch.empty(rows.size, dtype=torch.int32, device=dev)
    fm.locate(_i32(rows, dev), pos)
    assert np.array_equal(pos.cpu().numpy(), O.fm_locate(f, rows))


def test_gpu_suffix_array_c2_size(dev):
    """BASELINE C2's full text: 2^24 Zipf tokens (V = 32000) plus the sentinel. The GPU suffix array (prefix doubling
    on hipCUB radix sorts) equals the oracle's radix-doubling suffix array, every entry."""
    from chromofold_amd import synth
    from chromofold_amd.search import gpu_suffix_array
    tok = synth.zipf_tokens(1 << 24, 32000, 1.1, synth.SEED_C1 + 24)
    s = O.fm_text(tok)
    assert np.array_equal(gpu_suffix_array(_i32(s, dev)).cpu().numpy(), O.suffix_array(s))


def test_fm_c2_shape_patterns_8_to_32(dev):
    """BASELINE C2's shape: the FM index of 2^24 Zipf tokens built on the GPU, queried with patterns of length 8-32
    (cut from the text, plus random ones that almost never occur). Count and ranges of 300K patterns and locate of
    256K rows, against the oracle over the same index arrays, bit for bit; the cut patterns all occur."""
    import torch
    from chromofold_amd import synth
    from chromofold_amd.search import build_fm
    vocab, n = 32000, 1 << 24
    tok = synth.zipf_tokens(n, vocab, 1.1, synth.SEED_C1 + 25)
    fm, _ = build_fm(torch.from_numpy(tok.view(np.int32)).to(dev), 32)
    flat, pstart, plen = synth.fm_patterns(tok, 270_000, 30_000, vocab, 46, 8, 32)
    assert plen.min() == 8 and plen.max() == 32
    dpat, dps, dpl = (_i32(a, dev) for a in (flat, pstart, plen))
    cnt = fm.count(dpat, dps, dpl).cpu().numpy().view(np.uint32)
    lo, hi = (x.cpu().numpy() for x in fm.ranges(dpat, dps, dpl))
    f = _fm_oracle_view(fm)
    assert np.array_equal(cnt, O.fm_count(f, flat, pstart, plen))
    assert (cnt[:270_000] >= 1).all()
    rlo, rhi = O.fm_ranges(f, flat, pstart, plen)
    assert np.array_equal(lo, rlo) and np.array_equal(hi, rhi)
    rows = np.concatenate([np.arange(a, b, dtype=np.int32) for a, b in zip(lo, hi) if b > a])[:256 * 1024]
    pos = torch.empty(rows.size, dtype=torch.int32, device=dev)
    fm.locate(_i32(rows, dev), pos)
    assert np.array_equal(pos.cpu().numpy(), O.fm_locate(f, rows))
