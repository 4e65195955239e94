"""GPU parity of the derived line layout of the FM-index (cf_fm_lines_build_async and the cf_fm_*_lines_async search
entry points, chromofold_index.h) and of the derived 4-ary layout (cf_fm_quads_*), checked the same way (its records,
bucket starts and lfb against a 4-ary wavelet matrix of the BWT built here by stable sorts).

The layout has no counterpart in the reference: it is built on the device from the same cf_fm_view, and the search
entry points over it must return exactly what the RRR entry points return. Anchors:
  * the records themselves, word for word, against the wavelet matrix of the BWT built here in numpy by the
    textbook rule (level l = bit l of each symbol from the top, then a stable zeros-first partition), independent of
    the RRR arrays the device build decodes; lfb[c] against C[c] minus the end of c's rank walk on those levels;
  * count / ranges / locate against the reference fixture tiny.cffm's goldens, against the oracle on random texts
    (including out-of-alphabet and negative symbols and the empty pattern), and against the RRR entry points on
    the BASELINE C2 index (2^24 Zipf tokens). Bit-exact throughout.
Text lengths are chosen so that the BWT length n is a multiple of 480 and of 960 (the last record then starts at
bit n and holds only the level's total), and neither.
"""
import numpy as np
import pytest

import cf_fixtures as F
import oracle as O
from test_gpu_fm_index import _fm_oracle_view

pytestmark = pytest.mark.gpu
LINE_BITS = 480


@pytest.fixture(scope="module")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _i32(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev)


def _wm_levels(bwt: np.ndarray, bits: int) -> list[np.ndarray]:
    seq = bwt.astype(np.int64)
    levels = []
    for lvl in range(bits):
        b = (seq >> (bits - 1 - lvl)) & 1
        levels.append(b.astype(np.uint8))
        seq = np.concatenate([seq[b == 0], seq[b == 1]])
    return levels


def expected_lines(seq: np.ndarray, bits: int, X: np.ndarray, nrec: int | None = None):
    """Records and per-symbol table of the line layout of the wavelet matrix of `seq`: (records [bits][nrec][16],
    base[c] = X[c] - e(c) for c < X.size)."""
    n = seq.size
    nrec = n // LINE_BITS + 1 if nrec is None else nrec
    assert nrec * LINE_BITS > n
    recs = np.zeros((bits, nrec, 16), np.uint32)
    levels = _wm_levels(seq, bits)
    for lvl, b in enumerate(levels):
        padded = np.zeros(nrec * LINE_BITS, np.uint8)
        padded[:n] = b
        blk = padded.reshape(nrec, LINE_BITS)
        recs[lvl, :, 0] = np.concatenate([[0], np.cumsum(blk.sum(1, dtype=np.int64))[:-1]])
        recs[lvl, :, 1:] = np.packbits(blk.reshape(nrec, 15, 32), axis=2, bitorder="little").view("<u4")[..., 0]
    # end of each symbol's rank walk from position 0
    sigma = X.size
    c = np.arange(sigma, dtype=np.int64)
    p = np.zeros(sigma, np.int64)
    for lvl, b in enumerate(levels):
        pre = np.concatenate([[0], np.cumsum(b, dtype=np.int64)])
        rp = pre[p]
        zeros = n - int(b.sum())
        p = np.where((c >> (bits - 1 - lvl)) & 1, zeros + rp, p - rp)
    return recs, (X.astype(np.int64) - p).astype(np.int32)


def check_layout(lines, bits, recs, base):
    """The built layout (uint8 device tensor) against expected_lines' records and table, word for word."""
    lines = lines.cpu().numpy().view(np.uint32)
    nw = recs.size
    assert lines.size == nw + base.size
    got = lines[:nw].reshape(recs.shape)
    for lvl in range(bits):
        bad = np.nonzero((got[lvl] != recs[lvl]).any(1))[0]
        assert bad.size == 0, f"level {lvl}: {bad.size} records differ, first {bad[:5]}"
    assert np.array_equal(lines[nw:].view(np.int32), base)


def _check_layout(idx, bwt):
    from test_gpu_rrr_wavelet import expected_quads
    bits = idx.w.bits
    C = idx.tensors["C"].cpu().numpy()
    recs, lfb = expected_lines(bwt, bits, C)
    check_layout(idx.build_lines(), bits, recs, lfb)
    q = idx.build_quads().cpu().numpy().view(np.uint32)
    qrecs, Z, qlfb = expected_quads(bwt, bits, C)
    nw = qrecs.size
    assert q.size == nw + Z.size + qlfb.size
    assert np.array_equal(q[:nw].reshape(qrecs.shape), qrecs)
    assert np.array_equal(q[nw:nw + Z.size].reshape(Z.shape), Z)
    assert np.array_equal(q[nw + Z.size:].view(np.int32), qlfb)


def _search_both(idx, pat, ps, pl, dev):
    dp, ds, dl = _i32(pat, dev), _i32(ps, dev), _i32(pl, dev)
    cnt = idx.count_lines(dp, ds, dl).cpu().numpy().view(np.uint32)
    lo, hi = (x.cpu().numpy() for x in idx.ranges_lines(dp, ds, dl))
    rcnt = idx.count(dp, ds, dl).cpu().numpy().view(np.uint32)
    rlo, rhi = (x.cpu().numpy() for x in idx.ranges(dp, ds, dl))
    assert np.array_equal(cnt, rcnt)
    assert np.array_equal(lo, rlo) and np.array_equal(hi, rhi)
    qcnt = idx.count_quads(dp, ds, dl).cpu().numpy().view(np.uint32)
    qlo, qhi = (x.cpu().numpy() for x in idx.ranges_quads(dp, ds, dl))
    assert np.array_equal(qcnt, rcnt)
    assert np.array_equal(qlo, rlo) and np.array_equal(qhi, rhi)
    return cnt, lo, hi


def test_tiny_cffm_fixture(dev):
    from chromofold_amd.search import FmIndex
    d = F.load_cffm()
    idx = FmIndex.from_host(d, dev)
    w = O.RrrwArrays(d["bits"], d["cwords"], d["nsb"], d["na"], d["classes"], d["offsets"], d["rank_a"],
                     d["rank_d"], d["off_a"], d["off_d"], d["offbase"], d["zeros"])
    bwt = O.rrrw_access(w, np.arange(d["n"], dtype=np.uint32))
    _check_layout(idx, bwt)
    cnt, lo, hi = _search_both(idx, d["pat"], d["pstart"], d["plen"], dev)
    assert np.array_equal(cnt, d["count_golden"])
    rows = np.concatenate([np.arange(a, b, dtype=np.int32) for a, b in zip(lo, hi)])
    pos = idx.locate_lines(_i32(rows, dev)).cpu().numpy()
    assert np.array_equal(idx.locate_quads(_i32(rows, dev)).cpu().numpy(), pos)
    at = 0
    for t, (a, b) in enumerate(zip(lo, hi)):
        got = np.sort(pos[at:at + (b - a)])
        at += b - a
        assert np.array_equal(got, d["locpos"][d["locoff"][t]:d["locoff"][t + 1]]), t


@pytest.mark.parametrize("ntok,vocab,sample,seed", [
    (4799, 3, 4, 1),            # n = 4800 = 10 records exactly (n % 480 == 0, n % 960 == 0): the tail record
    (20159, 64, 16, 2),         # n = 20160 = 42 records (n % 960 == 0)
    (20639, 64, 16, 3),         # n = 20640 = 43 records (n % 480 == 0, odd record count)
    (200_000, 32000, 32, 4),    # 15 levels
    (77_777, 1, 3, 5),          # one symbol (sigma 2: one level)
])
def test_random_text_vs_oracle(dev, ntok, vocab, sample, seed):
    from chromofold_amd import synth
    from chromofold_amd.search import FmIndex
    rng = np.random.default_rng(seed)
    tok = synth.zipf_tokens(ntok, vocab, 1.1, seed) if vocab > 100 else rng.integers(0, vocab, ntok).astype(np.uint32)
    f, bwt = O.fm_build(tok, sample)
    idx = FmIndex.from_host(f, dev)
    _check_layout(idx, np.asarray(bwt))
    pats, starts, lens = [], [], []
    at = 0
    for k in range(3000):
        L = int(rng.integers(1, 33))
        if k % 10 == 9:
            p = rng.integers(0, vocab, L) + 1
        else:
            o = int(rng.integers(0, max(1, ntok - L)))
            p = tok[o:o + L].astype(np.int64) + 1
        if k == 7:
            p = np.array([f.sigma + 5, 1, 2])      # symbol past the alphabet -> empty range
        if k == 11:
            p = np.array([-3, 1])                  # negative symbol -> empty range
        if k == 13:
            p = np.zeros(0, np.int64)              # empty pattern -> the whole BWT
        if k == 17:
            p = np.array([f.sigma - 1])            # the largest symbol alone
        pats.append(p)
        starts.append(at)
        lens.append(len(p))
        at += len(p)
    pat = np.concatenate(pats).astype(np.int32)
    ps, pl = np.array(starts, np.int32), np.array(lens, np.int32)
    cnt, lo, hi = _search_both(idx, pat, ps, pl, dev)
    assert np.array_equal(cnt, O.fm_count(f, pat, ps, pl))
    rlo, rhi = O.fm_ranges(f, pat, ps, pl)
    assert np.array_equal(lo, rlo) and np.array_equal(hi, rhi)
    assert cnt[13] == f.n and cnt[7] == 0 and cnt[11] == 0
    # locate of every row (SA itself), many LF steps per lane from the per-workgroup queue
    rows = np.arange(f.n, dtype=np.int32)
    got = idx.locate_lines(_i32(rows, dev)).cpu().numpy()
    assert np.array_equal(got, O.fm_locate(f, rows))
    assert np.array_equal(got, idx.locate(_i32(rows, dev)).cpu().numpy())
    assert np.array_equal(idx.locate_quads(_i32(rows, dev)).cpu().numpy(), got)


def test_fm_c2_index_lines_vs_rrr(dev):
    """BASELINE C2's index (2^24 Zipf tokens, V = 32000, SA sample 32) built on the GPU: the line-layout search
    equals the RRR search for 1M patterns of length 8-32 (900K cut from the text, 100K random) and equals the oracle
    on the first 100K; locate of 1M occurrence rows equals the RRR locate."""
    import torch
    from chromofold_amd import synth
    from chromofold_amd.search import build_fm
    vocab, n = 32000, 1 << 24
    tok = synth.zipf_tokens(n, vocab, 1.1, synth.SEED_C2)
    fm, _ = build_fm(torch.from_numpy(tok.view(np.int32)).to(dev), 32)
    flat, pstart, plen = synth.fm_patterns(tok, 900_000, 100_000, vocab, synth.SEED_C2 + 1)
    cnt, lo, hi = _search_both(fm, flat, pstart, plen, dev)
    assert (cnt[:900_000] >= 1).all()
    k = 100_000
    f = _fm_oracle_view(fm)
    assert np.array_equal(cnt[:k], O.fm_count(f, flat, pstart[:k], plen[:k]))
    rows = np.concatenate([np.arange(a, b, dtype=np.int32) for a, b in zip(lo, hi) if b > a])[:1 << 20]
    dr = _i32(rows, dev)
    got = fm.locate_lines(dr).cpu().numpy()
    assert np.array_equal(got, fm.locate(dr).cpu().numpy())
    assert np.array_equal(fm.locate_quads(dr).cpu().numpy(), got)
    assert np.array_equal(got[:50_000], O.fm_locate(f, rows[:50_000]))


def test_lines_entry_points_reject_bad_arguments(dev):
    from chromofold_amd import _abi as A
    from chromofold_amd.search import FmIndex
    d = F.load_cffm()
    idx = FmIndex.from_host(d, dev)
    v = idx.view()
    lines = idx.build_lines()
    nb = int(A.lib().cf_fm_lines_bytes(v))
    assert nb == lines.numel()
    L = A.lib()
    assert L.cf_fm_lines_build_async(v, lines.data_ptr(), nb - 4, None) == A.CF_ERR_INVALID_ARGUMENT
    assert L.cf_fm_lines_build_async(v, None, nb, None) == A.CF_ERR_INVALID_ARGUMENT
    out = _i32(np.zeros(4), dev)
    assert L.cf_fm_count_lines_async(v, None, out.data_ptr(), out.data_ptr(), out.data_ptr(), out.data_ptr(), 4,
                                     None) == A.CF_ERR_INVALID_ARGUMENT
    assert L.cf_fm_count_lines_async(v, lines.data_ptr(), out.data_ptr(), out.data_ptr(), out.data_ptr(),
                                     out.data_ptr(), 0, None) == A.CF_OK
    bad = A.cf_fm_view.from_buffer_copy(v)
    bad.sigma = (1 << bad.w.bits) + 1  # more symbols than the levels can hold
    assert int(L.cf_fm_lines_bytes(bad)) > 0
    assert L.cf_fm_lines_build_async(bad, lines.data_ptr(), 1 << 30, None) == A.CF_ERR_INVALID_ARGUMENT
    assert L.cf_fm_locate_lines_async(v, lines.data_ptr(), None, out.data_ptr(), 4, None) == \
        A.CF_ERR_INVALID_ARGUMENT
