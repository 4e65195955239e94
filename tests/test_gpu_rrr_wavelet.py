"""GPU parity of cf_rrrw_access_async / cf_rrrw_rank_async against the reference fixture and the CPU oracle.

Mirrors the reference's own check (benchmarks/rrr_wavelet.cu:135-143: access and rank std::equal to the golden
arrays) and adds closed-form ground truth at the C1 shape: access(i) == tokens[i], rank(c, i) == #{j < i: t_j = c}.
The derived line layout (cf_rrrw_lines_*, chromofold_index.h) answers the same queries in every test and must equal
the RRR entry points; its records are checked word for word against the textbook wavelet matrix of the tokens. So
does the derived 4-ary layout (cf_rrrw_quads_*): its records, digit bucket starts and walk table are checked word
for word against a 4-ary wavelet matrix built here from the tokens by stable sorts. Bit-exact throughout.
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


def _index(arrays, dev):
    from chromofold_amd.search import RrrWaveletIndex
    return RrrWaveletIndex.from_host(arrays, dev)


def _lines_access(idx, pos):
    from chromofold_amd.search import to_u32, u32_dev
    dp = u32_dev(pos)
    out = dp.clone()
    idx.access_lines_into(dp, out)
    return to_u32(out)


def _lines_rank(idx, c, i):
    from chromofold_amd.search import to_u32, u32_dev
    dc, di = u32_dev(c), u32_dev(i)
    out = di.clone()
    idx.rank_lines_into(dc, di, out)
    return to_u32(out)


def _check_lines_layout(idx, tok, bits):
    from test_gpu_fm_lines import check_layout, expected_lines
    recs, base = expected_lines(np.asarray(tok), bits, np.zeros(1 << bits, np.int32), 2 * idx.nsb + 1)
    check_layout(idx.build_lines(), bits, recs, base)


def expected_quads(tok, bits, X=None):
    """The 4-ary wavelet matrix of `tok` as the layout stores it: records [L4][nrec][16] (counts of digits 0..2
    before the record, then 13 words of 16 two-bit digits), Z [L4][4] and base[c] = X[c] - (end of the walk of c
    from 0) for c < X.size (X = zeros of 2^bits when not given), built with numpy stable sorts and cumulative
    counts."""
    tok = np.asarray(tok, np.uint32)
    L4, n = (bits + 1) // 2, tok.size
    nrec = n // 208 + 1
    recs = np.zeros((L4, nrec, 16), np.uint32)
    Z = np.zeros((L4, 4), np.uint32)
    cums, S = [], tok.copy()
    for lvl in range(L4):
        d = (S >> np.uint32(2 * (L4 - 1 - lvl))) & np.uint32(3)
        cl = [np.concatenate([[0], np.cumsum(d == v)]).astype(np.int64) for v in range(4)]
        cums.append(cl)
        starts = np.minimum(np.arange(nrec) * 208, n)
        for v in range(3):
            recs[lvl, :, v] = cl[v][starts]
        dp = np.zeros(nrec * 208, np.uint32)
        dp[:n] = d
        dp = dp.reshape(nrec, 13, 16)
        for j in range(16):
            recs[lvl, :, 3:] |= dp[:, :, j] << np.uint32(2 * j)
        tot = [int(cl[v][n]) for v in range(4)]
        Z[lvl] = [0, tot[0], tot[0] + tot[1], tot[0] + tot[1] + tot[2]]
        S = S[np.argsort(d, kind="stable")]
    X = np.zeros(1 << bits, np.int64) if X is None else np.asarray(X, np.int64)
    cs = np.arange(X.size, dtype=np.int64)
    pw = np.zeros(cs.size, np.int64)
    for lvl in range(L4):
        d = (cs >> (2 * (L4 - 1 - lvl))) & 3
        pw = Z[lvl][d].astype(np.int64) + np.choose(d, [cums[lvl][v][pw] for v in range(4)])
    return recs, Z, (X - pw).astype(np.int32)


def _quads(idx, tok, bits):
    """Builds the 4-ary layout and checks it word for word against expected_quads."""
    n = len(tok)
    q = idx.build_quads(n).cpu().numpy().view(np.uint32)
    recs, Z, base = expected_quads(tok, bits)
    nw = recs.size
    assert np.array_equal(q[:nw].reshape(recs.shape), recs)
    assert np.array_equal(q[nw:nw + Z.size].reshape(Z.shape), Z)
    assert np.array_equal(q[nw + Z.size:nw + Z.size + base.size].view(np.int32), base)


def _quads_access(idx, pos):
    from chromofold_amd.search import to_u32, u32_dev
    dp = u32_dev(pos)
    out = dp.clone()
    idx.access_quads_into(dp, out)
    return to_u32(out)


def _quads_rank(idx, c, i):
    from chromofold_amd.search import to_u32, u32_dev
    dc, di = u32_dev(c), u32_dev(i)
    out = di.clone()
    idx.rank_quads_into(dc, di, out)
    return to_u32(out)


def test_tiny_cfrw_fixture(dev):
    from chromofold_amd.search import to_u32, u32_dev
    d = F.load_cfrw()
    idx = _index(d, dev)
    assert np.array_equal(to_u32(idx.access(u32_dev(d["pos"]))), d["access_golden"])
    assert np.array_equal(to_u32(idx.rank(u32_dev(d["rank_c"]), u32_dev(d["rank_i"]))), d["rank_golden"])
    # every position of the fixture, against the oracle
    allpos = np.arange(d["n"], dtype=np.uint32)
    w = O.RrrwArrays(d["bits"], d["cwords"], d["nsb"], d["na"], d["classes"], d["offsets"], d["rank_a"],
                     d["rank_d"], d["off_a"], d["off_d"], d["offbase"], d["zeros"])
    ref = O.rrrw_access(w, allpos)
    assert np.array_equal(to_u32(idx.access(u32_dev(allpos))), ref)
    _check_lines_layout(idx, ref, d["bits"])
    assert np.array_equal(_lines_access(idx, allpos), ref)
    assert np.array_equal(_lines_access(idx, d["pos"]), d["access_golden"])
    assert np.array_equal(_lines_rank(idx, d["rank_c"], d["rank_i"]), d["rank_golden"])
    _quads(idx, ref, d["bits"])
    assert np.array_equal(_quads_access(idx, allpos), ref)
    assert np.array_equal(_quads_access(idx, d["pos"]), d["access_golden"])
    assert np.array_equal(_quads_rank(idx, d["rank_c"], d["rank_i"]), d["rank_golden"])


# sizes at and just past the 4-ary layout's 208-digit records (208, 209, 416, 624), and 22 / 24 bits (the layouts'
# widest symbols)
@pytest.mark.parametrize("n,bits,seed", [(1, 1, 1), (15, 3, 2), (16, 4, 3), (961, 5, 4), (4095, 9, 5),
                                         (65536, 15, 6), (100003, 16, 7), (30000, 17, 8), (208, 2, 9), (416, 6, 10),
                                         (209, 7, 11), (624, 8, 12), (20000, 22, 13), (3000, 24, 14)])
def test_random_shapes_vs_closed_form(dev, n, bits, seed):
    from chromofold_amd.search import to_u32, u32_dev
    rng = np.random.default_rng(seed)
    tok = rng.integers(0, 1 << bits, n).astype(np.uint32)
    w = O.rrrw_build(tok, bits)
    idx = _index(w, dev)
    allpos = np.arange(n, dtype=np.uint32)
    assert np.array_equal(to_u32(idx.access(u32_dev(allpos))), tok)
    c = np.concatenate([tok[rng.integers(0, n, 500)], rng.integers(0, 1 << bits, 500).astype(np.uint32)])
    i = rng.integers(0, n + 1, c.size).astype(np.uint32)
    i[:3] = [0, n, n // 2]  # edges: empty prefix, whole sequence
    got = to_u32(idx.rank(u32_dev(c), u32_dev(i)))
    assert np.array_equal(got, O.rrrw_rank(w, c, i))
    _check_lines_layout(idx, tok, bits)
    assert np.array_equal(_lines_access(idx, allpos), tok)
    assert np.array_equal(_lines_rank(idx, c, i), got)
    hi = c | np.uint32(1 << 31)  # bits above the levels are ignored, as by the RRR walk
    assert np.array_equal(_lines_rank(idx, hi, i), to_u32(idx.rank(u32_dev(hi), u32_dev(i))))
    _quads(idx, tok, bits)
    assert np.array_equal(_quads_access(idx, allpos), tok)
    assert np.array_equal(_quads_rank(idx, c, i), got)
    assert np.array_equal(_quads_rank(idx, hi, i), got)


def test_c1_shape_zipf_closed_form(dev):
    """C1: 1,048,576 Zipf(1.1) tokens over vocab 32000 (15 levels); 1M access + 1M rank queries."""
    import torch
    from chromofold_amd import synth
    from chromofold_amd.search import to_u32, u32_dev
    n, vocab = 1 << 20, 32000
    tok = synth.zipf_tokens(n, vocab, 1.1, synth.SEED_C1)
    w = O.rrrw_build(tok, 15)
    idx = _index(w, dev)
    pos, c, i = synth.rrr_queries(tok, 1 << 20, vocab, synth.SEED_C1 + 1)
    got = to_u32(idx.access(u32_dev(pos)))
    assert np.array_equal(got, tok[pos])
    gr = to_u32(idx.rank(u32_dev(c), u32_dev(i)))
    # closed form on a sample (exact counting), the oracle on everything
    order = np.argsort(tok, kind="stable")
    sorted_tok = tok[order]
    for t in range(0, c.size, 4099):
        lo, hi = np.searchsorted(sorted_tok, c[t], "left"), np.searchsorted(sorted_tok, c[t], "right")
        assert gr[t] == np.count_nonzero(order[lo:hi] < i[t]), t
    assert np.array_equal(gr, O.rrrw_rank(w, c, i))
    assert np.array_equal(_lines_access(idx, pos), got)
    assert np.array_equal(_lines_rank(idx, c, i), gr)
    _check_lines_layout(idx, tok, 15)
    _quads(idx, tok, 15)
    assert np.array_equal(_quads_access(idx, pos), got)
    assert np.array_equal(_quads_rank(idx, c, i), gr)
    torch.cuda.synchronize()


def test_quads_entry_points_reject_bad_arguments(dev):
    """The 4-ary layout's host-side checks: byte counts 0 past 24 bits or past what the levels hold, and builds or
    queries with short buffers, NULL or misaligned pointers refused before any launch; an empty query is a no-op."""
    import torch
    from chromofold_amd import _abi as A
    rng = np.random.default_rng(77)
    n, bits = 5000, 11
    tok = rng.integers(0, 1 << bits, n).astype(np.uint32)
    idx = _index(O.rrrw_build(tok, bits), dev)
    v = idx.view()
    L = A.lib()
    nb, nw = int(L.cf_rrrw_quads_bytes(v, n)), int(L.cf_rrrw_quads_workspace_bytes(v, n))
    assert nb > 0 and nw > 0
    assert int(L.cf_rrrw_quads_bytes(v, idx.nsb * 960 + 1)) == 0
    bad = A.cf_rrrw_view.from_buffer_copy(v)
    bad.bits = 25
    assert int(L.cf_rrrw_quads_bytes(bad, n)) == 0
    q = torch.empty(nb + 16, dtype=torch.uint8, device=dev)
    ws = torch.empty(nw, dtype=torch.uint8, device=dev)
    INV = A.CF_ERR_INVALID_ARGUMENT
    assert L.cf_rrrw_quads_build_async(v, n, q.data_ptr(), nb - 4, ws.data_ptr(), nw, None) == INV
    assert L.cf_rrrw_quads_build_async(v, n, q.data_ptr(), nb, ws.data_ptr(), nw - 4, None) == INV
    assert L.cf_rrrw_quads_build_async(v, n, q.data_ptr(), nb, None, nw, None) == INV
    assert L.cf_rrrw_quads_build_async(v, n, q.data_ptr() + 4, nb, ws.data_ptr(), nw, None) == INV
    out = torch.zeros(4, dtype=torch.int32, device=dev)
    assert L.cf_rrrw_access_quads_async(v, n, None, out.data_ptr(), out.data_ptr(), 4, None) == INV
    assert L.cf_rrrw_rank_quads_async(v, n, q.data_ptr(), None, out.data_ptr(), out.data_ptr(), 4, None) == INV
    assert L.cf_rrrw_access_quads_async(v, n, q.data_ptr(), out.data_ptr(), out.data_ptr(), 0, None) == A.CF_OK
    torch.cuda.synchronize()
