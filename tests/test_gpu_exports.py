"""GPU parity of the remaining exported entry points against the oracle / closed forms, through the C ABI:

  packed wavelet  cf_access_async, cf_rank_async, cf_rank2_async, cf_embedding_gather(_tpq)_async
                  (tiny.cfwv goldens + raw tokens; random indexes at every specialised level count)
  RRR bitvector   cf_rrr_rank_async (tiny.cfrr goldens; prefix popcount of random planes)
  RRR sparse      cf_sparse_gather_fused_async, cf_sparse_decode_all_async, cf_sparse_gather_async
  delta fetch     cf_delta_fetch_async (closed form: base overridden by the leaf's delta)
  block rANS      cf_rans_decode_async (symbols the encoder was given, bit for bit)
  windowed KV     cf_kv_attn_fused_async / cf_kv_attn_dense_async (fp64 oracle, 1e-3 normwise; fused == dense
                  bit for bit)
Bar: bit-exact for every integer/index/gather result; attention within 1e-3 normwise relative.
"""
import ctypes as C

import numpy as np
import pytest

import cf_fixtures as F
import oracle as O
from legacy_helpers import canonical_codes, huffman_lengths, huffman_stream_np, rans_encode_blocks

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _d(a, dev):
    from chromofold_amd.search import _dev
    return _dev(np.ascontiguousarray(a), dev)


def _np(t, dtype):
    return t.cpu().numpy().view(dtype)


def _lib():
    from chromofold_amd import _abi
    return _abi.lib()


def _ok(st, what):
    from chromofold_amd import _abi
    _abi.check(st, what)


def _sync():
    import torch
    torch.cuda.synchronize()


def _wview(bp, sb, z, levels, nwords, nblocks, n, keep):
    from chromofold_amd import _abi
    keep += [bp, sb, z]
    return _abi.cf_wavelet_view(bp.data_ptr(), sb.data_ptr(), z.data_ptr(), n, levels, nwords, nblocks)


def _two_level(bp_host, levels, nwords, CB):
    """coarse[level * ncoarse + w / CB] + fine[level * (nwords + 1) + w] = set bits of the level before word w."""
    ncoarse = nwords // CB + 1
    coarse = np.zeros(levels * ncoarse, np.int32)
    fine = np.zeros(levels * (nwords + 1), np.uint16)
    for lvl in range(levels):
        w = bp_host[lvl * nwords:(lvl + 1) * nwords]
        pc = np.array([bin(int(x)).count("1") for x in w], np.int64)
        pre = np.concatenate([[0], np.cumsum(pc)])  # nwords + 1 prefixes
        idx = np.arange(nwords + 1)
        c = pre[(idx // CB) * CB]
        coarse[lvl * ncoarse:(lvl + 1) * ncoarse] = pre[np.arange(ncoarse) * CB].astype(np.int32)
        fine[lvl * (nwords + 1):(lvl + 1) * (nwords + 1)] = (pre - c).astype(np.uint16)
    return coarse, fine, ncoarse


def _packed_case(dev, tokens, levels, seed):
    rng = np.random.default_rng(seed)
    n = tokens.size
    bp, sb, z, nwords, nblocks = O.packed_build(tokens, levels)
    keep = []
    v = _wview(_d(bp, dev), _d(sb, dev), _d(z, dev), levels, nwords, nblocks, n, keep)
    import torch
    pos = rng.integers(0, n, 3000).astype(np.uint32)
    out = torch.empty(pos.size, dtype=torch.int32, device=dev)
    dpos = _d(pos, dev)  # (keep device buffers referenced until the kernels have run)
    _ok(_lib().cf_access_async(v, dpos.data_ptr(), out.data_ptr(), pos.size, None), "access")
    assert np.array_equal(_np(out, np.uint32), tokens[pos])
    c = np.where(rng.random(3000) < 0.5, tokens[rng.integers(0, n, 3000)], rng.integers(0, 1 << levels, 3000))
    c = c.astype(np.uint32)
    i = rng.integers(0, n + 1, 3000).astype(np.uint32)
    exp = O.packed_rank(bp, sb, z, levels, nwords, nblocks, c, i)
    dc, di = _d(c, dev), _d(i, dev)
    _ok(_lib().cf_rank_async(v, dc.data_ptr(), di.data_ptr(), out.data_ptr(), i.size, None), "rank")
    assert np.array_equal(_np(out, np.uint32), exp)
    for CB in (4, 32):
        coarse, fine, ncoarse = _two_level(bp, levels, nwords, CB)
        dco, dfi = _d(coarse, dev), _d(fine, dev)
        out2 = torch.full((i.size,), -1, dtype=torch.int32, device=dev)
        _ok(_lib().cf_rank2_async(v, dco.data_ptr(), dfi.data_ptr(), ncoarse, CB, dc.data_ptr(), di.data_ptr(),
                                  out2.data_ptr(), i.size, None), "rank2")
        assert np.array_equal(_np(out2, np.uint32), exp)
    # gathers: vector path (dim % 4 == 0), scalar path (odd dim), short rows, a ragged last wave
    V = 1 << levels
    for dim, count in ((64, 1000), (7, 130), (256, 65), (3, 64)):
        E = rng.standard_normal((V, dim)).astype(np.float32)
        dE = torch.from_numpy(E).to(dev)
        gp = rng.integers(0, n, count).astype(np.uint32)
        dgp = _d(gp, dev)
        for fn in ("cf_embedding_gather_async", "cf_embedding_gather_tpq_async"):
            g = torch.full((count, dim), float("nan"), device=dev)
            _ok(getattr(_lib(), fn)(v, dE.data_ptr(), dim, dgp.data_ptr(), g.data_ptr(), count, None), fn)
            assert np.array_equal(g.cpu().numpy(), E[tokens[gp]]), (fn, dim)
    _sync()


def test_packed_wavelet_fixture(dev):
    d = F.load_cfwv()
    tok = d["tokens"]
    bp, sb, z, nwords, nblocks = O.packed_build(tok, d["levels"])
    assert np.array_equal(bp, d["bitplanes"]) and np.array_equal(sb, d["superblocks"])
    keep = []
    v = _wview(_d(bp, dev), _d(sb, dev), _d(z, dev), d["levels"], nwords, nblocks, d["n"], keep)
    import torch
    out = torch.empty(d["pos"].size, dtype=torch.int32, device=dev)
    dpos = _d(d["pos"], dev)
    _ok(_lib().cf_access_async(v, dpos.data_ptr(), out.data_ptr(), d["pos"].size, None), "access")
    assert np.array_equal(_np(out, np.uint32), d["access_golden"])
    out = torch.empty(d["rank_i"].size, dtype=torch.int32, device=dev)
    dc, di = _d(d["rank_c"], dev), _d(d["rank_i"], dev)
    _ok(_lib().cf_rank_async(v, dc.data_ptr(), di.data_ptr(), out.data_ptr(), d["rank_i"].size, None), "rank")
    assert np.array_equal(_np(out, np.uint32), d["rank_golden"])
    _packed_case(dev, tok, d["levels"], 1)


@pytest.mark.parametrize("levels,n", [(2, 5000), (4, 777), (8, 20011), (15, 30000), (5, 4097)])
def test_packed_wavelet_random(dev, levels, n):
    rng = np.random.default_rng(levels * 7 + n)
    ranks = np.arange(1, (1 << levels) + 1, dtype=np.float64)
    p = ranks ** -1.1
    tok = rng.choice(1 << levels, size=n, p=p / p.sum()).astype(np.uint32)
    _packed_case(dev, tok, levels, levels)


def test_rrr_bitvector_rank(dev):
    import torch
    d = F.load_cfrr()
    args = [_d(d[k], dev) for k in ("classes", "offsets", "sbrank", "sboff")]
    out = torch.empty(d["pos"].size, dtype=torch.int32, device=dev)
    dpos = _d(d["pos"], dev)
    _ok(_lib().cf_rrr_rank_async(*[a.data_ptr() for a in args], None, None, dpos.data_ptr(), out.data_ptr(),
                                 d["pos"].size, None), "rrr_rank")
    assert np.array_equal(_np(out, np.uint32), d["rank_golden"])
    rng = np.random.default_rng(9)
    for n, dens in ((1, 0.5), (15, 0.3), (64 * 15 + 1, 0.02), (100003, 0.4), (50000, 0.97)):
        bits = (rng.random(n) < dens).astype(np.uint8)
        pl = O.rrr_plane_build(bits)
        args = [_d(pl[k], dev) for k in ("classes", "offsets", "sbrank", "sboff")]
        pos = np.concatenate([[0, n], rng.integers(0, n + 1, 4000)]).astype(np.uint32)
        out = torch.empty(pos.size, dtype=torch.int32, device=dev)
        dpos = _d(pos, dev)
        _ok(_lib().cf_rrr_rank_async(*[a.data_ptr() for a in args], None, None, dpos.data_ptr(), out.data_ptr(),
                                     pos.size, None), "rrr_rank")
        pre = np.concatenate([[0], np.cumsum(bits)])
        assert np.array_equal(_np(out, np.uint32), pre[pos].astype(np.uint32)), n


@pytest.mark.parametrize("bits,n", [(7, 4000), (15, 25000), (6, 999), (9, 3000)])
def test_rrr_sparse_gathers(dev, bits, n):
    import torch
    from chromofold_amd.search import RrrWaveletIndex
    rng = np.random.default_rng(bits + n)
    tok = rng.integers(0, 1 << bits, n).astype(np.uint32)
    w = O.rrrw_build(tok, bits)
    idx = RrrWaveletIndex.from_host(w, dev)
    v = idx.view()
    ids = torch.full((n,), -1, dtype=torch.int32, device=dev)
    _ok(_lib().cf_sparse_decode_all_async(v, ids.data_ptr(), n, None), "decode_all")
    assert np.array_equal(_np(ids, np.uint32), tok)
    V = 1 << bits
    # row lengths: 16-byte rows of 8 and 32 units, float rows of 5 units (one unit per lane and pass) and of 300
    # units (several per lane)
    for dim, K in ((32, 700), (5, 200), (128, 333), (300, 130)):
        E = rng.standard_normal((V, dim)).astype(np.float32)
        dE = torch.from_numpy(E).to(dev)
        pos = rng.integers(0, n, K).astype(np.uint32)
        dp = _d(pos, dev)
        g = torch.full((K, dim), float("nan"), device=dev)
        _ok(_lib().cf_sparse_gather_fused_async(v, dE.data_ptr(), dim, dp.data_ptr(), g.data_ptr(), K, None), "fused")
        assert np.array_equal(g.cpu().numpy(), E[tok[pos]])
        g3 = torch.full((K, dim), float("nan"), device=dev)
        idx.gather_fused_lines_into(dE, dp, g3)  # the same gather over the line layout
        assert np.array_equal(g3.cpu().numpy(), E[tok[pos]])
        g4 = torch.full((K, dim), float("nan"), device=dev)
        idx.build_quads(n)
        idx.gather_fused_quads_into(dE, dp, g4)  # and over the 4-ary layout
        assert np.array_equal(g4.cpu().numpy(), E[tok[pos]])
        g2 = torch.full((K, dim), float("nan"), device=dev)
        _ok(_lib().cf_sparse_gather_async(ids.data_ptr(), dE.data_ptr(), dim, dp.data_ptr(), g2.data_ptr(), K, None),
            "gather")
        assert np.array_equal(g2.cpu().numpy(), E[tok[pos]])


def test_delta_fetch(dev):
    import torch
    rng = np.random.default_rng(5)
    nbase, leaves = 8000, 37
    base = rng.integers(0, 32000, nbase).astype(np.int32)
    dpos, dval, dstart, dlen = [], [], [], []
    for leaf in range(leaves):
        k = int(rng.integers(0, 200)) if leaf % 5 else 0  # some leaves carry no delta
        p = np.sort(rng.choice(nbase + 64, size=k, replace=False)).astype(np.int32)  # deltas may extend the base
        dstart.append(len(dpos))
        dlen.append(k)
        dpos.extend(p)
        dval.extend(rng.integers(0, 32000, k))
    dpos, dval = np.array(dpos + [0], np.int32), np.array(dval + [0], np.int32)
    dstart, dlen = np.array(dstart, np.int32), np.array(dlen, np.int32)
    Q = 50000
    leaf = rng.integers(0, leaves, Q).astype(np.int32)
    pos = rng.integers(0, nbase + 64, Q).astype(np.int32)
    exp = np.where(pos < nbase, base[np.minimum(pos, nbase - 1)], -1).astype(np.int32)
    for t in range(Q):  # closed form: the leaf's own delta wins
        s, l = dstart[leaf[t]], dlen[leaf[t]]
        hit = np.nonzero(dpos[s:s + l] == pos[t])[0]
        if hit.size:
            exp[t] = dval[s + hit[0]]
    out = torch.empty(Q, dtype=torch.int32, device=dev)
    a = [_d(x, dev) for x in (base, dpos, dval, dstart, dlen, leaf, pos)]
    _ok(_lib().cf_delta_fetch_async(a[0].data_ptr(), nbase, *[x.data_ptr() for x in a[1:]], out.data_ptr(), Q, None),
        "delta")
    assert np.array_equal(out.cpu().numpy(), exp)


def test_delta_fetch_edges(dev):
    """Leaf lengths 1..9 (around the search's switch to its final scan) and 3000, repeated delta positions (the
    first one's value wins), queries at every delta position, one before and one after it, and negative positions
    (-1, like a position past the base)."""
    import torch
    rng = np.random.default_rng(11)
    nbase = 5000
    base = rng.integers(0, 1 << 30, nbase).astype(np.int32)
    dpos, dval, dstart, dlen = [], [], [], []
    for k in list(range(0, 10)) + [3000, 64, 65, 255]:
        p = np.sort(rng.integers(0, nbase + 10, k)).astype(np.int32)  # with repeats
        dstart.append(len(dpos))
        dlen.append(k)
        dpos.extend(p)
        dval.extend(rng.integers(0, 1 << 30, k))
    leaves = len(dlen)
    dpos, dval = np.array(dpos + [0], np.int32), np.array(dval + [0], np.int32)
    dstart, dlen = np.array(dstart, np.int32), np.array(dlen, np.int32)
    leaf, pos = [], []
    for lf in range(leaves):
        s, n = dstart[lf], dlen[lf]
        for v in list(dpos[s:s + n]) + [0, nbase - 1, nbase, nbase + 9, -1, -7]:
            for dv in (-1, 0, 1):
                leaf.append(lf)
                pos.append(int(v) + dv)
    leaf, pos = np.array(leaf, np.int32), np.array(pos, np.int32)
    exp = np.where((pos >= 0) & (pos < nbase), base[np.clip(pos, 0, nbase - 1)], -1).astype(np.int32)
    for t in range(pos.size):
        s, n = dstart[leaf[t]], dlen[leaf[t]]
        hit = np.nonzero(dpos[s:s + n] == pos[t])[0]
        if hit.size:
            exp[t] = dval[s + hit[0]]
    Q = pos.size
    out = torch.empty(Q, dtype=torch.int32, device=dev)
    a = [_d(x, dev) for x in (base, dpos, dval, dstart, dlen, leaf, pos)]
    _ok(_lib().cf_delta_fetch_async(a[0].data_ptr(), nbase, *[x.data_ptr() for x in a[1:]], out.data_ptr(), Q, None),
        "delta")
    assert np.array_equal(out.cpu().numpy(), exp)


@pytest.mark.parametrize("n,V,block", [(50000, 16, 64), (30001, 256, 1024), (4096, 4, 1), (1000, 9, 333)])
def test_rans_decode(dev, n, V, block):
    import torch
    rng = np.random.default_rng(n + V)
    p = rng.dirichlet(np.ones(V) * 0.7)
    sym = rng.choice(V, size=n, p=p)
    cnt = np.bincount(sym, minlength=V)
    f = np.maximum(1, cnt * 4096 // cnt.sum()).astype(np.int64)
    f[cnt == 0] = 0
    f[np.argmax(f)] += 4096 - f.sum()
    enc = rans_encode_blocks(sym, f, block)
    assert np.array_equal(O.rans_block_decode(*enc, block, n), sym)
    a = [_d(x, dev) for x in enc]
    out = torch.full((n,), -1, dtype=torch.int32, device=dev)
    _ok(_lib().cf_rans_decode_async(*[x.data_ptr() for x in a], block, n, out.data_ptr(), None), "rans")
    assert np.array_equal(out.cpu().numpy(), sym)


def _kivi_huffman(x, per_token, bits, maxlen, block, rng):
    """KIVI int quantisation (K per channel, V per token) + canonical Huffman; returns stream, scales, dequant."""
    qmax = (1 << (bits - 1)) - 1
    zero = 1 << (bits - 1)
    amax = np.abs(x).max(axis=1 if per_token else 0)
    sc = np.where(amax > 0, amax / qmax, 1.0).astype(np.float32)
    q = np.clip(np.rint(x / (sc[:, None] if per_token else sc[None, :])), -qmax - 1, qmax).astype(np.int64) + zero
    L = huffman_lengths(np.bincount(q.ravel(), minlength=1 << bits), maxlen)
    w, b, lut = huffman_stream_np(q.ravel(), L, maxlen, block)
    deq = ((q - zero).astype(np.float32) * (sc[:, None] if per_token else sc[None, :])).astype(np.float32)
    return w, b, lut, sc, deq, zero


@pytest.mark.parametrize("seq,dim,nq,window,block,bits,maxlen", [
    (600, 128, 600, 256, 64, 4, 8), (300, 64, 250, 512, 64, 8, 12), (133, 96, 133, 1, 50, 4, 6),
    (1000, 32, 777, 100, 128, 8, 14), (70, 128, 0, 16, 64, 4, 8)])
def test_kv_window_attention(dev, seq, dim, nq, window, block, bits, maxlen):
    import torch
    rng = np.random.default_rng(seq + dim)
    K = rng.standard_normal((seq, dim)).astype(np.float32)
    V = rng.standard_normal((seq, dim)).astype(np.float32)
    Q = rng.standard_normal((seq, dim)).astype(np.float32)
    kw, kb, kl, ksc, kd, zero = _kivi_huffman(K, False, bits, maxlen, block, rng)
    vw, vb, vl, vsc, vd, _ = _kivi_huffman(V, True, bits, maxlen, block, rng)
    ss = 1.0 / np.sqrt(dim)
    a = [_d(x, dev) for x in (kw, kb, kl, vw, vb, vl, ksc, vsc, Q)]
    outf = torch.full((seq, dim), 7.0, device=dev)
    outd = torch.full((seq, dim), 7.0, device=dev)
    Kd = torch.empty((seq, dim), device=dev)
    Vd = torch.empty((seq, dim), device=dev)
    p = [x.data_ptr() for x in a]
    _ok(_lib().cf_kv_attn_fused_async(p[0], p[1], p[2], maxlen, p[3], p[4], p[5], maxlen, p[6], p[7], p[8],
                                      outf.data_ptr(), seq, dim, nq, window, block, zero, ss, None), "fused")
    _ok(_lib().cf_kv_attn_dense_async(p[0], p[1], p[2], maxlen, p[3], p[4], p[5], maxlen, p[6], p[7], p[8],
                                      Kd.data_ptr(), Vd.data_ptr(), outd.data_ptr(), seq, dim, nq, window, block,
                                      zero, ss, None), "dense")
    gf, gd = outf.cpu().numpy(), outd.cpu().numpy()
    assert np.array_equal(gf, gd), "fused and dense paths must agree bit for bit"
    assert (gf[nq:] == 7.0).all()  # rows past nq untouched
    if nq:
        assert np.array_equal(Kd.cpu().numpy(), kd) and np.array_equal(Vd.cpu().numpy(), vd)  # exact dequant
        ref = O.kv_window_attention_f64(kd, vd, Q, nq, window, ss)
        err = np.abs(gf[:nq] - ref).max() / np.abs(ref).max()
        assert err <= 1e-3, err


def test_kv_window_attention_contract(dev):
    """reference fused_kv_attention.cu:101-113: null -> INVALID, dim > 128 / window > 512 -> UNSUPPORTED."""
    from chromofold_amd import _abi
    import torch
    L = _lib()
    t = torch.zeros(16, device=dev)
    p = t.data_ptr()
    args = lambda dim, window, nq=1: (p, p, p, 4, p, p, p, 4, p, p, p, p, 8, dim, nq, window, 64, 8, 1.0, None)
    assert L.cf_kv_attn_fused_async(*args(129, 4)) == _abi.CF_ERR_UNSUPPORTED
    assert L.cf_kv_attn_fused_async(*args(64, 513)) == _abi.CF_ERR_UNSUPPORTED
    assert L.cf_kv_attn_fused_async(*args(64, 4, 9)) == _abi.CF_ERR_INVALID_ARGUMENT  # nq > seq
    assert L.cf_kv_attn_fused_async(None, p, p, 4, p, p, p, 4, p, p, p, p, 8, 4, 1, 4, 64, 8, 1.0,
                                    None) == _abi.CF_ERR_INVALID_ARGUMENT
    assert L.cf_kv_attn_fused_async(p, p, p, 4, p, p, p, 4, p, p, p, p, 8, 4, 1, 4, 64, 8, float("nan"),
                                    None) == _abi.CF_ERR_INVALID_ARGUMENT
