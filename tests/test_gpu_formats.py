"""Exchange files drive the kernels: each format is written by chromofold_amd.formats from payloads made by the
test encoders, with the golden section computed independently (closed forms or the float64 oracle); the file is
read back and the kernel that consumes it runs on the arrays read from the file:

  .cfrs -> cf_rans_decode_async (bit-exact against golden)
  .cffw -> cf_fused_matmul_async (golden = float64 oracle product; 1e-3 relative)
  .cfkv -> cf_kv_attn_fused_async (golden = float64 windowed attention; 1e-3 relative)
  .cfdc -> cf_delta_fetch_async (every position of every sequence equals originals; bit-exact)
  .cfsg -> cf_sparse_gather_fused_async (golden = emb[token[pos]]; bit-exact)
"""
import numpy as np
import pytest

import oracle as O
from legacy_helpers import huffman_lengths, huffman_stream_np, rans_encode_blocks

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


def _lib():
    from chromofold_amd import _abi
    return _abi.lib()


def _ok(st, what):
    from chromofold_amd import _abi
    _abi.check(st, what)


def _roundtrip(tmp_path, kind, fields):
    from chromofold_amd import formats as X
    p = str(tmp_path / f"t.{kind}")
    X.write(p, kind, fields)
    k, d = X.read(p)
    assert k == kind
    return d


def test_cfrs_drives_rans_decode(dev, tmp_path):
    import torch
    rng = np.random.default_rng(1)
    n, V, block = 20000, 12, 256
    sym = rng.choice(V, size=n, p=rng.dirichlet(np.ones(V)))
    cnt = np.bincount(sym, minlength=V)
    f = np.maximum(1, cnt * 4096 // cnt.sum()).astype(np.int64)
    f[cnt == 0] = 0
    f[np.argmax(f)] += 4096 - f.sum()
    data, boff, st0, s2s, freq, cum = rans_encode_blocks(sym, f, block)
    p = cnt[cnt > 0] / n
    d = _roundtrip(tmp_path, "cfrs", dict(n=n, block=block, V=V, M=4096, nblocks=boff.size, data_bytes=data.size,
                                          slotlen=s2s.size, h0=float(-(p * np.log2(p)).sum()),
                                          rans_bits=8 * data.size, huff_bits=0, data=data, byte_off=boff,
                                          state0=st0, slot2sym=s2s, freq=freq, cum=cum, golden=sym))
    a = [_d(d[k], dev) for k in ("data", "byte_off", "state0", "slot2sym", "freq", "cum")]
    out = torch.full((d["n"],), -1, dtype=torch.int32, device=dev)
    _ok(_lib().cf_rans_decode_async(*[x.data_ptr() for x in a], d["block"], d["n"], out.data_ptr(), None), "rans")
    assert np.array_equal(out.cpu().numpy(), d["golden"])


def test_cffw_drives_fused_matmul(dev, tmp_path):
    import torch
    from chromofold_amd import qw
    rng = np.random.default_rng(2)
    M, K, B, block, maxlen, bits = 96, 700, 5, 64, 8, 4
    W = rng.standard_normal((M, K)) / np.sqrt(K)
    scale = np.float32(np.abs(W).max() / 7)
    sym = (np.clip(np.rint(W / scale), -8, 7) + 8).astype(np.int64)
    words, boff, lut = huffman_stream_np(sym.ravel(), huffman_lengths(np.bincount(sym.ravel(), minlength=16), maxlen),
                                         maxlen, block)
    x = rng.standard_normal((B, K)).astype(np.float32)
    y = O.qmatmul_f64(x, sym, scale, 8).astype(np.float32)
    d = _roundtrip(tmp_path, "cffw", dict(M=M, K=K, B=B, bits=bits, block=block, maxlen=maxlen, zero=8,
                                          nwords=words.size, nblocks=boff.size, lutlen=lut.size, scale=float(scale),
                                          resident_bytes=words.nbytes + boff.nbytes + lut.nbytes,
                                          dense_bytes=M * K * 4, words=words, block_off=boff, lut=lut, x=x,
                                          y_golden=y))
    dw, db, dl = (_d(d[k].view(np.int32) if d[k].dtype == np.uint32 else d[k], dev)
                  for k in ("words", "block_off", "lut"))
    dx = _d(d["x"].reshape(d["B"], d["K"]), dev)
    yf = torch.full((d["B"], d["M"]), float("nan"), device=dev)
    qw.fused_matmul(dw, db, dl, d["maxlen"], d["block"], dx, yf, d["M"], d["K"], float(d["scale"]), d["zero"])
    torch.cuda.synchronize()
    ref = d["y_golden"].reshape(d["B"], d["M"])
    assert np.abs(yf.cpu().numpy() - ref).max() / np.abs(ref).max() <= 1e-3


def test_cfkv_drives_window_attention(dev, tmp_path):
    import torch
    rng = np.random.default_rng(3)
    seq, dim, nq, window, block, bits, maxlen = 200, 64, 150, 40, 64, 4, 8
    K = rng.standard_normal((seq, dim)).astype(np.float32)
    V = rng.standard_normal((seq, dim)).astype(np.float32)
    Q = rng.standard_normal((nq, dim)).astype(np.float32)
    zero = 8

    def kivi(x, per_token):
        amax = np.abs(x).max(axis=1 if per_token else 0)
        sc = np.where(amax > 0, amax / 7, 1.0).astype(np.float32)
        q = np.clip(np.rint(x / (sc[:, None] if per_token else sc[None, :])), -8, 7).astype(np.int64) + zero
        w, b, lut = huffman_stream_np(q.ravel(), huffman_lengths(np.bincount(q.ravel(), minlength=16), maxlen),
                                      maxlen, block)
        deq = ((q - zero).astype(np.float32) * (sc[:, None] if per_token else sc[None, :])).astype(np.float32)
        return w, b, lut, sc, deq

    kw, kb, kl, ksc, kd = kivi(K, False)
    vw, vb, vl, vsc, vd = kivi(V, True)
    ss = 1.0 / np.sqrt(dim)
    golden = O.kv_window_attention_f64(kd, vd, np.concatenate([Q, np.zeros((seq - nq, dim), np.float32)]), nq,
                                        window, ss)[:nq].astype(np.float32)
    d = _roundtrip(tmp_path, "cfkv", dict(seq=seq, dim=dim, nq=nq, window=window, bits=bits, block=block, zero=zero,
                                          kmaxlen=maxlen, knwords=kw.size, knblocks=kb.size, klutlen=kl.size,
                                          vmaxlen=maxlen, vnwords=vw.size, vnblocks=vb.size, vlutlen=vl.size,
                                          softmax_scale=ss, resident_bytes=0, dense_bytes=2 * seq * dim * 4,
                                          kwords=kw, kboff=kb, klut=kl, vwords=vw, vboff=vb, vlut=vl, kscale=ksc,
                                          vscale=vsc, Q=Q, golden=golden))
    qfull = np.zeros((d["seq"], d["dim"]), np.float32)
    qfull[:d["nq"]] = d["Q"].reshape(d["nq"], d["dim"])
    a = [_d(d[k].view(np.int32) if d[k].dtype == np.uint32 else d[k], dev)
         for k in ("kwords", "kboff", "klut", "vwords", "vboff", "vlut", "kscale", "vscale")] + [_d(qfull, dev)]
    out = torch.zeros((d["seq"], d["dim"]), device=dev)
    p = [x.data_ptr() for x in a]
    _ok(_lib().cf_kv_attn_fused_async(p[0], p[1], p[2], d["kmaxlen"], p[3], p[4], p[5], d["vmaxlen"], p[6], p[7],
                                      p[8], out.data_ptr(), d["seq"], d["dim"], d["nq"], d["window"], d["block"],
                                      d["zero"], d["softmax_scale"], None), "kv fused")
    got = out.cpu().numpy()[:d["nq"]]
    ref = d["golden"].reshape(d["nq"], d["dim"])
    assert np.abs(got - ref).max() / np.abs(ref).max() <= 1e-3


def test_cfdc_drives_delta_fetch(dev, tmp_path):
    import torch
    rng = np.random.default_rng(4)
    N, nbase = 9, 3000
    base = rng.integers(0, 32000, nbase).astype(np.int32)
    lengths, dstart, dlen, dpos, dval, originals, ostart = [], [], [], [], [], [], [0]
    for s in range(N):
        div = np.sort(rng.choice(nbase, size=int(rng.integers(0, 40)), replace=False))
        app = int(rng.integers(0, 50))  # appended suffix: every position carries a delta
        pos = np.concatenate([div, nbase + np.arange(app)]).astype(np.int32)
        val = rng.integers(0, 32000, pos.size).astype(np.int32)
        seq = np.concatenate([base, np.zeros(app, np.int32)])
        seq[pos] = val
        dstart.append(len(dpos))
        dlen.append(pos.size)
        dpos.extend(pos)
        dval.extend(val)
        lengths.append(nbase + app)
        originals.append(seq)
        ostart.append(ostart[-1] + seq.size)
    orig = np.concatenate(originals)
    d = _roundtrip(tmp_path, "cfdc", dict(N=N, nbase=nbase, ndelta=len(dpos), vocab=32000, total_tokens=orig.size,
                                          base=base, lengths=lengths, dstart=dstart, dlen=dlen, dpos=dpos, dval=dval,
                                          ostart=ostart, originals=orig))
    leaf = np.concatenate([np.full(d["lengths"][s], s, np.int32) for s in range(d["N"])])
    pos = np.concatenate([np.arange(d["lengths"][s], dtype=np.int32) for s in range(d["N"])])
    dp = d["dpos"] if d["dpos"].size else np.zeros(1, np.int32)
    dv = d["dval"] if d["dval"].size else np.zeros(1, np.int32)
    a = [_d(x, dev) for x in (d["base"], dp, dv, d["dstart"], d["dlen"], leaf, pos)]
    out = torch.empty(leaf.size, dtype=torch.int32, device=dev)
    _ok(_lib().cf_delta_fetch_async(a[0].data_ptr(), d["nbase"], *[x.data_ptr() for x in a[1:]], out.data_ptr(),
                                    leaf.size, None), "delta")
    assert np.array_equal(out.cpu().numpy(), d["originals"])


def test_cfsg_drives_fused_sparse_gather(dev, tmp_path):
    import torch
    from chromofold_amd.search import RrrWaveletIndex
    rng = np.random.default_rng(5)
    n, bits, dim, npos = 30000, 7, 24, 5000
    tok = rng.integers(0, 1 << bits, n).astype(np.uint32)
    w = O.rrrw_build(tok, bits)
    emb = rng.standard_normal((1 << bits, dim)).astype(np.float32)
    pos = rng.integers(0, n, npos).astype(np.uint32)
    fields = dict(n=n, bits=bits, vocab=1 << bits, emb_rows=1 << bits, dim=dim, cwords=w.cwords, nsb=w.nsb, na=w.na,
                  owords=w.offsets.size, npos=npos, rrr_bytes=w.rrr_bytes, embedding=emb, positions=pos,
                  golden=emb[tok[pos]])
    fields.update({k: getattr(w, k) for k in ("classes", "offsets", "rank_a", "rank_d", "off_a", "off_d", "offbase",
                                              "zeros")})
    d = _roundtrip(tmp_path, "cfsg", fields)
    idx = RrrWaveletIndex.from_host(dict(d, cwords=d["cwords"], nsb=d["nsb"], na=d["na"], bits=d["bits"]), dev)
    de = _d(d["embedding"], dev)
    dp = _d(d["positions"].view(np.int32), dev)
    out = torch.full((d["npos"], d["dim"]), float("nan"), device=dev)
    _ok(_lib().cf_sparse_gather_fused_async(idx.view(), de.data_ptr(), d["dim"], dp.data_ptr(), out.data_ptr(),
                                            d["npos"], None), "fused gather")
    assert np.array_equal(out.cpu().numpy(), d["golden"].reshape(d["npos"], d["dim"]))
