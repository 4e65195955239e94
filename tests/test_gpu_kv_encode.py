"""Device-side sealing (cf_kv_encode_groups_async) against the host encoder cf_kv_encode_groups: the same pool bytes,
offsets and end, bit for bit, over head dims 16..128 (RANS_HYBRID at multiples of 32), both codecs, ragged pages,
chain pairs and single groups, several table pairs, the INT8 fallback of a group holding -128 inside a RANS_HYBRID
pool (its pair partner then starts its own chain), all-zero / non-finite / denormal / huge / all-big pages, and a
non-zero pool_at. The host encoder is itself closed against the oracle here: the oracle decodes every device blob
(chains in order) back to exactly the symbols of the oracle's quantiser. Error cases leave the pool untouched and
report CF_ERR_INVALID_ARGUMENT in the device status word, where the host encoder returns the same status."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu
SENTINEL = 0xA5


@pytest.fixture(scope="module")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _groups(rng, pages_per_head, heads, ragged, paired=True):
    """Consecutive pages of each head cut into groups of 1..4 pages -> first_page, page_counts, heads, token counts,
    continues (the groups 2k + 1 of each head continue the chain of group 2k when `paired`)."""
    first, counts, hd, cont = [], [], [], []
    for h in range(heads):
        p, j = 0, 0
        while p < pages_per_head:
            c = int(min(rng.integers(1, 5), pages_per_head - p))
            first.append(h * pages_per_head + p)
            counts.append(c)
            hd.append(h)
            cont.append(1 if paired and j % 2 == 1 else 0)
            p += c
            j += 1
    tc = rng.integers(1, 17, size=heads * pages_per_head) if ragged else np.full(heads * pages_per_head, 16)
    return (np.array(first, np.uint64), np.array(counts, np.uint32), np.array(hd, np.uint32), tc.astype(np.uint32),
            np.array(cont, np.uint8))


def _tables(rng, heads, D):
    from chromofold_amd import kv
    parts = []
    for _ in range(heads):
        parts += [kv.build_table(rng.standard_normal((8, 16, D)).astype(np.float32)),
                  kv.build_table((rng.standard_normal((8, 16, D)) * rng.choice([0.1, 1, 5], size=D)).astype(np.float32))]
    return np.concatenate(parts)


def _device(dev, codec, K, V, D, tables, first, counts, heads, tc, pool_bytes, pool_at, capacity=None, cont=None):
    import torch
    from chromofold_amd import kv
    pool = torch.full((pool_bytes,), SENTINEL, dtype=torch.uint8, device=dev)
    if capacity is not None:
        pool = pool[:capacity]
    r = kv.encode_groups_device(
        codec, torch.from_numpy(K).to(dev), torch.from_numpy(V).to(dev), D,
        None if tables is None else torch.from_numpy(tables).to(dev),
        torch.from_numpy(first.astype(np.int64)).to(dev), torch.from_numpy(counts.view(np.int32)).to(dev), pool,
        pool_at, torch.from_numpy(heads.view(np.int32)).to(dev), torch.from_numpy(tc.view(np.int32)).to(dev),
        continues=None if cont is None else torch.from_numpy(cont).to(dev))
    torch.cuda.synchronize()
    return (int(r.status.item()), pool.cpu().numpy(), r.offsets.cpu().numpy().view(np.uint32),
            int(r.pool_end.item()))


def _special(K, V, rng, kind):
    if kind == "zero":
        K[0] = 0.0
        V[1] = 0.0
    elif kind == "nonfinite":
        K[0, 3, 5] = np.nan
        K[1, 0, 0] = np.inf
        V[0, 2, 7] = -np.inf
        V[2, 1, 1] = np.nan
    elif kind == "denormal":
        K[0] = rng.standard_normal(K[0].shape).astype(np.float32) * np.float32(1e-41)
        V[1] = rng.standard_normal(V[1].shape).astype(np.float32) * np.float32(3e-44)
    elif kind == "huge":
        K[0] *= np.float32(1e38)
        V[0, 0, 0] = np.float32(3.4e38)
    elif kind == "extremes":  # every value at +-absmax: every big bit set, the tables' rarest joint symbol, so
        # every lane renormalises at (nearly) every step: the word bound of kv_codec_ext.h is reached, still coded
        K[:] = rng.choice([-1.0, 1.0], K.shape).astype(np.float32)
        V[:] = rng.choice([-1.0, 1.0], V.shape).astype(np.float32)


CASES = [  # (D, codec, heads, pages per head, ragged, special, paired)
    (128, 2, 3, 9, True, None, True), (128, 2, 3, 9, True, None, False), (128, 1, 2, 6, True, None, True),
    (64, 2, 2, 7, False, None, True), (16, 1, 1, 5, True, None, True), (32, 2, 2, 4, True, None, True),
    (48, 1, 1, 6, True, None, True), (96, 2, 2, 5, True, None, True), (112, 1, 1, 3, True, None, True),
    (128, 2, 1, 4, False, "zero", True), (128, 2, 2, 4, True, "nonfinite", True), (64, 2, 2, 4, False, "denormal", True),
    (128, 2, 1, 4, True, "huge", True), (128, 2, 1, 8, False, "extremes", True), (64, 1, 1, 4, True, "nonfinite", True),
]


@pytest.mark.parametrize("D,codec,heads,pph,ragged,special,paired", CASES)
def test_device_encoder_matches_host(dev, D, codec, heads, pph, ragged, special, paired):
    from chromofold_amd import kv
    rng = np.random.default_rng(1000 * D + 10 * codec + heads + pph)
    K = rng.standard_normal((heads * pph, 16, D)).astype(np.float32)
    V = rng.standard_normal((heads * pph, 16, D)).astype(np.float32)
    _special(K, V, rng, special)
    first, counts, hd, tc, cont = _groups(rng, pph, heads, ragged, paired)
    tables = _tables(rng, heads, D) if codec == 2 else None
    host, hoff = kv.encode_groups(codec, K, V, D, tables, first, counts, hd, tc, continues=cont)
    pool_at = 48
    cap = pool_at + len(first) * int(kv.A.lib().cf_kv_group_blob_max_bytes(codec, D)) + 64
    st, pool, off, end = _device(dev, codec, K, V, D, tables, first, counts, hd, tc, cap, pool_at, cont=cont)
    assert st == 0
    assert end == pool_at + host.size
    assert np.array_equal(pool[pool_at:end], host)
    assert np.array_equal(off, hoff + pool_at // 16)
    assert (pool[:pool_at] == SENTINEL).all() and (pool[end:] == SENTINEL).all()
    codecs = [int(host[int(o) * 16]) for o in hoff]
    if special == "extremes":
        assert all(c == kv.CODEC_RANS_HYBRID for c in codecs)
    if special == "nonfinite" and codec == 2:  # the groups holding -128 are INT8, the others coded
        assert kv.CODEC_INT8 in codecs and kv.CODEC_RANS_HYBRID in codecs
    # close the loop without the host encoder: the oracle decodes the device blobs (each head's chains in order) to
    # the oracle quantiser's symbols
    decoded = {}
    for h in range(heads):
        idx = [i for i in range(len(first)) if hd[i] == h]
        for i, dec in zip(idx, O.kv_decode_run([pool[int(off[i]) * 16:][:65536] for i in idx], tables, h, D)):
            decoded[i] = dec
    for i in range(len(first)):
        ks, vs, ksc, vsc, gtc = decoded[i]
        for G in range(int(counts[i])):
            p = int(first[i]) + G
            n = int(tc[p])
            assert gtc[G] == n
            if special in ("nonfinite", "denormal", "huge"):
                continue  # the oracle quantiser is only pinned for finite normal data; bytes equal the host above
            for sym, sc, x in ((ks, ksc, K), (vs, vsc, V)):
                want, wsc = O.kv_quantize_absmax(x[p, :n])
                assert np.array_equal(sym[G, :n], want) and np.float32(sc[G]) == np.float32(wsc)


def test_device_encoder_errors_leave_pool_untouched(dev):
    from chromofold_amd import kv
    rng = np.random.default_rng(77)
    D, heads, pph = 64, 2, 4
    K = rng.standard_normal((heads * pph, 16, D)).astype(np.float32)
    V = rng.standard_normal((heads * pph, 16, D)).astype(np.float32)
    first, counts, hd, tc, _ = _groups(rng, pph, heads, True, paired=False)
    tables = _tables(rng, heads, D)
    host, _ = kv.encode_groups(2, K, V, D, tables, first, counts, hd, tc)
    cap = 32 + len(first) * int(kv.A.lib().cf_kv_group_blob_max_bytes(2, D))
    # pool one 16-byte unit too small
    st, pool, _, end = _device(dev, 2, K, V, D, tables, first, counts, hd, tc, cap, 32, capacity=32 + host.size - 16)
    assert st == 1 and end == 0 and (pool == SENTINEL).all()
    st, pool, _, end = _device(dev, 2, K, V, D, tables, first, counts, hd, tc, cap, 32, capacity=32 + host.size)
    assert st == 0 and end == 32 + host.size
    # a present page with 0 tokens: the host rejects it too
    bad_tc = tc.copy()
    bad_tc[int(first[1])] = 0
    with pytest.raises(kv.A.CfError):
        kv.encode_groups(2, K, V, D, tables, first, counts, hd, bad_tc)
    st, pool, _, end = _device(dev, 2, K, V, D, tables, first, counts, hd, bad_tc, cap, 32)
    assert st == 1 and end == 0 and (pool == SENTINEL).all()
    # a table pair past the end of `tables`
    bad_hd = hd.copy()
    bad_hd[-1] = heads
    st, pool, _, end = _device(dev, 2, K, V, D, tables, first, counts, bad_hd, tc, cap, 32)
    assert st == 1 and (pool == SENTINEL).all()
    # an unusable table (every slot zero: symbols without a frequency): the host loader rejects it too
    bad_tab = tables.copy()
    bad_tab[:kv.TABLE_BYTES] = 0
    with pytest.raises(kv.A.CfError):
        kv.encode_groups(2, K, V, D, bad_tab, first, counts, hd, tc)
    st, pool, _, end = _device(dev, 2, K, V, D, bad_tab, first, counts, hd, tc, cap, 32)
    assert st == 1 and (pool == SENTINEL).all()
    # a good call on the same buffers afterwards starts from a clean status
    st, pool, _, end = _device(dev, 2, K, V, D, tables, first, counts, hd, tc, cap, 32)
    assert st == 0 and np.array_equal(pool[32:end], host)


def test_device_sealed_pool_serves_batched_attention(dev):
    """A pool sealed on the device decodes through the batched entry point to exactly the output of the host-sealed
    pool (same bytes, same offsets)."""
    import torch
    from chromofold_amd import kv
    from kv_helpers import make_seqs
    D, H, gqa = 128, 2, 4
    toks = [300, 64, 1000, 17, 200]
    data = make_seqs(toks, H, D, 4242)
    rng = np.random.default_rng(5)
    tables = _tables(rng, H, D)
    a = kv.build_batched(2, lambda s: data[s], len(toks), H, np.array(toks), D, tables, dev, keep_host=True)
    b = kv.build_batched(2, lambda s: data[s], len(toks), H, np.array(toks), D, tables, dev, keep_host=True,
                         encoder="device")
    assert np.array_equal(a.host_offsets, b.host_offsets)
    assert np.array_equal(a.host_pool, b.host_pool)
    q = torch.from_numpy(rng.standard_normal((len(toks), H * gqa, D)).astype(np.float32)).to(dev)
    qp = torch.tensor([t - 1 for t in toks], dtype=torch.int32, device=dev)
    oa, ob = torch.empty_like(q), torch.empty_like(q)
    a.attention(q, oa, qp, 0.088)
    b.attention(q, ob, qp, 0.088)
    torch.cuda.synchronize()
    assert torch.equal(oa, ob)
