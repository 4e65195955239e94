"""Device-side sealing (cf_kv_encode_groups_async) against the host encoder cf_kv_encode_groups: the same pool bytes,
offsets and end, bit for bit, over head dims 16..128, both codecs, ragged pages, several table pairs, the INT8
fallback inside a RANS_HYBRID pool, all-zero / non-finite / denormal / huge pages, and a non-zero pool_at. The host
encoder is itself closed against the oracle here: the oracle decodes every device blob back to exactly the symbols
of the oracle's quantiser. Error cases leave the pool untouched and report CF_ERR_INVALID_ARGUMENT in the device
status word, where the host encoder returns the same status."""
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


def _groups(rng, pages_per_head, heads, ragged):
    """Consecutive pages of each head cut into groups of 1..4 pages -> first_page, page_counts, heads, token counts."""
    first, counts, hd = [], [], []
    for h in range(heads):
        p = 0
        while p < pages_per_head:
            c = int(min(rng.integers(1, 5), pages_per_head - p))
            first.append(h * pages_per_head + p)
            counts.append(c)
            hd.append(h)
            p += c
    tc = rng.integers(1, 17, size=heads * pages_per_head) if ragged else np.full(heads * pages_per_head, 16)
    return (np.array(first, np.uint64), np.array(counts, np.uint32), np.array(hd, np.uint32), tc.astype(np.uint32))


def _tables(rng, heads, D):
    from chromofold_amd import kv
    parts = []
    for _ in range(heads):
        parts += [kv.build_table(rng.standard_normal((8, 16, D)).astype(np.float32)),
                  kv.build_table((rng.standard_normal((8, 16, D)) * rng.choice([0.1, 1, 5], size=D)).astype(np.float32))]
    return np.concatenate(parts)


def _device(dev, codec, K, V, D, tables, first, counts, heads, tc, pool_bytes, pool_at, capacity=None):
    import torch
    from chromofold_amd import kv
    pool = torch.full((pool_bytes,), SENTINEL, dtype=torch.uint8, device=dev)
    if capacity is not None:
        pool = pool[:capacity]
    r = kv.encode_groups_device(
        codec, torch.from_numpy(K).to(dev), torch.from_numpy(V).to(dev), D,
        None if tables is None else torch.from_numpy(tables).to(dev),
        torch.from_numpy(first.astype(np.int64)).to(dev), torch.from_numpy(counts.view(np.int32)).to(dev), pool,
        pool_at, torch.from_numpy(heads.view(np.int32)).to(dev), torch.from_numpy(tc.view(np.int32)).to(dev))
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
    elif kind == "extremes":  # every value at +-absmax: high parts 0/3 only, the tables' rarest joint symbols, so
        # both streams cost ~11 bits per quad and the group falls back to INT8
        K[:] = rng.choice([-1.0, 1.0], K.shape).astype(np.float32)
        V[:] = rng.choice([-1.0, 1.0], V.shape).astype(np.float32)


CASES = [  # (D, codec, heads, pages per head, ragged, special)
    (128, 2, 3, 9, True, None), (128, 1, 2, 6, True, None), (64, 2, 2, 7, False, None), (16, 2, 1, 5, True, None),
    (32, 2, 2, 4, True, None), (48, 2, 1, 6, True, None), (96, 2, 2, 5, True, None), (112, 1, 1, 3, True, None),
    (128, 2, 1, 4, False, "zero"), (128, 2, 2, 4, True, "nonfinite"), (64, 2, 2, 4, False, "denormal"),
    (128, 2, 1, 4, True, "huge"), (128, 2, 1, 8, False, "extremes"), (64, 1, 1, 4, True, "nonfinite"),
]


@pytest.mark.parametrize("D,codec,heads,pph,ragged,special", CASES)
def test_device_encoder_matches_host(dev, D, codec, heads, pph, ragged, special):
    from chromofold_amd import kv
    rng = np.random.default_rng(1000 * D + 10 * codec + heads + pph)
    K = rng.standard_normal((heads * pph, 16, D)).astype(np.float32)
    V = rng.standard_normal((heads * pph, 16, D)).astype(np.float32)
    _special(K, V, rng, special)
    first, counts, hd, tc = _groups(rng, pph, heads, ragged)
    tables = _tables(rng, heads, D) if codec == 2 else None
    host, hoff = kv.encode_groups(codec, K, V, D, tables, first, counts, hd, tc)
    pool_at = 48
    cap = pool_at + len(first) * int(kv.A.lib().cf_kv_group_blob_max_bytes(codec, D)) + 64
    st, pool, off, end = _device(dev, codec, K, V, D, tables, first, counts, hd, tc, cap, pool_at)
    assert st == 0
    assert end == pool_at + host.size
    assert np.array_equal(pool[pool_at:end], host)
    assert np.array_equal(off, hoff + pool_at // 16)
    assert (pool[:pool_at] == SENTINEL).all() and (pool[end:] == SENTINEL).all()
    if special == "extremes":
        codecs = [int(host[int(o) * 16]) for o in hoff]  # full groups exceed the word budget, short ones may not
        assert all(c == kv.CODEC_INT8 for c, n in zip(codecs, counts) if n >= 3) and kv.CODEC_INT8 in codecs
    # close the loop without the host encoder: the oracle decodes the device blobs to the oracle quantiser's symbols
    for i, o in enumerate(off):
        blob = pool[int(o) * 16:]
        ks, vs, ksc, vsc, gtc = O.kv_decode_group(blob[:65536], tables, int(hd[i]), D)
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
    first, counts, hd, tc = _groups(rng, pph, heads, True)
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
    toks = [300, 64, 1000, 17]
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
