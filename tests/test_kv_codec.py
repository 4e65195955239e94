"""CPU tests of the KV page codecs (kv_codec_ext.h): the library's host encoder against the oracle's independent
decoder written from the format text. Decode must be bit-exact: every symbol equals the absmax quantiser's symbol
(the quantiser itself is checked against a numpy closed form), scales equal, every rANS stream ends exactly at
its word count, and every chain (one group, or a pair of groups) ends with all 64 states back at 2^16."""
import numpy as np
import pytest

import oracle as O


@pytest.fixture(scope="module")
def kv():
    from chromofold_amd import kv
    return kv


def _absmax_closed_form(x):
    m = np.abs(x).max()
    s = np.float32(1.0) if m == 0 else np.float32(m) / np.float32(127.0)
    return (np.clip(np.rint(x / s), -128, 127) + 128).astype(np.uint8), s


def test_absmax_quantiser_closed_form():
    rng = np.random.default_rng(0)
    for x in [rng.standard_normal((16, 128)).astype(np.float32), np.zeros((16, 64), np.float32),
              np.full((3, 128), -2.5, np.float32), (rng.standard_normal((16, 128)) * 1e-30).astype(np.float32)]:
        sym, sc = O.kv_quantize_absmax(x)
        sym2, sc2 = _absmax_closed_form(x)
        assert sc == sc2 and np.array_equal(sym, sym2)
    # round half to even on exact halves: scale 1 (max 127) and values k + 0.5
    x = np.array([127.0, 0.5, 1.5, 2.5, -0.5, -1.5], np.float32)
    sym, sc = O.kv_quantize_absmax(x)
    assert sc == 1.0 and list(sym.astype(int) - 128) == [127, 0, 2, 2, 0, -2]


def _check_group(got, K, V, first, count, tc):
    ks, vs, ksc, vsc, t = got
    for G in range(4):
        if G >= count:
            assert t[G] == 0 and (ks[G] == 128).all() and (vs[G] == 128).all()
            continue
        p = int(first) + G
        n_t = int(tc[p])
        assert t[G] == n_t
        ek, eks = O.kv_quantize_absmax(K[p, :n_t])
        ev, evs = O.kv_quantize_absmax(V[p, :n_t])
        assert ksc[G] == eks and vsc[G] == evs
        assert np.array_equal(ks[G, :n_t], ek) and np.array_equal(vs[G, :n_t], ev), G
        assert (ks[G, n_t:] == 128).all() and (vs[G, n_t:] == 128).all()


def _sample_pages(rng, n, D):
    K = rng.standard_normal((n, 16, D)).astype(np.float32)
    V = rng.standard_normal((n, 16, D)).astype(np.float32)
    K[3] = 0.0                                   # all-zero page (scale 1, every symbol 128)
    V[4] *= 1e4                                  # large magnitudes
    K[5, :, 7] = 50.0                            # one outlier channel
    V[6] = np.sign(V[6])                         # two-valued page
    K[7] = np.linspace(-1, 1, 16 * D, dtype=np.float32).reshape(16, D)
    V[10, :, :] = 127.0                          # every value big
    K[11] = np.where(rng.random((16, D)) < 0.5, 1.0, -1.0).astype(np.float32)  # signs only
    tc = np.full(n, 16, np.uint32)
    tc[8], tc[9], tc[39] = 1, 11, 5              # partial pages (padded with symbol 128)
    return K, V, tc


@pytest.mark.parametrize("codec", [1, 2])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("paired", [False, True])
def test_group_roundtrip(kv, codec, D, paired):
    """Every group decodes (oracle decoder written from the format text) to the absmax quantiser's symbols, with
    groups coded alone or as chain pairs (the second group of a pair starts from the states the first ends with;
    every chain ends at 2^16 with every stream exactly consumed)."""
    rng = np.random.default_rng(D + codec)
    n = 40                                       # pages
    K, V, tc = _sample_pages(rng, n, D)
    # groups of 4, 3, 2 and 1 pages (absent pages padded), assorted table pairs; with `paired` groups (0,1), (2,3),
    # ... of the same head form chains
    first = np.array([0, 4, 8, 12, 15, 17, 18, 22, 26, 30, 34, 38], np.uint64)
    counts = np.array([4, 4, 4, 3, 2, 1, 4, 4, 4, 4, 4, 2], np.uint32)
    heads = (np.arange(first.size) // 2 % 3).astype(np.uint32)
    cont = (np.arange(first.size) % 2 == 1).astype(np.uint8) if paired else None
    tables = None
    if codec == 2:
        tables = np.concatenate([kv.build_table(K[h::3][:5]) if s == 0 else kv.build_table(V[h::3][:5])
                                 for h in range(3) for s in range(2)])
    blob, offs = kv.encode_groups(codec, K, V, D, tables, first, counts, heads, tc, continues=cont)
    assert blob.size % 16 == 0 and (offs[1:] > offs[:-1]).all()
    runs = [[g, g + 1] for g in range(0, first.size, 2)] if paired else [[g] for g in range(first.size)]
    for run in runs:
        got = O.kv_decode_run([blob[int(offs[g]) * 16:] for g in run], tables, int(heads[run[0]]), D)
        for g, dec in zip(run, got):
            _check_group(dec, K, V, first[g], counts[g], tc)
            if codec == 2:
                assert O.kv_group_continues(blob[int(offs[g]) * 16:]) == (paired and g % 2 == 1)


def test_pairs_are_smaller_and_decode_alike(kv):
    """A chain pair stores one set of lane states for two groups: its blobs are smaller than the two groups coded
    alone by the 512 bytes of the second group's states, less what the first group's stream grows by carrying the
    second group's end states instead of starting from 2^16 (at most one 16-bit word per lane and stream, 256 bytes),
    and decode to the same symbols."""
    rng = np.random.default_rng(5)
    D = 128
    K = rng.standard_normal((8, 16, D)).astype(np.float32)
    V = rng.standard_normal((8, 16, D)).astype(np.float32)
    tables = np.concatenate([kv.build_table(K[:4]), kv.build_table(V[:4])])
    first, counts = np.array([0, 4], np.uint64), np.array([4, 4], np.uint32)
    solo, so = kv.encode_groups(2, K, V, D, tables, first, counts)
    pair, po = kv.encode_groups(2, K, V, D, tables, first, counts, continues=np.array([0, 1], np.uint8))
    assert 512 - 256 - 32 <= solo.size - pair.size <= 512 + 32
    a = O.kv_decode_run([solo[int(o) * 16:] for o in so], tables, 0, D)
    b = O.kv_decode_run([pair[int(o) * 16:] for o in po], tables, 0, D)
    for x, y in zip(a, b):
        for u, v in zip(x, y):
            assert np.array_equal(u, v)
    with pytest.raises(ValueError):  # a continuing group cannot be decoded without its chain's states
        O.kv_decode_group(pair[int(po[1]) * 16:], tables, 0, D)


def test_nan_group_falls_back_to_int8_and_breaks_its_pair(kv):
    """A NaN input quantises to -128 (x86 lrint), which sign-magnitude cannot hold: that group is stored INT8 and
    the other group of its pair starts a chain of its own; both decode to the quantiser's symbols."""
    rng = np.random.default_rng(9)
    D = 64
    K = rng.standard_normal((16, 16, D)).astype(np.float32)
    V = rng.standard_normal((16, 16, D)).astype(np.float32)
    tables = np.concatenate([kv.build_table(K[:4]), kv.build_table(V[:4])])
    tc = np.full(16, 16, np.uint32)
    for bad in (0, 1):  # NaN in the first, then in the second group of a pair
        Kb = K.copy()
        Kb[4 * bad + 2, 3, 5] = np.nan
        first, counts = np.array([0, 4, 8, 12], np.uint64), np.full(4, 4, np.uint32)
        blob, offs = kv.encode_groups(2, Kb, V, D, tables, first, counts, token_counts=tc,
                                      continues=np.array([0, 1, 0, 1], np.uint8))
        codecs = [int(blob[int(o) * 16:][:4].view(np.uint32)[0]) for o in offs]
        assert codecs == [1 if g == bad else 2 for g in range(4)]
        assert not O.kv_group_continues(blob[int(offs[1]) * 16:]) and O.kv_group_continues(blob[int(offs[3]) * 16:])
        dec = O.kv_decode_run([blob[int(o) * 16:] for o in offs], tables, 0, D)
        for g in range(4):
            _check_group(dec[g], Kb, V, first[g], 4, tc)


def test_raw_word_layout_closed_form(kv):
    """The raw words of a chain-start group follow the frame layout of kv_codec_ext.h: for quad k of a sign group
    (frame r = (0, 4, 2, 6, 1, 5, 3, 7)[k]) and value i, bit (8 i + r + f) mod 32 of its nibble / crumb / sign
    word is bit f of |q| / bit f of |q| >> 4 / the sign. Checked on one lane of the K stream, one quad at a time,
    with a page whose values are all distinct patterns."""
    D = 64
    K = np.zeros((4, 16, D), np.float32)
    rng = np.random.default_rng(2)
    vals = rng.integers(-127, 128, (16, D))
    vals[0, 0] = 127  # scale exactly 1: q = value
    K[0] = vals.astype(np.float32)
    V = np.zeros_like(K)
    tables = np.concatenate([kv.build_table(K[:1]), kv.build_table(V[:1] + 1)])
    blob, _ = kv.encode_groups(2, K, V, D, tables, np.array([0], np.uint64), np.array([1], np.uint32))
    raw = blob[64 + 512:].view(np.uint32)
    frame, nword = (0, 4, 2, 6, 1, 5, 3, 7), (0, 0, 1, 1, 3, 3, 4, 4)
    for L in (0, 5, 15):  # token L of page 0
        for q in range(D // 4):
            sg, k = divmod(q, 8)
            r = frame[k]
            N = int(raw[(7 * sg + nword[k]) * 64 + L])
            Cw = int(raw[(7 * sg + (2 if k < 4 else 5)) * 64 + L])
            S = int(raw[(7 * sg + 6) * 64 + L])
            for i in range(4):
                v = int(vals[L, 4 * q + i])
                a = abs(v)
                for f in range(4):
                    assert (N >> ((8 * i + r + f) % 32)) & 1 == (a >> f) & 1
                for f in range(2):
                    assert (Cw >> ((8 * i + r + 4 + f) % 32)) & 1 == (a >> (4 + f)) & 1
                assert (S >> ((8 * i + r + 7) % 32)) & 1 == (1 if v < 0 else 0)


def test_rans_compression_near_entropy(kv):
    """On N(0,1) pages with chain pairs the RANS_HYBRID pool is within 0.2 b/value of the int8 symbol entropy plus
    the fixed overhead (a 64-byte header per group, 2 x 64 lane states per pair), and below 7.55 b/value (7.52 here:
    signs and 6 low bits raw, 8 big bits per rANS step; the INT8 codec stores 8.03)."""
    rng = np.random.default_rng(11)
    n, D = 256, 128
    K = rng.standard_normal((n, 16, D)).astype(np.float32)
    V = rng.standard_normal((n, 16, D)).astype(np.float32)
    tables = np.concatenate([kv.build_table(K[:64]), kv.build_table(V[:64])])
    first = np.arange(0, n, 4, dtype=np.uint64)
    cont = (np.arange(first.size) % 2).astype(np.uint8)
    blob, _ = kv.encode_groups(2, K, V, D, tables, first, np.full(first.size, 4, np.uint32), continues=cont)
    syms = np.concatenate([O.kv_quantize_absmax(K[p])[0].ravel() for p in range(n)] +
                          [O.kv_quantize_absmax(V[p])[0].ravel() for p in range(n)])
    c = np.bincount(syms, minlength=256).astype(np.float64)
    pr = c[c > 0] / c.sum()
    h0 = -(pr * np.log2(pr)).sum()
    bits_per_value = blob.size * 8 / (2 * n * 16 * D)
    overhead = (2 * 64 + 512) * 8 / (2 * 8 * 16 * D)
    assert bits_per_value < h0 + overhead + 0.2, (bits_per_value, h0, overhead)
    assert bits_per_value < 7.55, bits_per_value


def test_table_every_symbol_codable(kv):
    hist = np.zeros((1, 16, 64), np.float32)  # all-zero sample -> joint symbol 0 only
    t = kv.build_table(hist)
    lo = t.view(np.uint32)[0::2]
    hi = t.view(np.uint32)[1::2]
    f = lo & 2047
    cs = (lo >> 11) & 2047
    j = (lo >> 22) & 255
    starts = cs == 0
    assert starts.sum() == 256 and sorted(j[starts]) == list(range(256))
    assert f[starts].sum() == 2048
    # the spread word of every slot: big bit i of quad A at 8i + 6, of quad B at (8i + 10) mod 32
    exp = np.zeros_like(hi)
    for i in range(4):
        exp |= ((j >> i) & 1) << (8 * i + 6)
        exp |= ((j >> (4 + i)) & 1) << ((8 * i + 10) % 32)
    assert np.array_equal(hi, exp)
    # a page whose big bits never occurred in the sample still codes and decodes
    rng = np.random.default_rng(3)
    K = (rng.standard_normal((2, 16, 64)) * 3).astype(np.float32)
    tt = np.concatenate([t, t])
    blob, offs = kv.encode_groups(2, K, K, 64, tt, np.array([0], np.uint64), np.array([2], np.uint32))
    ks, vs, *_ = O.kv_decode_group(blob, tt, 0, 64)
    assert np.array_equal(ks[0], O.kv_quantize_absmax(K[0])[0])
    assert np.array_equal(ks[1], O.kv_quantize_absmax(K[1])[0])


def test_device_encoder_rejects_bad_arguments_before_any_device_call(kv):
    """cf_kv_encode_groups_async checks its arguments on the host (no device is touched, so this runs without a
    GPU): NULLs, misaligned K/V or pool pointers, a misaligned pool_at, a bad head_dim or codec, a RANS call without
    tables, and a workspace smaller than cf_kv_encode_groups_workspace_bytes."""
    L = kv.A.lib()
    f = L.cf_kv_encode_groups_async
    ws = int(L.cf_kv_encode_groups_workspace_bytes(2, 128, 4, 2))
    assert ws > 4 * int(L.cf_kv_group_blob_max_bytes(2, 128))
    assert L.cf_kv_encode_groups_workspace_bytes(2, 20, 4, 2) == 0
    assert L.cf_kv_encode_groups_workspace_bytes(3, 128, 4, 2) == 0
    A = 1 << 20  # a fake, aligned address: never dereferenced because every call below fails validation

    def call(codec=2, keys=A, values=A, n=4, D=128, tables=A, tcount=2, pool=A, pool_at=0, ws_bytes=ws):
        return f(codec, keys, values, n, A, A, None, D, tables, tcount, None, None, pool, 1 << 30, pool_at, A, A, A,
                 A, ws_bytes, None)

    assert call(keys=None) == 1 and call(values=A + 8) == 1 and call(pool=A + 4) == 1 and call(pool_at=8) == 1
    assert call(n=0) == 1 and call(tables=None) == 1 and call(tcount=1) == 1 and call(ws_bytes=ws - 1) == 1
    assert call(D=20) == 2 and call(D=256) == 2 and call(codec=7) == 2


def test_batched_desc_validation(kv):
    """cf_kv_validate_batched_desc is host-only (fake, never dereferenced addresses): a well-formed descriptor is
    accepted; NULL pointers, a RANS_HYBRID descriptor without tables, pool or table pointers off 16-byte alignment,
    and heads or head_dims the kernels do not take are refused."""
    import ctypes as C
    L = kv.A.lib()
    A = 1 << 20

    def desc(**kw):
        d = kv.cf_kv_batched_desc()
        d.struct_size, d.abi_version, d.codec = C.sizeof(kv.cf_kv_batched_desc), kv.EXT_ABI_VERSION, 2
        d.seq_count, d.kv_head_count, d.query_head_count, d.head_dim, d.max_groups = 2, 8, 32, 128, 4
        d.pool = d.group_offsets = d.seq_tokens = d.query_pos = d.tables = d.queries = d.output = A
        d.softmax_scale = 0.125
        for k, v in kw.items():
            setattr(d, k, v)
        return L.cf_kv_validate_batched_desc(C.byref(d))

    assert desc() == 0 and desc(codec=1, tables=None) == 0
    assert desc(pool=None) == 1 and desc(tables=None) == 1 and desc(queries=None) == 1
    assert desc(pool=A + 8) == 1 and desc(tables=A + 4) == 1 and desc(tables=A + 8) == 1
    assert desc(query_head_count=40) == 2 and desc(head_dim=96) == 2 and desc(codec=3) == 2


def test_mixed_pool_raw_prefix(kv):
    """build_batched(raw_groups=...) on the host: a sequence's leading groups are INT8 blobs inside a RANS_HYBRID
    pool. Every group decodes (oracle decoder) to the same symbols and scales as in an all-INT8 and an all-rANS pool,
    the leading groups carry the INT8 codec byte and the rest the RANS_HYBRID one, and sharing the raw prefix with
    other sequences reuses the donor's blobs."""
    rng = np.random.default_rng(77)
    H, D, T = 2, 128, [300, 300, 200]
    data = [(rng.standard_normal((H, t, D)).astype(np.float32), rng.standard_normal((H, t, D)).astype(np.float32))
            for t in T]
    for s in (1, 2):  # the first 128 tokens (2 groups) of sequences 1 and 2 are sequence 0's
        data[s][0][:, :128] = data[0][0][:, :128]
        data[s][1][:, :128] = data[0][1][:, :128]
    tables = np.concatenate([kv.build_table(data[0][i][h][:256].reshape(-1, 16, D)) for h in range(H) for i in (0, 1)])
    shared = {1: (0, 2), 2: (0, 2)}
    args = (lambda s: data[s], 3, H, np.array(T), D)
    mixed = kv.build_batched(kv.CODEC_RANS_HYBRID, *args, tables, "cpu", keep_host=True, shared=shared,
                             raw_groups={0: 2, 1: 3})
    rans = kv.build_batched(kv.CODEC_RANS_HYBRID, *args, tables, "cpu", keep_host=True, shared=shared)
    raw = kv.build_batched(kv.CODEC_INT8, *args, None, "cpu", keep_host=True, shared=shared)
    assert mixed.pool_bytes < rans.pool_bytes + 2 * raw.pool_bytes  # sanity: nothing duplicated wholesale
    for s in range(3):
        for h in range(H):
            ng = (T[s] + 63) // 64
            runs = {}
            for name, pool in (("mixed", mixed), ("ref_raw", raw), ("ref_rans", rans)):
                blobs = [pool.host_pool[int(pool.host_offsets[s, h, g]) * 16:][:65536] for g in range(ng)]
                runs[name] = (O.kv_decode_run(blobs, tables, h, D), blobs)
            for g in range(ng):
                is_raw = g < (2 if s != 1 else 3)
                exp = runs["ref_raw" if is_raw else "ref_rans"][0][g]
                for a, b in zip(runs["mixed"][0][g], exp):
                    assert np.array_equal(a, b), (s, h, g)
                codec = int(runs["mixed"][1][g][:4].view(np.uint32)[0])  # cf_kv_group_header.codec
                assert codec == (kv.CODEC_INT8 if is_raw else kv.CODEC_RANS_HYBRID), (s, h, g)
            if s:
                assert np.array_equal(mixed.host_offsets[s, h, :2], mixed.host_offsets[0, h, :2])
    with pytest.raises(ValueError):
        kv.build_batched(kv.CODEC_RANS_HYBRID, *args, tables, "cpu", encoder="device", raw_groups={0: 1})


def test_pool_attention_matches_paged_oracle(kv):
    """O.kv_pool_attention (the all-core CPU baseline: decode every group of a batched pool, chains in order, and
    attend in float64) equals the paged fp64 oracle (O.paged_attention_f64, pinned against the reference's
    kv_reference.cpp) over the same decoded pages, for ragged lengths, a causal query position, GQA 4, chain pairs
    and a raw INT8 group inside the pool; and agrees with itself on 1 and on all threads."""
    from kv_helpers import make_seqs, oracle_batched
    D, H, gqa = 64, 2, 4
    toks = [300, 129, 64, 700]
    data = make_seqs(toks, H, D, 123)
    tables = np.concatenate([kv.build_table(data[0][i][h][:256].reshape(-1, 16, D)) for h in range(H) for i in (0, 1)])
    kvb = kv.build_batched(2, lambda s: data[s], len(toks), H, np.array(toks), D, tables, "cpu", keep_host=True,
                           raw_groups={1: 1})
    rng = np.random.default_rng(124)
    q = rng.standard_normal((len(toks), H * gqa, D)).astype(np.float32)
    qp = np.array([299, 100, 63, 699], np.uint32)
    sc = 1.0 / np.sqrt(D)
    ref = oracle_batched(kvb, data, q, qp, sc, gqa)
    got = O.kv_pool_attention(kvb.host_pool, kvb.host_offsets, np.array(toks, np.uint32), qp, tables, q, H, D, sc)
    assert np.abs(got - ref).max() <= 1e-6 * np.abs(ref).max()
    one = O.kv_pool_attention(kvb.host_pool, kvb.host_offsets, np.array(toks, np.uint32), qp, tables, q, H, D, sc,
                              nseq=2, threads=1)
    assert np.array_equal(one, got[:2])


def test_planted_mistakes_change_the_decode(kv):
    """The oracle decoder reads every part of a format-4 blob: one flipped bit in a raw word changes exactly that
    value's symbol; a flipped bit in the rANS word stream, or decoding with another head's table, either changes
    the symbols or leaves the chain's end states off 2^16 (kv_decode_run raises)."""
    rng = np.random.default_rng(77)
    D = 128
    K = rng.standard_normal((4, 16, D)).astype(np.float32)
    V = rng.standard_normal((4, 16, D)).astype(np.float32)
    tc = np.full(4, 16, np.uint32)
    tab = np.concatenate([kv.build_table(K), kv.build_table(V)])
    other = np.concatenate([kv.build_table(V * 0.02), kv.build_table(K * 0.02)])  # a different distribution
    first, counts, heads = np.array([0], np.uint64), np.array([4], np.uint32), np.array([0], np.uint32)
    blob, _ = kv.encode_groups(2, K, V, D, tab, first, counts, heads, tc)
    good = O.kv_decode_run([blob], tab, 0, D)[0]
    _check_group(good, K, V, 0, 4, tc)
    raw0 = 64 + 512  # header + the chain start's lane states
    RAW = 7 * (D // 32) * 64

    def decoded_or_failed(b, t):
        try:
            return O.kv_decode_run([b], t, 0, D)[0]
        except ValueError:
            return None

    # a raw K nibble word (word 0 of sign group 1, lane 5): one bit -> one value
    bad = blob.copy()
    bad[raw0 + ((7 * 1 + 0) * 64 + 5) * 4] ^= 0x01
    got = decoded_or_failed(bad, tab)
    assert got is not None
    diff = (got[0] != good[0]).sum() + (got[1] != good[1]).sum()
    assert diff == 1
    # a raw V sign word: one value's sign
    bad = blob.copy()
    bad[raw0 + RAW * 4 + ((7 * 2 + 6) * 64 + 9) * 4 + 3] ^= 0x10
    got = decoded_or_failed(bad, tab)
    assert got is not None and (got[1] != good[1]).sum() == 1 and (got[0] == good[0]).all()
    # the K word stream (first rANS word after the raw words)
    bad = blob.copy()
    bad[raw0 + 2 * RAW * 4 + 1] ^= 0x40
    got = decoded_or_failed(bad, tab)
    assert got is None or not (np.array_equal(got[0], good[0]) and np.array_equal(got[1], good[1]))
    # another table
    got = decoded_or_failed(blob, other)
    assert got is None or not (np.array_equal(got[0], good[0]) and np.array_equal(got[1], good[1]))
