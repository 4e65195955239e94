"""CPU tests of the KV page codecs (kv_codec_ext.h): the library's host encoder against the oracle's independent
decoder written from the format text. Decode must be bit-exact: every symbol equals the absmax quantiser's symbol
(the quantiser itself is checked against a numpy closed form), scales equal, and every rANS stream ends exactly at
its word count with all 64 states back at 2^16."""
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


@pytest.mark.parametrize("codec", [1, 2])
@pytest.mark.parametrize("D", [64, 128])
def test_group_roundtrip(kv, codec, D):
    rng = np.random.default_rng(D + codec)
    n = 40                                       # pages
    K = rng.standard_normal((n, 16, D)).astype(np.float32)
    V = rng.standard_normal((n, 16, D)).astype(np.float32)
    K[3] = 0.0                                   # all-zero page (scale 1, every symbol 128)
    V[4] *= 1e4                                  # large magnitudes
    K[5, :, 7] = 50.0                            # one outlier channel
    V[6] = np.sign(V[6])                         # two-valued page
    K[7] = np.linspace(-1, 1, 16 * D, dtype=np.float32).reshape(16, D)
    tc = np.full(n, 16, np.uint32)
    tc[8], tc[9], tc[39] = 1, 11, 5              # partial pages (padded with symbol 128)
    # groups of 4, 3, 2 and 1 pages (absent pages padded), assorted table pairs
    first = np.array([0, 4, 8, 12, 15, 17, 18, 22, 26, 30, 34, 38], np.uint64)
    counts = np.array([4, 4, 4, 3, 2, 1, 4, 4, 4, 4, 4, 2], np.uint32)
    heads = (np.arange(first.size) % 3).astype(np.uint32)
    tables = None
    if codec == 2:
        tables = np.concatenate([kv.build_table(K[h::3][:5]) if s == 0 else kv.build_table(V[h::3][:5])
                                 for h in range(3) for s in range(2)])
    blob, offs = kv.encode_groups(codec, K, V, D, tables, first, counts, heads, tc)
    assert blob.size % 16 == 0 and (offs[1:] > offs[:-1]).all()
    for g in range(first.size):
        o = int(offs[g]) * 16
        ks, vs, ksc, vsc, t = O.kv_decode_group(blob[o:], tables, int(heads[g]), D)
        for G in range(4):
            if G >= counts[g]:
                assert t[G] == 0 and (ks[G] == 128).all() and (vs[G] == 128).all()
                continue
            p = int(first[g]) + G
            n_t = int(tc[p])
            assert t[G] == n_t
            ek, eks = O.kv_quantize_absmax(K[p, :n_t])
            ev, evs = O.kv_quantize_absmax(V[p, :n_t])
            assert ksc[G] == eks and vsc[G] == evs
            assert np.array_equal(ks[G, :n_t], ek) and np.array_equal(vs[G, :n_t], ev), (g, G)
            assert (ks[G, n_t:] == 128).all() and (vs[G, n_t:] == 128).all()


def test_rans_compression_near_entropy(kv):
    """On N(0,1) pages the RANS_HYBRID blob is within 0.3 b/value of the int8 symbol entropy plus the fixed
    per-group overhead (header + 4 x 64 states = 1088 B) — i.e. the coder itself loses little."""
    rng = np.random.default_rng(11)
    n, D = 256, 128
    K = rng.standard_normal((n, 16, D)).astype(np.float32)
    V = rng.standard_normal((n, 16, D)).astype(np.float32)
    tables = np.concatenate([kv.build_table(K[:64]), kv.build_table(V[:64])])
    first = np.arange(0, n, 4, dtype=np.uint64)
    blob, _ = kv.encode_groups(2, K, V, D, tables, first, np.full(first.size, 4, np.uint32))
    syms = np.concatenate([O.kv_quantize_absmax(K[p])[0].ravel() for p in range(n)] +
                          [O.kv_quantize_absmax(V[p])[0].ravel() for p in range(n)])
    c = np.bincount(syms, minlength=256).astype(np.float64)
    pr = c[c > 0] / c.sum()
    h0 = -(pr * np.log2(pr)).sum()
    bits_per_value = blob.size * 8 / (2 * n * 16 * D)
    overhead = 1088 * 8 / (2 * 4 * 16 * D)
    assert bits_per_value < h0 + overhead + 0.3, (bits_per_value, h0, overhead)
    assert bits_per_value < 8.0  # smaller than the raw int8 page


def test_table_every_symbol_codable(kv):
    hist = np.zeros((1, 16, 64), np.float32)  # all-zero sample -> joint symbol 0xAA only
    t = kv.build_table(hist)
    lo = t.view(np.uint32)[0::2]
    f = lo & 2047
    cs = (lo >> 11) & 2047
    j = (lo >> 22) & 255
    starts = cs == 0
    assert starts.sum() == 256 and sorted(j[starts]) == list(range(256))
    assert f[starts].sum() == 2048
    # a page whose high parts never occurred in the sample still codes and decodes
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
        return f(codec, keys, values, n, A, A, None, D, tables, tcount, None, pool, 1 << 30, pool_at, A, A, A, A,
                 ws_bytes, None)

    assert call(keys=None) == 1 and call(values=A + 8) == 1 and call(pool=A + 4) == 1 and call(pool_at=8) == 1
    assert call(n=0) == 1 and call(tables=None) == 1 and call(tcount=1) == 1 and call(ws_bytes=ws - 1) == 1
    assert call(D=20) == 2 and call(D=256) == 2 and call(codec=7) == 2


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
            for g in range((T[s] + 63) // 64):
                is_raw = g < (2 if s != 1 else 3)
                ref = raw if is_raw else rans
                off_m = int(mixed.host_offsets[s, h, g]) * 16
                off_r = int(ref.host_offsets[s, h, g]) * 16
                got = O.kv_decode_group(mixed.host_pool[off_m:off_m + 65536], tables, h, D)
                exp = O.kv_decode_group(ref.host_pool[off_r:off_r + 65536], tables, h, D)
                for a, b in zip(got, exp):
                    assert np.array_equal(a, b), (s, h, g)
                codec = int(mixed.host_pool[off_m:off_m + 4].view(np.uint32)[0])  # cf_kv_group_header.codec
                assert codec == (kv.CODEC_INT8 if is_raw else kv.CODEC_RANS_HYBRID), (s, h, g)
            if s:
                assert np.array_equal(mixed.host_offsets[s, h, :2], mixed.host_offsets[0, h, :2])
    with pytest.raises(ValueError):
        kv.build_batched(kv.CODEC_RANS_HYBRID, *args, tables, "cpu", encoder="device", raw_groups={0: 1})
