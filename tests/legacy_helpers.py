"""Builders of reference-format KV pages for the legacy-seam tests: fixed-width pages exactly as the reference's
encoder writes them (src/runtime/kv_gpu_fixture.cpp:20-95, via the oracle's restatement) and canonical
length-limited Huffman pages (the reference decoder's LUT format, include/chromofold/detail/block_huffman_device.cuh;
its encoder lived in the absent warp_compress prototype, so this test-side encoder is checked by round trip
through the oracle's LUT decoder)."""
from __future__ import annotations

import heapq

import numpy as np

import oracle as O
from chromofold_amd.legacy import HostPage


def fixed_page(k, v, kv_head, token_begin, bits, block=64):
    """Reference fixture page: K per-channel / V per-token scales, fixed-width MSB-first, degenerate LUT."""
    ks, vs, ksc, vsc, kd, vd = O.kv_fixture_quantize(k, v, bits)
    n = ks.size
    boff = (np.arange(0, n, block, dtype=np.int64) * bits).astype(np.int32)
    lut = np.array([s | (bits << 8) for s in range(1 << bits)], np.int32)
    page = HostPage(kv_head, token_begin, k.shape[0], k.shape[1], O.pack_fixed(ks, bits), boff, lut, ksc,
                    O.pack_fixed(vs, bits), boff.copy(), lut.copy(), vsc, block, bits, bits, 1 << (bits - 1), bits)
    return page, kd, vd


def huffman_lengths(freq, maxlen):
    """Huffman code lengths, then length-limited: clamp to maxlen and lengthen the deepest shorter codes until the
    Kraft sum is <= 1 (every symbol with nonzero frequency gets a code)."""
    syms = [s for s in range(len(freq)) if freq[s] > 0]
    if len(syms) == 1:
        L = np.zeros(len(freq), np.int32)
        L[syms[0]] = 1
        return L
    heap = [(int(freq[s]), i, [s]) for i, s in enumerate(syms)]
    heapq.heapify(heap)
    depth = np.zeros(len(freq), np.int32)
    uid = len(heap)
    while len(heap) > 1:
        f1, _, a = heapq.heappop(heap)
        f2, _, b = heapq.heappop(heap)
        for s in a + b:
            depth[s] += 1
        heapq.heappush(heap, (f1 + f2, uid, a + b))
        uid += 1
    L = np.minimum(depth, maxlen)
    L[[s for s in range(len(freq)) if freq[s] == 0]] = 0
    while sum(2.0 ** -int(l) for l in L if l) > 1.0:
        cand = [s for s in range(len(freq)) if 0 < L[s] < maxlen]
        s = max(cand, key=lambda x: (L[x], -freq[x]))
        L[s] += 1
    return L


def canonical_codes(L):
    order = sorted([s for s in range(len(L)) if L[s] > 0], key=lambda s: (L[s], s))
    codes, code, prev = {}, 0, 0
    for s in order:
        code <<= (L[s] - prev)
        codes[s] = (code, int(L[s]))
        prev = L[s]
        code += 1
    return codes


def huffman_stream(sym, codes, maxlen, block):
    """MSB-first bit stream + bit offsets of every block + LUT (lut[look] = sym | len << 8)."""
    bits, boff = [], []
    for i, s in enumerate(sym):
        if i % block == 0:
            boff.append(len(bits))
        c, l = codes[int(s)]
        bits.extend((c >> (l - 1 - j)) & 1 for j in range(l))
    bits.extend([0] * (maxlen + 32))
    bits.extend([0] * (-len(bits) % 32))
    nw = (len(bits) + 31) // 32
    arr = np.array(bits[:nw * 32], np.uint64).reshape(nw, 32)
    words = (arr << np.arange(31, -1, -1, dtype=np.uint64)).sum(1).astype(np.uint32)
    lut = np.zeros(1 << maxlen, np.int32)
    for s, (c, l) in codes.items():
        base = c << (maxlen - l)
        lut[base:base + (1 << (maxlen - l))] = s | (l << 8)
    return words, np.array(boff, np.int32), lut


def huffman_page(k, v, kv_head, token_begin, bits=8, maxlen=12, block=64):
    """Fixture quantisation, then canonical Huffman per stream (variable-length codes, fixed_code_length 0)."""
    ks, vs, ksc, vsc, kd, vd = O.kv_fixture_quantize(k, v, bits)
    out = []
    for sym in (ks.ravel(), vs.ravel()):
        freq = np.bincount(sym, minlength=1 << bits)
        codes = canonical_codes(huffman_lengths(freq, maxlen))
        w, b, lut = huffman_stream(sym, codes, maxlen, block)
        assert np.array_equal(O.huffman_decode(w, lut, maxlen, 0, sym.size), sym)  # round trip
        out.append((w, b, lut))
    (kw, kb, kl), (vw, vb, vl) = out
    page = HostPage(kv_head, token_begin, k.shape[0], k.shape[1], kw, kb, kl, ksc, vw, vb, vl, vsc, block, maxlen,
                    maxlen, 1 << (bits - 1), 0)
    return page, kd, vd


def huffman_stream_np(sym, lengths, maxlen, block):
    """Vectorised twin of huffman_stream for large inputs: canonical codes from `lengths` (per symbol value), MSB-first
    packing, bit offset of every block, LUT. Codes of different symbols never share bits, so OR-packing is a sum."""
    sym = np.asarray(sym).ravel().astype(np.int64)
    codes = canonical_codes(lengths)
    cv = np.zeros(len(lengths), np.uint64)
    cl = np.zeros(len(lengths), np.int64)
    for s, (c, l) in codes.items():
        cv[s], cl[s] = c, l
    L = cl[sym]
    assert (L > 0).all(), "symbol without a code"
    pos = np.concatenate([[0], np.cumsum(L)[:-1]])
    nbits = int(pos[-1] + L[-1]) if sym.size else 0
    nw = (nbits + maxlen + 64) // 32 + 1
    wide = np.zeros(nw + 1, np.uint64)  # 64-bit accumulation of each code's window [word, word + 1]
    w0 = pos >> 5
    shift = (64 - L - (pos & 31)).astype(np.uint64)
    v = cv[sym] << shift
    hi, lo = (v >> np.uint64(32)), (v & np.uint64(0xFFFFFFFF))
    np.add.at(wide, w0, hi)
    np.add.at(wide, w0 + 1, lo)
    words = wide[:nw].astype(np.uint32)
    boff = pos[::block].astype(np.int32)
    lut = np.zeros(1 << maxlen, np.int32)
    for s, (c, l) in codes.items():
        base = c << (maxlen - l)
        lut[base:base + (1 << (maxlen - l))] = s | (l << 8)
    return words, boff, lut


def rans_encode_blocks(sym, freq, block):
    """Block rANS encoder for the reference decoder format (src/cuda/rans.cu:11-50: M = 4096, L = 2^23, 32-bit
    state, byte renormalisation read upward): each block encoded backwards, its bytes stored in read order.
    Returns data, byte_off, state0, slot2sym, freq, cum."""
    sym = np.asarray(sym, np.int64)
    freq = np.asarray(freq, np.int64)
    assert freq.sum() == 4096
    cum = np.concatenate([[0], np.cumsum(freq)[:-1]])
    slot2sym = np.repeat(np.arange(freq.size), freq).astype(np.int32)
    L = 1 << 23
    data, boff, st0 = [], [], []
    for b0 in range(0, sym.size, block):
        x = L
        out = []
        for s in sym[b0:b0 + block][::-1]:
            f, c = int(freq[s]), int(cum[s])
            xmax = ((L >> 12) << 8) * f
            while x >= xmax:
                out.append(x & 0xFF)
                x >>= 8
            x = ((x // f) << 12) + (x % f) + c
        boff.append(len(data))
        data.extend(out[::-1])
        st0.append(x)
    data.extend([0] * 8)
    return (np.array(data, np.uint8), np.array(boff, np.int32), np.array(st0, np.uint32), slot2sym,
            freq.astype(np.int32), cum.astype(np.int32))


def rans_page(k, v, kv_head, token_begin, codec=2, tables=None, continues=False, second=None):
    """An rANS page of the reference seam (tag: fixed_code_length == 0 and k_max_code_length == 0): one
    kv_codec_ext.h group of up to 64 tokens, coded on its own by the library's host encoder (codec 2 = RANS_HYBRID,
    1 = INT8), k_words = the blob, k_lut / v_lut = its K and V tables. kd / vd are the values the oracle decodes from
    the blob. `continues` codes it as the second group of a chain pair after `second` (k, v of the first group) and
    returns that second blob: a page the seam must refuse."""
    from chromofold_amd import kv
    T, D = k.shape

    def pages_of(x):
        n = (x.shape[0] + 15) // 16
        P = np.zeros((n, 16, D), np.float32)
        P.reshape(-1, D)[:x.shape[0]] = x
        return P, np.array([min(16, x.shape[0] - 16 * g) for g in range(n)], np.uint32)
    K, tc = pages_of(k)
    V, _ = pages_of(v)
    npg = K.shape[0]
    if tables is None:
        tables = np.concatenate([kv.build_table(K), kv.build_table(V)])
    if continues:
        K0, tc0 = pages_of(second[0])
        V0, _ = pages_of(second[1])
        blob, offs = kv.encode_groups(codec, np.concatenate([K0, K]), np.concatenate([V0, V]), D, tables,
                                      np.array([0, K0.shape[0]], np.uint64), np.array([K0.shape[0], npg], np.uint32),
                                      np.array([0, 0], np.uint32), np.concatenate([tc0, tc]),
                                      continues=np.array([0, 1], np.uint8))
        blob = blob[int(offs[1]) * 16:].copy()
        kd = vd = None
    else:
        blob, _ = kv.encode_groups(codec, K, V, D, tables, np.array([0], np.uint64), np.array([npg], np.uint32),
                                   np.array([0], np.uint32), tc)
        ks, vs, ksc, vsc, _ = O.kv_decode_group(blob, tables, 0, D)
        kd = np.concatenate([(ks[g, :tc[g]].astype(np.float32) - 128) * ksc[g] for g in range(npg)])
        vd = np.concatenate([(vs[g, :tc[g]].astype(np.float32) - 128) * vsc[g] for g in range(npg)])
    tb = kv.TABLE_BYTES
    zi, zf = np.zeros(4, np.int32), np.zeros(4, np.float32)
    page = HostPage(kv_head, token_begin, T, D, blob, zi, tables[:tb], zf, blob[:16], zi, tables[tb:2 * tb], zf,
                    64, 0, 0, 128, 0)
    return page, kd, vd
