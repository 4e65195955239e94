"""Shared builders for the paged-KV tests: synthetic sequences, expected outputs from the fp64 CPU oracle."""
from __future__ import annotations

import numpy as np

import oracle as O


def make_seqs(seq_tokens, kv_heads, D, seed, scale_spread=False, v_mult=None, cancel=None, page_spread=None):
    """K, V ~ N(0,1) per sequence [kv_heads, T, D]. v_mult[s][h] (optional) multiplies all of V of sequence s,
    head h: whole sequences / heads of small or huge V magnitude, so every page scale of that head is small or
    huge (not only single tokens inside a page, as scale_spread does).
    cancel = eps (optional): 16-token pages 2j and 2j + 1 get equal keys (so equal softmax weights) and values v
    and -(1 - eps) v (so the odd page's V scale is the even page's times 1 - eps and its symbols are the negated
    ones): every output is a sum of near-cancelling pairs p (v1 + v2) ~ eps p v, while a kernel that rounds each
    token's weight p * v_scale on its own makes errors of the size of p v that no longer cancel.
    page_spread = b (optional): V of every 16-token page multiplied by 2^u, u uniform in [0, b), so the pages of one
    64-token group have V scales up to 2^b apart."""
    rng = np.random.default_rng(seed)
    data = []
    for s, T in enumerate(seq_tokens):
        K = rng.standard_normal((kv_heads, T, D)).astype(np.float32)
        V = rng.standard_normal((kv_heads, T, D)).astype(np.float32)
        if scale_spread:  # channels / tokens of very different magnitude (outlier channels, tiny tokens)
            K *= rng.choice([0.01, 1.0, 30.0], size=(1, 1, D)).astype(np.float32)
            V *= rng.choice([1e-3, 1.0, 8.0], size=(1, T, 1)).astype(np.float32)
        if v_mult is not None:
            V *= np.asarray(v_mult[s], np.float32).reshape(kv_heads, 1, 1)
        if page_spread is not None:
            npg = (T + 15) // 16
            f = np.exp2(rng.uniform(0, page_spread, size=(kv_heads, npg))).astype(np.float32)
            V *= np.repeat(f, 16, axis=1)[:, :T, None]
        if cancel is not None:
            for p0 in range(0, T - 31, 32):
                K[:, p0 + 16:p0 + 32] = K[:, p0:p0 + 16]
                V[:, p0 + 16:p0 + 32] = -(1.0 - cancel) * V[:, p0:p0 + 16]
        data.append((K, V))
    return data


def decoded_pages(kv, s, h, T):
    """(token_begin, K, V) dequantised pages of sequence s, head h, decoded by the oracle from the host pool (the
    groups in token order, chain states carried from each group to the one that continues it)."""
    D = kv.head_dim
    out = []
    blobs = [kv.host_pool[int(kv.host_offsets[s, h, g]) * 16:][:65536] for g in range((T + 63) // 64)]
    for g, (ks, vs, ksc, vsc, tc) in enumerate(O.kv_decode_run(blobs, kv.host_tables, h, D)):
        for G in range(4):
            p = 4 * g + G
            n = min(16, T - 16 * p)
            if n <= 0:
                assert tc[G] == 0
                continue
            assert tc[G] == n, (s, h, g, G, tc[G], n)
            out.append((16 * p, (ks[G, :n].astype(np.float32) - 128) * ksc[G],
                        (vs[G, :n].astype(np.float32) - 128) * vsc[G]))
    return out


def oracle_batched(kv, data, queries, query_pos, softmax_scale, gqa):
    """fp64 reference over the values the decoder must reproduce: every group blob is decoded by the oracle's own
    decoder (which also checks the stream), dequantised as (sym - 128) * scale."""
    S, H = kv.seq_count, kv.kv_heads
    D = kv.head_dim
    out = np.zeros((S, H * gqa, D), np.float32)
    for s in range(S):
        T = int(data[s][0].shape[1])
        pages = []
        for h in range(H):
            pages += [(h, t0, k, v) for t0, k, v in decoded_pages(kv, s, h, T)]
        o, empty = O.paged_attention_f64(queries[s], H * gqa, H, D, gqa, int(query_pos[s]), 0, softmax_scale, pages)
        out[s] = o
    return out


def normwise_err(got, ref):
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))


def head_err(got, ref):
    """Worst normwise relative error over (sequence, query head) rows: max over rows of max_d |err| / max_d |ref|
    for outputs [S, QH, D]. Unlike normwise_err over the whole batch, a wrong head of small magnitude cannot hide
    behind a large one. Rows whose reference is all zero (nothing visible) must be exactly zero."""
    got = np.asarray(got, np.float64).reshape(-1, got.shape[-1])
    ref = np.asarray(ref, np.float64).reshape(-1, ref.shape[-1])
    den = np.abs(ref).max(axis=1)
    err = np.abs(got - ref).max(axis=1)
    zero = den == 0
    if zero.any() and err[zero].max() != 0:
        return float("inf")
    return float((err[~zero] / den[~zero]).max()) if (~zero).any() else 0.0
