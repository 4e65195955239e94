"""Pins the oracle's restatements against the reference's own CPU code, compiled from its sources into oracle/_ref/
by `make -C oracle ref` (only where the reference tree is mounted; skipped elsewhere):

  * or_kv_fixture_quantize + or_pack_fixed  vs  gpu_fixture::encode_int{4,8}_page (kv_gpu_fixture.cpp:46-125):
    words, block offsets, scales and dequantised values bit for bit;
  * or_paged_attention_f64  vs  reference::paged_attention (kv_reference.cpp:164-243) over int4 pages sealed by the
    reference itself, with GQA, causal windows and an active tail;
  * the oracle's RRR-wavelet builder  vs  tools/build_index (the reference's .cfrw writer) on Markov streams larger
    than the committed tiny fixture: every array byte for byte, and the tool's own access/rank goldens.
"""
import os
import subprocess

import numpy as np
import pytest

import cf_fixtures as F
import oracle as O

needs_ref = pytest.mark.skipif(O.ref_lib() is None, reason="oracle/_ref not built (reference tree not mounted)")


@needs_ref
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("T,D", [(16, 64), (16, 128), (7, 96), (32, 32)])
def test_fixture_encoder_matches_reference(bits, T, D):
    rng = np.random.default_rng(bits * 1000 + T * 10 + D)
    k = rng.standard_normal((T, D)).astype(np.float32) * 1.7
    v = rng.standard_normal((T, D)).astype(np.float32) * 0.3
    k[0, :] = 0.0  # a zero row and zero column exercise the scale-1.0 fallback
    v[:, 1] = 0.0
    ref = O.ref_fixture_page(bits, k, v)
    ks, vs, ksc, vsc, kd, vd = O.kv_fixture_quantize(k, v, bits)
    assert np.array_equal(ksc, ref["ks"]) and np.array_equal(vsc, ref["vs"])
    assert np.array_equal(kd, ref["kdeq"]) and np.array_equal(vd, ref["vdeq"])
    assert np.array_equal(O.pack_fixed(ks, bits), ref["kw"]) and np.array_equal(O.pack_fixed(vs, bits), ref["vw"])
    assert np.array_equal(ref["kboff"], np.arange(0, T * D, 64, dtype=np.int64).astype(np.int32) * bits)
    assert ref["zero_point"] == 1 << (bits - 1)
    assert np.array_equal(ref["lut"], np.array([s | (bits << 8) for s in range(1 << bits)], np.int32))


def _pages(rng, kv_heads, D, spans):
    pages = []
    for h in range(kv_heads):
        for t0, n in spans:
            pages.append((h, t0, rng.standard_normal((n, D)).astype(np.float32),
                          rng.standard_normal((n, D)).astype(np.float32)))
    return pages


@needs_ref
@pytest.mark.parametrize("q_heads,kv_heads,D", [(4, 4, 32), (14, 2, 64), (32, 8, 128)])
@pytest.mark.parametrize("window", [0, 5, 40])
def test_paged_attention_oracle_matches_reference(q_heads, kv_heads, D, window):
    rng = np.random.default_rng(q_heads * 100 + D + window)
    spans = [(32, 16), (0, 16), (16, 16), (48, 9)]  # out of order, ragged last page
    raw = _pages(rng, kv_heads, D, spans)
    tail_n = 3
    tail = (57, rng.standard_normal((tail_n, kv_heads, D)).astype(np.float32),
            rng.standard_normal((tail_n, kv_heads, D)).astype(np.float32))
    q = rng.standard_normal((q_heads, D)).astype(np.float32)
    scale = 1.0 / np.sqrt(D)
    for query_token in (59, 50, 20):
        ref = O.ref_paged_attention(q, q_heads, kv_heads, D, query_token, window, scale, raw, tail)
        assert ref is not None
        deq = [(h, t0, *O.ref_seal_dequant(k, v, t0, h)) for h, t0, k, v in raw]
        got, empty = O.paged_attention_f64(q, q_heads, kv_heads, D, q_heads // kv_heads, query_token, window, scale,
                                           deq, tail)
        assert empty == 0
        np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-7)


@needs_ref
def test_paged_attention_empty_visible_set():
    """The reference CPU path throws when nothing is visible; the oracle (like the GPU seam) reports it."""
    rng = np.random.default_rng(3)
    raw = _pages(rng, 1, 32, [(100, 16)])
    q = rng.standard_normal((1, 32)).astype(np.float32)
    assert O.ref_paged_attention(q, 1, 1, 32, 50, 0, 0.2, raw) is None
    deq = [(h, t0, *O.ref_seal_dequant(k, v, t0, h)) for h, t0, k, v in raw]
    got, empty = O.paged_attention_f64(q, 1, 1, 32, 1, 50, 0, 0.2, deq)
    assert empty == 1 and not got.any()


def _bwt_of(tokens):
    s = np.concatenate([tokens.astype(np.int64) + 1, [0]]).astype(np.int32)
    sa = O.suffix_array(s)
    return s[(sa.astype(np.int64) - 1) % s.size].astype(np.uint32)


@pytest.mark.skipif(O.ref_build_index() is None, reason="oracle/_ref/build_index not built")
@pytest.mark.parametrize("n,vocab,seed", [(5000, 64, 1), (20011, 300, 7), (3, 2, 4)])
def test_rrr_builder_matches_reference_tool(tmp_path, n, vocab, seed):
    out, tok = str(tmp_path / "x.cfrw"), str(tmp_path / "x.tok")
    subprocess.run([O.ref_build_index(), out, "--n", str(n), "--vocab", str(vocab), "--queries", "200", "--rank",
                    "200", "--seed", str(seed), "--dump-tokens", tok], check=True, capture_output=True, timeout=120)
    raw = np.fromfile(tok, dtype=np.uint8)
    assert int(raw[:8].view(np.int64)[0]) == n
    tokens = raw[8:].view(np.int32)
    d = F.load_cfrw(out)
    bwt = _bwt_of(tokens)
    w = O.rrrw_build(bwt, d["bits"])
    for f in ["classes", "offsets", "rank_a", "rank_d", "off_a", "off_d", "offbase", "zeros"]:
        assert np.array_equal(getattr(w, f), d[f]), f
    assert w.rrr_bytes == d["rrr_bytes"]
    assert np.array_equal(O.rrrw_access(w, d["pos"]), d["access_golden"])
    assert np.array_equal(O.rrrw_rank(w, d["rank_c"], d["rank_i"]), d["rank_golden"])
