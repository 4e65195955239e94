// ref_shim.cpp — TEST INFRASTRUCTURE ONLY. A C face over the reference's own CPU code so the Python tests can call
// it through ctypes: compiled by `make -C oracle ref` together with the reference sources where they lie
// (/root/reference/src/runtime/{kv_gpu_fixture,kv_reference,kv_runtime}.cpp) into oracle/_ref/libcfref.so, which
// is never committed and never linked into the product. Used only to check the oracle's restatements
// (or_kv_fixture_quantize / or_pack_fixed / or_paged_attention_f64) against the code they restate.
#include <cstdint>
#include <cstring>
#include <exception>
#include <vector>

#include "chromofold/kv_gpu_fixture.hpp"
#include "chromofold/kv_reference.hpp"

extern "C" {

// reference gpu_fixture::encode_int{4,8}_page (kv_gpu_fixture.cpp:46-125). Writes the packed K/V words, scales,
// dequantised values and block offsets; `counts` receives {k_words, v_words, k_blocks, v_blocks, lut_entries,
// zero_point}. Returns 0, or -1 if the reference threw or a buffer is too small.
int cfref_fixture_page(int bits, const float *k, const float *v, uint32_t T, uint32_t D, uint32_t kv_head,
                       uint32_t block, uint32_t cap_words, uint32_t *kw, uint32_t *vw, float *ks, float *vs,
                       float *kdeq, float *vdeq, int32_t *kboff, int32_t *vboff, uint32_t cap_blocks,
                       int32_t *klut, uint32_t cap_lut, uint32_t *counts) {
  try {
    std::vector<float> kk(k, k + size_t(T) * D), vv(v, v + size_t(T) * D);
    namespace gf = chromofold::gpu_fixture;
    const gf::EncodedKvPage p = bits == 4 ? gf::encode_int4_page(kk, vv, 0, T, D, kv_head, block)
                                          : gf::encode_int8_page(kk, vv, 0, T, D, kv_head, block);
    if (p.k.words.size() > cap_words || p.v.words.size() > cap_words || p.k.block_offsets.size() > cap_blocks ||
        p.v.block_offsets.size() > cap_blocks || p.k.lut.size() > cap_lut)
      return -1;
    std::memcpy(kw, p.k.words.data(), 4 * p.k.words.size());
    std::memcpy(vw, p.v.words.data(), 4 * p.v.words.size());
    std::memcpy(ks, p.k_scales.data(), 4 * p.k_scales.size());
    std::memcpy(vs, p.v_scales.data(), 4 * p.v_scales.size());
    std::memcpy(kdeq, p.dequantized_k.data(), 4 * p.dequantized_k.size());
    std::memcpy(vdeq, p.dequantized_v.data(), 4 * p.dequantized_v.size());
    std::memcpy(kboff, p.k.block_offsets.data(), 4 * p.k.block_offsets.size());
    std::memcpy(vboff, p.v.block_offsets.data(), 4 * p.v.block_offsets.size());
    std::memcpy(klut, p.k.lut.data(), 4 * p.k.lut.size());
    counts[0] = uint32_t(p.k.words.size());
    counts[1] = uint32_t(p.v.words.size());
    counts[2] = uint32_t(p.k.block_offsets.size());
    counts[3] = uint32_t(p.v.block_offsets.size());
    counts[4] = uint32_t(p.k.lut.size());
    counts[5] = p.zero_point;
    return 0;
  } catch (const std::exception &) {
    return -1;
  }
}

// reference::seal_int4_page + dequantize_page (kv_reference.cpp): one int4 page's dequantised K/V [T, D].
int cfref_seal_dequant(const float *k, const float *v, uint32_t token_begin, uint32_t T, uint32_t kv_head,
                       uint32_t D, float *kdeq, float *vdeq) {
  try {
    namespace rf = chromofold::reference;
    const rf::SealedKvPage p = rf::seal_int4_page(k, v, token_begin, T, 0, kv_head, D);
    std::vector<float> dk, dv;
    rf::dequantize_page(p, &dk, &dv);
    std::memcpy(kdeq, dk.data(), 4 * dk.size());
    std::memcpy(vdeq, dv.data(), 4 * dv.size());
    return 0;
  } catch (const std::exception &) {
    return -1;
  }
}

// reference::paged_attention (kv_reference.cpp:164-243) over int4 pages sealed from raw K/V (page i: kv_head[i],
// token_begin[i], ntok[i] rows starting at row off[i] of k/v) and an optional active tail per kv head ([tail_n,
// kv_heads, D], starting at tail_begin). One query row. Returns 0, 1 if the reference threw (e.g. nothing
// visible, overlapping pages).
int cfref_paged_attention(const float *q, uint32_t q_heads, uint32_t kv_heads, uint32_t D, uint32_t query_token,
                          uint32_t window, float scale, uint32_t n_pages, const uint32_t *kvh, const uint32_t *tok0,
                          const uint32_t *ntok, const uint64_t *off, const float *k, const float *v,
                          const float *tail_k, const float *tail_v, uint32_t tail_begin, uint32_t tail_n,
                          float *out) {
  try {
    namespace rf = chromofold::reference;
    std::vector<rf::SealedKvPage> pages;
    for (uint32_t i = 0; i < n_pages; ++i)
      pages.push_back(rf::seal_int4_page(k + off[i] * D, v + off[i] * D, tok0[i], ntok[i], 0, kvh[i], D));
    // the tail arrives as [tail_n, kv_heads, D]; the reference's ActiveKvTail is per head, row-major [n, D]
    std::vector<std::vector<float>> tk(kv_heads), tv(kv_heads);
    std::vector<rf::ActiveKvTail> tails;
    if (tail_n) {
      for (uint32_t h = 0; h < kv_heads; ++h) {
        tk[h].resize(size_t(tail_n) * D);
        tv[h].resize(size_t(tail_n) * D);
        for (uint32_t t = 0; t < tail_n; ++t)
          for (uint32_t d = 0; d < D; ++d) {
            tk[h][size_t(t) * D + d] = tail_k[(size_t(t) * kv_heads + h) * D + d];
            tv[h][size_t(t) * D + d] = tail_v[(size_t(t) * kv_heads + h) * D + d];
          }
        rf::ActiveKvTail a;
        a.token_begin = tail_begin;
        a.token_count = tail_n;
        a.layer = 0;
        a.kv_head = h;
        a.head_dim = D;
        a.k = tk[h].data();
        a.v = tv[h].data();
        tails.push_back(a);
      }
    }
    rf::AttentionShape s;
    s.query_count = 1;
    s.query_head_count = q_heads;
    s.kv_head_count = kv_heads;
    s.head_dim = D;
    s.query_token_begin = query_token;
    s.causal_window = window;
    s.score_scale = scale;
    std::vector<float> o;
    rf::paged_attention(pages, tails, q, s, &o);
    std::memcpy(out, o.data(), 4 * o.size());
    return 0;
  } catch (const std::exception &) {
    return 1;
  }
}

}  // extern "C"
