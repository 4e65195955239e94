// oracle_kv.cpp — TEST INFRASTRUCTURE ONLY (see oracle_succinct.cpp header). CPU restatements for the paged-KV
// path, used as the checker of the HIP kernels; never linked into libchromofold.so.
//
//   fixture quantiser + fixed-width packing   reference src/runtime/kv_gpu_fixture.cpp:12-95
//   paged attention, fp64 online softmax      reference src/runtime/kv_reference.cpp:50-67,164-243 and the GPU
//                                             seam semantics of src/cuda/paged_kv_attention.cu:41-176 (window,
//                                             GQA h / gqa_group_size, active tail, no visible token -> zeros)
//   canonical Huffman LUT decode              reference include/chromofold/detail/block_huffman_device.cuh:12-19
//   block rANS decode                         reference src/cuda/rans.cu:16-26
//   RANS_HYBRID / INT8 page decode            the byte format written out in include/chromofold/kv_codec_ext.h
//                                             (this project's codec; restated here from the format text, not
//                                             from the product encoder, so a format slip shows as a mismatch)
//   windowed attention (fp64)                 reference src/cuda/fused_kv_attention.cu:27-65
//
// Parity pins (tests/test_oracle_vs_reference.py, tests/test_oracle_codecs.py, tests/test_kv_codec.py):
//   quantiser + packing      bit-identical to the reference's own encode_int{4,8}_page, compiled from its sources
//   paged attention          within 1e-6 of the reference's own paged_attention (GQA, windows, tail, page order)
//   dense / window attention reduce to the pinned paged attention on one page (closed-form special case)
//   Huffman LUT decode       inverts two independent packers (per-symbol and vectorised) from any block offset
//   block rANS decode        inverts an independent encoder (ryg-style byte renormalisation), incl. the
//                            single-symbol distribution and 1-symbol blocks; a corrupted byte changes the output
//   group decode             inverts the product encoder and reproduces the quantiser's symbols exactly
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

extern "C" {

// ---------------------------------------------------------------------------------------- fixture quantiser
// K per-channel scale, V per-token scale, both max|x|/qmax (0 -> 1.0); sym = clamp(lrint(x/s), -(qmax+1), qmax)
// + zp; fixed-width MSB-first packing, block offsets every block_size symbols. Outputs: syms [T*D] (K then V),
// scales (K [D] then V [T]), dequantised values (K then V).
void or_kv_fixture_quantize(const float *k, const float *v, uint32_t T, uint32_t D, uint32_t bits, uint8_t *k_sym,
                            uint8_t *v_sym, float *k_scales, float *v_scales, float *k_deq, float *v_deq) {
  const int qmax = (1 << (bits - 1)) - 1, zp = 1 << (bits - 1);
  for (uint32_t d = 0; d < D; ++d) {
    float m = 0.0f;
    for (uint32_t t = 0; t < T; ++t) m = std::max(m, std::fabs(k[(size_t)t * D + d]));
    k_scales[d] = m == 0.0f ? 1.0f : m / (float)qmax;
  }
  for (uint32_t t = 0; t < T; ++t) {
    float m = 0.0f;
    for (uint32_t d = 0; d < D; ++d) m = std::max(m, std::fabs(v[(size_t)t * D + d]));
    v_scales[t] = m == 0.0f ? 1.0f : m / (float)qmax;
  }
  for (uint32_t t = 0; t < T; ++t)
    for (uint32_t d = 0; d < D; ++d) {
      const size_t i = (size_t)t * D + d;
      const int qk = std::clamp((int)std::lrint(k[i] / k_scales[d]), -(qmax + 1), qmax);
      const int qv = std::clamp((int)std::lrint(v[i] / v_scales[t]), -(qmax + 1), qmax);
      k_sym[i] = (uint8_t)(qk + zp);
      v_sym[i] = (uint8_t)(qv + zp);
      k_deq[i] = (float)qk * k_scales[d];
      v_deq[i] = (float)qv * v_scales[t];
    }
}

// MSB-first fixed-width packing (reference kv_gpu_fixture.cpp:31-41); words must be zeroed, n*bits/32 rounded up.
void or_pack_fixed(const uint8_t *sym, uint64_t n, uint32_t bits, uint32_t *words) {
  for (uint64_t i = 0; i < n; ++i) {
    const uint64_t bit = i * bits;
    words[bit >> 5] |= (uint32_t)(sym[i] & ((1u << bits) - 1u)) << ((32u - bits) - (uint32_t)(bit & 31u));
  }
}

// canonical-Huffman LUT decode of n symbols starting at bit `pos` (reference block_huffman_device.cuh:12-19:
// read maxlen bits MSB-first, lut[look] = sym | len << 8)
void or_huffman_decode(const uint32_t *words, const int32_t *lut, int maxlen, int64_t pos, int64_t n,
                       int32_t *out) {
  for (int64_t i = 0; i < n; ++i) {
    int look = 0;
    for (int b = 0; b < maxlen; ++b) {
      const int64_t w = pos + b;
      look = (look << 1) | (int)((words[w >> 5] >> (31 - (w & 31))) & 1u);
    }
    const int e = lut[look];
    out[i] = e & 0xff;
    pos += e >> 8;
  }
}

// block rANS decode (reference src/cuda/rans.cu:16-36): M = 4096, L = 2^23, byte renorm ascending
void or_rans_block_decode(const uint8_t *data, const int32_t *byte_off, const uint32_t *state0,
                          const int32_t *slot2sym, const int32_t *freq, const int32_t *cum, int block, int n,
                          int32_t *out) {
  const int nb = (n + block - 1) / block;
  for (int b = 0; b < nb; ++b) {
    int pos = byte_off[b];
    uint32_t x = state0[b];
    const int cnt = std::min(block, n - b * block);
    for (int j = 0; j < cnt; ++j) {
      const int slot = (int)(x & 4095u);
      const int s = slot2sym[slot];
      x = (uint32_t)freq[s] * (x >> 12) + (uint32_t)(slot - cum[s]);
      while (x < (1u << 23)) x = (x << 8) | data[pos++];
      out[b * block + j] = s;
    }
  }
}

// Interleaved pair-rANS matrix decode (the CF_QW_CODEC_RANS layout of include/chromofold/chromofold_qw.h): per
// band a 256-pair table of cumulative starts (frequencies summing to 4096), per 256-column stripe 64 lane states decoding 32 pairs each, the words of a step
// taken by the lanes that need one in lane order; a band's slots are nchunks - 1 of chunk_words and one of
// last_words 16-bit words. The decode step is the block-rANS step of reference
// src/cuda/rans.cu:16-24 (slot lookup, x = f * (x >> 12) + slot - cum) with 16-bit renormalisation words and
// L = 2^16. Writes sym[rows * cols]; returns the number of stripes whose lanes do not end at 2^16 or whose word
// cursor does not end at the next stripe's first word (0 for a consistent matrix).
// `mistake` plants an error for the tests that show the checks catch one: 1 = words taken in reverse lane order,
// 2 = stripe columns with the roles of g and (t >> 1) & 3 swapped, 3 = x off by one after the update.
int or_qw_rans_decode(const uint16_t *w16, uint32_t chunk_words, uint32_t last_words, const uint32_t *offsets,
                      const uint32_t *states, const uint16_t *cums, uint32_t rows, uint32_t cols, int mistake,
                      uint8_t *sym) {
  const uint64_t bands = (rows + 15) / 16, nstripes = (cols + 255ull) / 256, nchunks = (nstripes + 15) / 16;
  const uint64_t band_words = (nchunks - 1) * chunk_words + last_words;
  int bad = 0;
  for (uint64_t b = 0; b < bands; ++b) {
    uint32_t cum[257], f[256];
    for (int s = 0; s < 256; ++s) cum[s] = cums[b * 256 + s];
    cum[256] = 4096;
    for (int s = 0; s < 256; ++s) f[s] = cum[s + 1] - cum[s];
    std::vector<uint8_t> of_slot(4096);
    for (int s = 0; s < 256; ++s)
      for (uint32_t k = cum[s]; k < cum[s + 1] && k < 4096; ++k) of_slot[k] = static_cast<uint8_t>(s);
    for (uint64_t st = 0; st < nstripes; ++st) {
      const uint64_t ch = st / 16;
      const uint16_t *slot = w16 + b * band_words + ch * chunk_words;
      const uint64_t slot_words = ch + 1 == nchunks ? last_words : chunk_words;
      uint64_t cur = offsets[b * nstripes + st];
      uint32_t x[64];
      for (int l = 0; l < 64; ++l) x[l] = states[(b * nstripes + st) * 64 + l];
      for (int t = 0; t < 32; ++t) {
        bool need[64];
        for (int l = 0; l < 64; ++l) {
          const uint32_t slot_i = x[l] & 4095u;
          const int s = of_slot[slot_i];
          x[l] = f[s] * (x[l] >> 12) + slot_i - cum[s] + (mistake == 3 ? 1u : 0u);
          need[l] = x[l] < 65536u;
          const int g = l >> 4, r = l & 15, jj = (t >> 1) & 3;
          const int c0 = 64 * (t >> 3) + (mistake == 2 ? 16 * jj + 4 * g : 16 * g + 4 * jj) + 2 * (t & 1);
          const uint64_t row = b * 16 + r;
          for (int e = 0; e < 2; ++e) {
            const uint64_t c = st * 256 + c0 + e;
            if (row < rows && c < cols) sym[row * cols + c] = static_cast<uint8_t>((s >> (4 * e)) & 15);
          }
        }
        for (int i = 0; i < 64; ++i) {
          const int l = mistake == 1 ? 63 - i : i;
          if (need[l]) x[l] = (x[l] << 16) | slot[cur++];
        }
      }
      for (int l = 0; l < 64; ++l) bad += x[l] != 65536u ? 1 : 0;
      const bool last_in_chunk = st + 1 == nstripes || (st + 1) % 16 == 0;
      if (!last_in_chunk && cur != offsets[b * nstripes + st + 1]) ++bad;
      if (cur > slot_words) ++bad;
    }
  }
  return bad;
}

// ---------------------------------------------------------------------------------------- paged attention
// One query row per call. Pages: for page p, kv head kvh[p], tokens [tok0[p], tok0[p]+ntok[p]), dequantised K/V
// at k + off[p]*D ([ntok, D] row-major). Tail: [tail_n, kv_heads, D] starting at tail_tok0. Output [q_heads, D].
// Returns the number of heads that had no visible token (their output is zero, as the GPU seam writes).
int or_paged_attention_f64(const float *q, uint32_t q_heads, uint32_t kv_heads, uint32_t D, uint32_t gqa,
                           uint32_t query_token, uint32_t window, float scale, uint32_t npages,
                           const uint32_t *kvh, const uint32_t *tok0, const uint32_t *ntok, const uint64_t *off,
                           const float *k, const float *v, const float *tail_k, const float *tail_v,
                           uint32_t tail_tok0, uint32_t tail_n, float *out) {
  const uint32_t lo = (window == 0 || query_token + 1 <= window) ? 0u : query_token + 1 - window;
  int empty = 0;
  for (uint32_t h = 0; h < q_heads; ++h) {
    const uint32_t kh = h / gqa;
    const float *qq = q + (size_t)h * D;
    double m = -std::numeric_limits<double>::infinity(), den = 0.0;
    std::vector<double> w(D, 0.0);
    auto add = [&](const float *kr, const float *vr) {
      double dot = 0.0;
      for (uint32_t d = 0; d < D; ++d) dot += (double)qq[d] * kr[d];
      const double s = dot * scale;
      const double nm = std::max(m, s);
      const double a = den == 0.0 ? 0.0 : std::exp(m - nm), b = std::exp(s - nm);
      den = den * a + b;
      for (uint32_t d = 0; d < D; ++d) w[d] = w[d] * a + (double)vr[d] * b;
      m = nm;
    };
    for (uint32_t p = 0; p < npages; ++p) {
      if (kvh[p] != kh) continue;
      for (uint32_t t = 0; t < ntok[p]; ++t) {
        const uint32_t tok = tok0[p] + t;
        if (tok < lo || tok > query_token) continue;
        add(k + (off[p] + t) * D, v + (off[p] + t) * D);
      }
    }
    for (uint32_t t = 0; t < tail_n; ++t) {
      const uint32_t tok = tail_tok0 + t;
      if (tok < lo || tok > query_token) continue;
      add(tail_k + ((size_t)t * kv_heads + kh) * D, tail_v + ((size_t)t * kv_heads + kh) * D);
    }
    for (uint32_t d = 0; d < D; ++d) out[(size_t)h * D + d] = den > 0.0 ? (float)(w[d] / den) : 0.0f;
    if (den == 0.0) ++empty;
  }
  return empty;
}

// Dense attention of one query row against contiguous K/V [T, D] of one kv head (all tokens < T visible
// up to query_token): the closed form the paged result must equal (reference tests/kv_reference_test.cpp:47-120).
void or_dense_attention_f64(const float *q, uint32_t D, const float *k, const float *v, uint32_t T, float scale,
                            float *out) {
  double m = -std::numeric_limits<double>::infinity();
  std::vector<double> s(T);
  for (uint32_t t = 0; t < T; ++t) {
    double dot = 0.0;
    for (uint32_t d = 0; d < D; ++d) dot += (double)q[d] * k[(size_t)t * D + d];
    s[t] = dot * scale;
    m = std::max(m, s[t]);
  }
  double den = 0.0;
  std::vector<double> w(D, 0.0);
  for (uint32_t t = 0; t < T; ++t) {
    const double e = std::exp(s[t] - m);
    den += e;
    for (uint32_t d = 0; d < D; ++d) w[d] += e * v[(size_t)t * D + d];
  }
  for (uint32_t d = 0; d < D; ++d) out[d] = (float)(w[d] / den);
}

// Causal-windowed attention of reference src/cuda/fused_kv_attention.cu:27-65 over dequantised rows K/V [seq, dim]:
// query i attends rows [max(0, i - window + 1), i], i.e. the dense attention above over that slice.
void or_kv_window_attention_f64(const float *K, const float *V, const float *Q, int seq, int dim, int nq, int window,
                                float sscale, float *out) {
  (void)seq;
  for (int i = 0; i < nq; ++i) {
    const int lo = std::max(0, i - window + 1);
    or_dense_attention_f64(Q + (size_t)i * dim, (uint32_t)dim, K + (size_t)lo * dim, V + (size_t)lo * dim,
                           (uint32_t)(i - lo + 1), sscale, out + (size_t)i * dim);
  }
}

// ---------------------------------------------------------------------------------------- kv_codec_ext pages
// Decode one INT8 / RANS_HYBRID (format 4) page-group blob into symbols [4 pages][16 tokens][D] for K and V
// (token-major, offset binary q + 128) plus per-page scales and token counts. tables: table blobs (16 KiB each);
// K uses tables[2*head], V tables[2*head+1]. states_io [2 x 64] (K lanes, then V lanes): for a RANS group that
// continues its chain (header chain == 0) the lane states the previous group of the chain ended with; on return
// the states this group ends with (a chain must end with every state at 2^16: the caller checks that where a chain
// ends). *chain_out = the header's chain flag (1 for INT8 groups). Returns 0 on success, -1 on a format
// inconsistency (bad codec or head_dim, a table whose spread word disagrees with its symbol, a stream over-run, a
// cursor short of its word count).
int or_kv_decode_group(const uint8_t *blob, const uint8_t *tables, uint32_t head, uint8_t *k_sym, uint8_t *v_sym,
                       float *k_scale, float *v_scale, uint32_t *token_count, uint32_t *states_io,
                       uint32_t *chain_out) {
  uint32_t codec;
  uint16_t wc[2], chain, tc[4], D, npg;
  std::memcpy(&codec, blob, 4);
  std::memcpy(wc, blob + 4, 4);  // words of the K and V streams
  std::memcpy(&chain, blob + 8, 2);
  std::memcpy(tc, blob + 12, 8);
  std::memcpy(&D, blob + 20, 2);
  std::memcpy(&npg, blob + 22, 2);
  std::memcpy(k_scale, blob + 32, 16);
  std::memcpy(v_scale, blob + 48, 16);
  for (int g = 0; g < 4; ++g) token_count[g] = tc[g];
  *chain_out = 1;
  const uint32_t nq = D / 4, page = 16u * D;
  // lane L (page L/16, t = L%16), quad q, position i -> flat index into [4][16][D]
  auto where = [&](bool is_v, uint32_t L, uint32_t q, uint32_t i) -> size_t {
    const uint32_t G = L / 16, t = L % 16;
    if (!is_v) return (size_t)G * page + (size_t)t * D + 4 * q + i;
    const uint32_t per = D / 16;
    return (size_t)G * page + (size_t)(4 * (q / per) + i) * D + t + 16 * (q % per);
  };
  if (codec == 1) {  // INT8: word (q*64 + L) = 4 bytes of quad q of lane L
    for (int s = 0; s < 2; ++s) {
      const uint8_t *b = blob + 64 + (size_t)s * 64 * D;
      uint8_t *out = s ? v_sym : k_sym;
      for (uint32_t q = 0; q < nq; ++q)
        for (uint32_t L = 0; L < 64; ++L)
          for (uint32_t i = 0; i < 4; ++i) out[where(s == 1, L, q, i)] = b[(q * 64 + L) * 4 + i];
    }
    return 0;
  }
  if (codec != 2 || D == 0 || D % 32 != 0) return -1;
  *chain_out = chain;
  static const uint32_t frame[8] = {0, 4, 2, 6, 1, 5, 3, 7};
  static const uint32_t nword[8] = {0, 0, 1, 1, 3, 3, 4, 4};  // N0 N1 C0 N2 N3 C1 S
  const uint32_t steps = D / 8, raw_words = 7 * (D / 32) * 64;
  const uint8_t *p = blob + 64;
  if (chain) {
    std::memcpy(states_io, p, 2 * 64 * 4);
    p += 2 * 64 * 4;
  }
  const uint32_t *raw = reinterpret_cast<const uint32_t *>(p);  // K raw words, then V
  const uint16_t *words = reinterpret_cast<const uint16_t *>(p + 2 * (size_t)raw_words * 4);
  auto bit = [](uint32_t w, uint32_t pos) { return (w >> (pos % 32)) & 1u; };
  for (int s = 0; s < 2; ++s) {
    const uint8_t *tab = tables + (size_t)(2 * head + s) * 16384;
    const uint16_t *w = words + (s ? wc[0] : 0);
    const uint32_t *rw = raw + (size_t)s * raw_words;
    uint32_t *x = states_io + 64 * s, cur = 0;
    uint8_t *out = s ? v_sym : k_sym;
    for (uint32_t st = 0; st < steps; ++st) {
      uint32_t j[64];
      for (uint32_t L = 0; L < 64; ++L) {  // all lanes decode step st
        uint32_t lo, hi;
        std::memcpy(&lo, tab + 8 * (x[L] & 2047u), 4);
        std::memcpy(&hi, tab + 8 * (x[L] & 2047u) + 4, 4);
        const uint32_t f = lo & 2047u, c = (lo >> 11) & 2047u;
        j[L] = (lo >> 22) & 255u;
        uint32_t spread = 0;  // the format's spread word of j
        for (uint32_t i = 0; i < 4; ++i)
          spread |= ((j[L] >> i) & 1u) << (8 * i + 6) | ((j[L] >> (4 + i)) & 1u) << ((8 * i + 10) % 32);
        if (hi != spread) return -1;
        x[L] = f * (x[L] >> 11) + c;
      }
      for (uint32_t L = 0; L < 64; ++L)  // renormalisation reads in ascending lane order
        if (x[L] < 65536u) {
          if (cur >= wc[s]) return -1;
          x[L] = (x[L] << 16) | w[cur++];
        }
      for (uint32_t h = 0; h < 2; ++h) {
        const uint32_t q = 2 * st + h, k = q % 8, sg = q / 8, r = frame[k];
        for (uint32_t L = 0; L < 64; ++L) {
          const uint32_t N = rw[(7 * sg + nword[k]) * 64 + L], Cw = rw[(7 * sg + (k < 4 ? 2 : 5)) * 64 + L],
                         S = rw[(7 * sg + 6) * 64 + L];
          for (uint32_t i = 0; i < 4; ++i) {
            uint32_t mag = 0;
            for (uint32_t f = 0; f < 4; ++f) mag |= bit(N, 8 * i + r + f) << f;
            for (uint32_t f = 0; f < 2; ++f) mag |= bit(Cw, 8 * i + r + 4 + f) << (4 + f);
            mag |= ((j[L] >> (4 * h + i)) & 1u) << 6;
            const int v = bit(S, 8 * i + r + 7) ? -(int)mag : (int)mag;
            out[where(s == 1, L, q, i)] = (uint8_t)(v + 128);
          }
        }
      }
    }
    if (cur != wc[s]) return -1;
  }
  return 0;
}

// Batched pool attention on the host (the CPU baseline of the batched decode, and a checker at full size): for
// every (sequence, KV head) of the first nseq sequences, decode its groups in token order with or_kv_decode_group
// (chain states carried from a group to the one that continues it), dequantise (q - 128) * scale, and compute the
// float64 softmax attention of the sequence's one query row for the gqa query heads of that KV head over the tokens
// [0, min(seq_tokens, query_pos + 1)). Layouts as cf_kv_batched_desc (group_offsets [nseq][kv_heads][max_groups]
// in 16-byte units, queries / out [nseq][q_heads][D]). Parallel over (sequence, head) on `threads` OpenMP threads
// (0 = all). Returns the number of (sequence, head) units whose blobs failed to decode (their rows are NaN).
int or_kv_pool_attention(const uint8_t *pool, const uint32_t *group_offsets, uint32_t max_groups,
                         const uint32_t *seq_tokens, const uint32_t *query_pos, const uint8_t *tables,
                         const float *queries, uint32_t nseq, uint32_t kv_heads, uint32_t q_heads, uint32_t D,
                         float softmax_scale, float *out, int threads) {
  const uint32_t gqa = q_heads / kv_heads;
  int bad = 0;
#pragma omp parallel for schedule(dynamic) reduction(+ : bad) num_threads(threads > 0 ? threads : omp_get_max_threads())
  for (int64_t u = 0; u < (int64_t)nseq * kv_heads; ++u) {
    const uint32_t s = (uint32_t)(u / kv_heads), h = (uint32_t)(u % kv_heads);
    const uint32_t vis = std::min(seq_tokens[s], query_pos[s] + 1);
    const uint32_t ng = (vis + 63) / 64;
    std::vector<double> Kd((size_t)ng * 64 * D), Vd((size_t)ng * 64 * D);
    std::vector<uint8_t> ks((size_t)4 * 16 * D), vs((size_t)4 * 16 * D);
    float ksc[4], vsc[4];
    uint32_t tc[4], st[128] = {0}, chain = 0;
    bool ok = true;
    for (uint32_t g = 0; g < ng && ok; ++g) {
      const uint8_t *blob = pool + (size_t)group_offsets[((size_t)s * kv_heads + h) * max_groups + g] * 16;
      ok = or_kv_decode_group(blob, tables, h, ks.data(), vs.data(), ksc, vsc, tc, st, &chain) == 0;
      for (uint32_t G = 0; G < 4; ++G)
        for (uint32_t t = 0; t < 16; ++t)
          for (uint32_t d = 0; d < D; ++d) {
            const size_t src = ((size_t)G * 16 + t) * D + d, dst = ((size_t)g * 64 + G * 16 + t) * D + d;
            Kd[dst] = ((double)ks[src] - 128.0) * ksc[G];
            Vd[dst] = ((double)vs[src] - 128.0) * vsc[G];
          }
    }
    if (!ok) ++bad;
    std::vector<double> p(vis);
    for (uint32_t i = 0; i < gqa; ++i) {
      const uint32_t qh = h * gqa + i;
      const float *q = queries + ((size_t)s * q_heads + qh) * D;
      float *o = out + ((size_t)s * q_heads + qh) * D;
      if (!ok) {
        for (uint32_t d = 0; d < D; ++d) o[d] = NAN;
        continue;
      }
      double m = -INFINITY;
      for (uint32_t t = 0; t < vis; ++t) {
        double acc = 0;
        for (uint32_t d = 0; d < D; ++d) acc += (double)q[d] * Kd[(size_t)t * D + d];
        p[t] = acc * softmax_scale;
        m = std::max(m, p[t]);
      }
      double l = 0;
      for (uint32_t t = 0; t < vis; ++t) l += (p[t] = std::exp(p[t] - m));
      for (uint32_t d = 0; d < D; ++d) {
        double acc = 0;
        for (uint32_t t = 0; t < vis; ++t) acc += p[t] * Vd[(size_t)t * D + d];
        o[d] = vis ? (float)(acc / l) : 0.0f;
      }
    }
  }
  return bad;
}

// per-page-per-head absmax int8 quantiser of the benchmark configuration (scale = max|x|/127, 0 -> 1;
// sym = clamp(lrint(x / scale), -128, 127) + 128) — the kv_gpu_fixture convention with one scale per page.
void or_kv_quantize_page_absmax(const float *x, uint32_t n, uint8_t *sym, float *scale) {
  float m = 0.0f;
  for (uint32_t i = 0; i < n; ++i) m = std::max(m, std::fabs(x[i]));
  *scale = m == 0.0f ? 1.0f : m / 127.0f;
  for (uint32_t i = 0; i < n; ++i) sym[i] = (uint8_t)(std::clamp(std::lrint(x[i] / *scale), -128L, 127L) + 128);
}

}  // extern "C"
