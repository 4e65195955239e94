// kv_codec.cpp — host-side KV page-group encoder for the additive codecs of kv_codec_ext.h (INT8, RANS_HYBRID).
//
// The quantiser follows the convention of the reference's page encoder (reference
// src/runtime/kv_gpu_fixture.cpp:12-16: symmetric, qmax = 127, zero point 128, lrint of the IEEE fp32 quotient,
// clamp to [-(qmax+1), qmax]); the scale granularity is one absmax scale per page and head for K and for V (the
// benchmark configuration's "per-page-per-head absmax"). The entropy coder is this project's own design (the
// reference has no rANS KV codec): joint 2-bit high parts coded with interleaved rANS (M = 2^11, 16-bit
// renormalisation; two chains of 64 lane states per stream), 6-bit low parts stored raw and bit-sliced. The byte
// format is specified in include/chromofold/kv_codec_ext.h.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "chromofold/kv_codec_ext.h"

namespace {

constexpr uint32_t kLanes = CF_KV_RANS_LANES;  // 64
constexpr uint32_t kPageTok = CF_KV_PAGE_TOKENS;
constexpr uint32_t kProbBits = CF_KV_RANS_PROB_BITS;
constexpr uint32_t kM = 1u << kProbBits;
constexpr uint32_t kL = 1u << 16;
constexpr uint32_t kHeader = 64;

// symbols of one page [16, D] token-major (absent tokens 128) and its scale
// reference src/runtime/kv_gpu_fixture.cpp:12-16 (quantize) with one scale per page/head
float quantize_page(const float *x, uint32_t tokens, uint32_t dim, uint8_t *sym) {
  float m = 0.0f;
  for (uint64_t i = 0; i < static_cast<uint64_t>(tokens) * dim; ++i) m = std::max(m, std::fabs(x[i]));
  const float scale = m == 0.0f ? 1.0f : m / 127.0f;
  std::fill(sym, sym + static_cast<size_t>(kPageTok) * dim, uint8_t(128));
  for (uint32_t t = 0; t < tokens; ++t)
    for (uint32_t d = 0; d < dim; ++d) {
      const long r = std::lrint(x[static_cast<size_t>(t) * dim + d] / scale);
      sym[static_cast<size_t>(t) * dim + d] = static_cast<uint8_t>(std::clamp(r, -128L, 127L) + 128);
    }
  return scale;
}

// symbol of lane L (page L/16, t = L%16), quad q, position i in the lane order of kv_codec_ext.h
// page_sym: 4 pages of [16, D] symbols
inline uint8_t lane_sym(const uint8_t *page_sym, uint32_t dim, bool is_v, uint32_t L, uint32_t q, uint32_t i) {
  const uint8_t *sym = page_sym + static_cast<size_t>(L / 16) * kPageTok * dim;
  const uint32_t t = L % 16;
  if (!is_v) return sym[static_cast<size_t>(t) * dim + 4 * q + i];
  const uint32_t per_tq = dim / 16;
  const uint32_t tq = q / per_tq, di = q % per_tq;
  return sym[static_cast<size_t>(4 * tq + i) * dim + t + 16 * di];
}

struct Table {
  uint32_t freq[256], cum[256];
};

bool load_table(const uint8_t *blob, Table *tb) {
  // recover freq/cum from the slot entries (lo = f | c << 11 | j << 22)
  std::fill(tb->freq, tb->freq + 256, 0u);
  std::fill(tb->cum, tb->cum + 256, 0u);
  for (uint32_t s = 0; s < kM; ++s) {
    uint32_t lo;
    std::memcpy(&lo, blob + 8 * s, 4);
    const uint32_t f = lo & (kM - 1), c = (lo >> 11) & (kM - 1), j = (lo >> 22) & 255;
    if (c == 0) {
      tb->freq[j] = f;
      tb->cum[j] = s;
    }
  }
  uint32_t total = 0;
  for (uint32_t j = 0; j < 256; ++j) {
    if (tb->freq[j] == 0) return false;
    total += tb->freq[j];
  }
  return total == kM;
}

uint32_t spread_highs(uint32_t j) {
  uint32_t v = 0;
  for (uint32_t i = 0; i < 4; ++i) v |= ((j >> (2 * i)) & 3u) << (8 * i + 6);
  return v;
}

// Interleaved rANS encode of one chain: the quads q = chain, chain + 2, ... of joint[L][q] (64 lanes x nq quads).
// Writes the 64 states and the chain's word stream in decode order (decoder: the chain's quads ascending, all lanes
// decode, renorm reads in ascending lane order).
void rans_encode(const Table &tb, const std::vector<uint8_t> &joint, uint32_t nq, uint32_t chain, uint32_t *states,
                 std::vector<uint16_t> *words) {
  uint32_t x[kLanes];
  for (uint32_t t = 0; t < kLanes; ++t) x[t] = kL;
  std::vector<uint16_t> emitted;
  emitted.reserve(static_cast<size_t>(nq) * kLanes / 2);
  for (int64_t q = static_cast<int64_t>(nq) - 2 + chain; q >= 0; q -= 2) {
    for (int t = static_cast<int>(kLanes) - 1; t >= 0; --t) {
      const uint32_t s = joint[static_cast<size_t>(t) * nq + q];
      const uint32_t f = tb.freq[s];
      const uint64_t x_max = static_cast<uint64_t>((kL >> kProbBits) << 16) * f;
      uint32_t v = x[t];
      if (v >= x_max) {
        emitted.push_back(static_cast<uint16_t>(v & 0xFFFFu));
        v >>= 16;
      }
      x[t] = ((v / f) << kProbBits) + (v % f) + tb.cum[s];
    }
  }
  for (uint32_t t = 0; t < kLanes; ++t) states[t] = x[t];
  words->assign(emitted.rbegin(), emitted.rend());
}

// bit-sliced low parts of one lane: groups of 16 values -> N0, N1, C
void pack_lows(const uint8_t *page_sym, uint32_t dim, bool is_v, uint32_t L, uint32_t *lows) {
  const uint32_t groups = dim / 16;
  for (uint32_t g = 0; g < groups; ++g) {
    uint32_t n[2] = {0, 0}, c = 0;
    for (uint32_t qd = 0; qd < 4; ++qd)
      for (uint32_t i = 0; i < 4; ++i) {
        const uint32_t l = lane_sym(page_sym, dim, is_v, L, 4 * g + qd, i) & 63u;
        n[qd >> 1] |= (l & 15u) << (8 * i + 4 * (qd & 1));
        c |= (l >> 4) << (8 * i + 2 * qd);
      }
    lows[(g * 3 + 0) * kLanes + L] = n[0];
    lows[(g * 3 + 1) * kLanes + L] = n[1];
    lows[(g * 3 + 2) * kLanes + L] = c;
  }
}

uint64_t align16(uint64_t v) { return (v + 15) & ~uint64_t(15); }

bool dim_ok(uint32_t d) { return d != 0 && d % 16 == 0 && d <= CF_KV_MAX_HEAD_DIM; }

}  // namespace

extern "C" uint64_t cf_kv_group_blob_max_bytes(uint32_t codec, uint32_t head_dim) {
  if (!dim_ok(head_dim)) return 0;
  if (codec == CF_KV_CODEC_INT8) return kHeader + 2ull * CF_KV_GROUP_PAGES * kPageTok * head_dim;
  if (codec != CF_KV_CODEC_RANS_HYBRID) return 0;
  // header, 4 x 64 states, K and V low parts, at most CF_KV_RANS_MAX_GROUP_WORDS words (above that the group is
  // stored raw, which is smaller than this bound)
  const uint64_t lows = 3ull * (head_dim / 16) * kLanes * 4;
  return align16(kHeader + 4 * kLanes * 4 + 2 * lows + 2ull * CF_KV_RANS_MAX_GROUP_WORDS);
}

extern "C" cf_status cf_kv_rans_page_histogram(const float *values, uint32_t token_count, uint32_t head_dim,
                                               uint64_t *hist256) {
  if (!values || !hist256 || token_count == 0 || token_count > kPageTok || !dim_ok(head_dim))
    return CF_ERR_INVALID_ARGUMENT;
  std::vector<uint8_t> sym(static_cast<size_t>(kPageTok) * head_dim);
  quantize_page(values, token_count, head_dim, sym.data());
  for (uint32_t t = 0; t < kPageTok; ++t)
    for (uint32_t q = 0; q < head_dim / 4; ++q) {
      uint32_t j = 0;
      for (uint32_t i = 0; i < 4; ++i)
        j |= static_cast<uint32_t>(sym[static_cast<size_t>(t) * head_dim + 4 * q + i] >> 6) << (2 * i);
      hist256[j]++;
    }
  return CF_OK;
}

extern "C" cf_status cf_kv_rans_build_table(const uint64_t *hist, uint8_t *out) {
  if (!hist || !out) return CF_ERR_INVALID_ARGUMENT;
  // Normalise to M slots: f = max(1, floor(p * M)) (every symbol stays codable), then hand out / take back the
  // remainder one slot at a time where it costs least: add to the symbol with the largest count per slot, remove
  // from the symbol with the smallest count per slot among those above 1. Deterministic (ties -> lowest j).
  uint64_t total = 0;
  for (int j = 0; j < 256; ++j) total += hist[j];
  uint32_t f[256];
  int64_t used = 0;
  for (int j = 0; j < 256; ++j) {
    f[j] = total ? static_cast<uint32_t>(std::max<uint64_t>(1, hist[j] * kM / total)) : kM / 256;
    used += f[j];
  }
  while (used < static_cast<int64_t>(kM)) {
    int best = 0;
    for (int j = 1; j < 256; ++j)
      if (hist[j] * f[best] > hist[best] * f[j]) best = j;  // hist[j]/f[j] > hist[best]/f[best]
    f[best]++;
    used++;
  }
  while (used > static_cast<int64_t>(kM)) {
    int best = -1;
    for (int j = 0; j < 256; ++j)
      if (f[j] > 1 && (best < 0 || hist[j] * f[best] < hist[best] * f[j])) best = j;
    f[best]--;
    used--;
  }
  uint32_t cum = 0;
  for (uint32_t j = 0; j < 256; ++j) {
    for (uint32_t c = 0; c < f[j]; ++c) {
      const uint32_t slot = cum + c;
      const uint32_t lo = f[j] | (c << 11) | (j << 22);
      const uint32_t hi = spread_highs(j);
      std::memcpy(out + 8 * slot, &lo, 4);
      std::memcpy(out + 8 * slot + 4, &hi, 4);
    }
    cum += f[j];
  }
  return CF_OK;
}

extern "C" cf_status cf_kv_encode_group(uint32_t codec, const float *keys, const float *values, uint32_t page_count,
                                        const uint32_t *token_counts, uint32_t head_dim, const uint8_t *k_table,
                                        const uint8_t *v_table, uint32_t k_table_index, uint32_t v_table_index,
                                        uint8_t *blob, uint64_t capacity, uint64_t *blob_bytes) {
  if (!keys || !values || !blob || !blob_bytes || page_count == 0 || page_count > CF_KV_GROUP_PAGES ||
      !dim_ok(head_dim))
    return CF_ERR_INVALID_ARGUMENT;
  if (codec != CF_KV_CODEC_INT8 && codec != CF_KV_CODEC_RANS_HYBRID) return CF_ERR_UNSUPPORTED;
  if (codec == CF_KV_CODEC_RANS_HYBRID && (!k_table || !v_table)) return CF_ERR_INVALID_ARGUMENT;
  if (capacity < cf_kv_group_blob_max_bytes(codec, head_dim)) return CF_ERR_INVALID_ARGUMENT;
  const size_t page_vals = static_cast<size_t>(kPageTok) * head_dim;
  cf_kv_group_header h{};
  h.codec = codec;
  h.head_dim = static_cast<uint16_t>(head_dim);
  h.page_count = static_cast<uint16_t>(page_count);
  h.k_table = k_table_index;
  h.v_table = v_table_index;
  std::vector<uint8_t> ks(CF_KV_GROUP_PAGES * page_vals), vs(CF_KV_GROUP_PAGES * page_vals);
  for (uint32_t g = 0; g < CF_KV_GROUP_PAGES; ++g) {
    const uint32_t tc = g < page_count ? (token_counts ? token_counts[g] : kPageTok) : 0;
    if (g < page_count && (tc == 0 || tc > kPageTok)) return CF_ERR_INVALID_ARGUMENT;
    h.token_count[g] = static_cast<uint16_t>(tc);
    if (tc) {
      h.k_scale[g] = quantize_page(keys + g * page_vals, tc, head_dim, ks.data() + g * page_vals);
      h.v_scale[g] = quantize_page(values + g * page_vals, tc, head_dim, vs.data() + g * page_vals);
    } else {
      std::fill(ks.begin() + g * page_vals, ks.begin() + (g + 1) * page_vals, uint8_t(128));
      std::fill(vs.begin() + g * page_vals, vs.begin() + (g + 1) * page_vals, uint8_t(128));
      h.k_scale[g] = h.v_scale[g] = 1.0f;
    }
  }
  const uint32_t nq = head_dim / 4;

  if (codec == CF_KV_CODEC_INT8) {
    uint8_t *p = blob + kHeader;
    for (int s = 0; s < 2; ++s)
      for (uint32_t q = 0; q < nq; ++q)
        for (uint32_t L = 0; L < kLanes; ++L)
          for (uint32_t i = 0; i < 4; ++i) *p++ = lane_sym(s ? vs.data() : ks.data(), head_dim, s == 1, L, q, i);
    std::memcpy(blob, &h, sizeof h);
    *blob_bytes = static_cast<uint64_t>(p - blob);
    return CF_OK;
  }

  Table tk, tv;
  if (!load_table(k_table, &tk) || !load_table(v_table, &tv)) return CF_ERR_INVALID_ARGUMENT;
  uint32_t states[4][kLanes];  // K A, K B, V A, V B
  std::vector<uint16_t> words[4];
  const uint32_t nlow = 3 * (head_dim / 16) * kLanes;
  std::vector<uint32_t> lows(2 * static_cast<size_t>(nlow), 0u);
  for (int s = 0; s < 2; ++s) {
    const uint8_t *sym = s ? vs.data() : ks.data();
    std::vector<uint8_t> joint(static_cast<size_t>(kLanes) * nq);
    for (uint32_t L = 0; L < kLanes; ++L) {
      for (uint32_t q = 0; q < nq; ++q) {
        uint32_t j = 0;
        for (uint32_t i = 0; i < 4; ++i)
          j |= static_cast<uint32_t>(lane_sym(sym, head_dim, s == 1, L, q, i) >> 6) << (2 * i);
        joint[static_cast<size_t>(L) * nq + q] = static_cast<uint8_t>(j);
      }
      pack_lows(sym, head_dim, s == 1, L, lows.data() + s * nlow);
    }
    for (uint32_t chain = 0; chain < 2; ++chain)
      rans_encode(s ? tv : tk, joint, nq, chain, states[2 * s + chain], &words[2 * s + chain]);
  }
  size_t total_words = 0;
  for (const auto &w : words) total_words += w.size();
  if (total_words > CF_KV_RANS_MAX_GROUP_WORDS)  // raw fallback (see kv_codec_ext.h)
    return cf_kv_encode_group(CF_KV_CODEC_INT8, keys, values, page_count, token_counts, head_dim, nullptr, nullptr,
                              k_table_index, v_table_index, blob, capacity, blob_bytes);
  for (int c = 0; c < 4; ++c) h.word_count[c] = static_cast<uint16_t>(words[c].size());
  uint64_t at = 0;
  std::memcpy(blob + at, &h, sizeof h);
  at += kHeader;
  std::memcpy(blob + at, states, sizeof states);
  at += sizeof states;
  std::memcpy(blob + at, lows.data(), lows.size() * 4);
  at += lows.size() * 4;
  for (int c = 0; c < 4; ++c) {
    std::memcpy(blob + at, words[c].data(), words[c].size() * 2);
    at += words[c].size() * 2;
  }
  const uint64_t end = align16(at);
  std::memset(blob + at, 0, end - at);
  *blob_bytes = end;
  return CF_OK;
}

extern "C" cf_status cf_kv_encode_groups(uint32_t codec, const float *keys, const float *values, uint64_t ngroups,
                                         const uint64_t *first_page, const uint32_t *page_counts,
                                         const uint32_t *token_counts, uint32_t head_dim, const uint8_t *tables,
                                         const uint32_t *heads, uint8_t *pool, uint64_t pool_capacity,
                                         uint64_t pool_at, uint32_t *offsets_out, uint64_t *pool_end,
                                         uint32_t threads) {
  if (!keys || !values || !first_page || !page_counts || !pool || !offsets_out || !pool_end || pool_at % 16 != 0)
    return CF_ERR_INVALID_ARGUMENT;
  if (codec == CF_KV_CODEC_RANS_HYBRID && !tables) return CF_ERR_INVALID_ARGUMENT;
  const uint64_t cap = cf_kv_group_blob_max_bytes(codec, head_dim);
  if (cap == 0) return CF_ERR_UNSUPPORTED;
  const uint64_t page_vals = static_cast<uint64_t>(kPageTok) * head_dim;
  std::vector<uint8_t> tmp(ngroups * cap);
  std::vector<uint64_t> sizes(ngroups, 0);
  std::atomic<int> status{CF_OK};
  std::atomic<uint64_t> next{0};
  if (threads == 0) threads = std::max(1u, std::thread::hardware_concurrency());
  auto work = [&]() {
    for (;;) {
      const uint64_t g = next.fetch_add(1);
      if (g >= ngroups) return;
      const uint64_t p0 = first_page[g];
      const uint32_t h = heads ? heads[g] : 0;
      const uint8_t *kt = tables ? tables + static_cast<uint64_t>(2 * h) * CF_KV_RANS_TABLE_BYTES : nullptr;
      const uint8_t *vt = tables ? kt + CF_KV_RANS_TABLE_BYTES : nullptr;
      uint64_t sz = 0;
      const cf_status st = cf_kv_encode_group(codec, keys + p0 * page_vals, values + p0 * page_vals, page_counts[g],
                                              token_counts ? token_counts + p0 : nullptr, head_dim, kt, vt, 2 * h,
                                              2 * h + 1, tmp.data() + g * cap, cap, &sz);
      if (st != CF_OK) status = st;
      sizes[g] = sz;
    }
  };
  std::vector<std::thread> workers;
  for (uint32_t i = 1; i < threads; ++i) workers.emplace_back(work);
  work();
  for (auto &th : workers) th.join();
  if (status != CF_OK) return static_cast<cf_status>(status.load());
  uint64_t at = pool_at;
  for (uint64_t g = 0; g < ngroups; ++g) {
    if (at + sizes[g] > pool_capacity || at / 16 > 0xFFFFFFFFull) return CF_ERR_INVALID_ARGUMENT;
    std::memcpy(pool + at, tmp.data() + g * cap, sizes[g]);
    offsets_out[g] = static_cast<uint32_t>(at / 16);
    at += sizes[g];
  }
  *pool_end = at;
  return CF_OK;
}
