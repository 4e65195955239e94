// kv_codec.cpp — host-side KV page encoder for the additive codecs of kv_codec_ext.h (INT8, RANS_HYBRID).
//
// The quantiser follows the convention of the reference's page encoder (reference
// src/runtime/kv_gpu_fixture.cpp:12-16: symmetric, qmax = 127, zero point 128, lrint of the IEEE fp32 quotient,
// clamp to [-(qmax+1), qmax]); the scale granularity is one absmax scale per page and head for K and for V (the
// benchmark configuration's "per-page-per-head absmax"). The entropy coder is this project's own design (the
// reference has no rANS KV codec): joint 2-bit high parts coded with 16-lane interleaved rANS (M = 2^11,
// 16-bit renormalisation), 6-bit low parts stored raw and bit-sliced. The byte format is specified in
// include/chromofold/kv_codec_ext.h.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#include "chromofold/kv_codec_ext.h"

namespace {

constexpr uint32_t kLanes = CF_KV_RANS_LANES;
constexpr uint32_t kProbBits = CF_KV_RANS_PROB_BITS;
constexpr uint32_t kM = 1u << kProbBits;
constexpr uint32_t kL = 1u << 16;

struct Quant {
  float scale;
  std::vector<uint8_t> sym;  // [16 tokens, D], padded tokens hold 128
};

// reference src/runtime/kv_gpu_fixture.cpp:12-16 (quantize) with one scale per page/head
Quant quantize_page(const float *x, uint32_t tokens, uint32_t dim) {
  float m = 0.0f;
  for (uint64_t i = 0; i < static_cast<uint64_t>(tokens) * dim; ++i) m = std::max(m, std::fabs(x[i]));
  Quant q;
  q.scale = m == 0.0f ? 1.0f : m / 127.0f;
  q.sym.assign(static_cast<size_t>(CF_KV_PAGE_TOKENS) * dim, 128);
  for (uint32_t t = 0; t < tokens; ++t)
    for (uint32_t d = 0; d < dim; ++d) {
      const long r = std::lrint(x[static_cast<size_t>(t) * dim + d] / q.scale);
      q.sym[static_cast<size_t>(t) * dim + d] = static_cast<uint8_t>(std::clamp(r, -128L, 127L) + 128);
    }
  return q;
}

// symbol of lane t, quad q, position i in the lane order of kv_codec_ext.h
inline uint8_t lane_sym(const std::vector<uint8_t> &sym, uint32_t dim, bool is_v, uint32_t t, uint32_t q,
                        uint32_t i) {
  if (!is_v) return sym[static_cast<size_t>(t) * dim + 4 * q + i];
  const uint32_t per_tq = dim / 16;
  const uint32_t tq = q / per_tq, di = q % per_tq;
  return sym[static_cast<size_t>(4 * tq + i) * dim + t + 16 * di];
}

struct Table {
  uint32_t freq[256], cum[256];
};

bool load_table(const uint8_t *blob, Table *tb) {
  // recover freq/cum from the slot entries (lo = (f-1) | c_slot << 11 | j << 22)
  std::fill(tb->freq, tb->freq + 256, 0u);
  std::fill(tb->cum, tb->cum + 256, 0u);
  for (uint32_t s = 0; s < kM; ++s) {
    uint32_t lo;
    std::memcpy(&lo, blob + 8 * s, 4);
    const uint32_t f = (lo & (kM - 1)) + 1, cs = (lo >> 11) & (kM - 1), j = (lo >> 22) & 255;
    if (cs == 0) {
      tb->freq[j] = f;
      tb->cum[j] = s;
    }
  }
  uint32_t total = 0;
  for (uint32_t j = 0; j < 256; ++j) total += tb->freq[j];
  return total == kM;
}

uint32_t spread_highs(uint32_t j) {
  uint32_t v = 0;
  for (uint32_t i = 0; i < 4; ++i) v |= ((j >> (2 * i)) & 3u) << (8 * i + 6);
  return v;
}

// Interleaved rANS encode of one stream: sym[t][q] for 16 lanes x nq quads. Writes states and the shared word
// stream in decode order. Decoder (kernel): step q = 0..nq-1, all lanes decode, renorm reads in lane order.
void rans_encode(const Table &tb, const std::vector<uint8_t> &joint, uint32_t nq, uint32_t *states,
                 std::vector<uint16_t> *words) {
  uint32_t x[kLanes];
  for (uint32_t t = 0; t < kLanes; ++t) x[t] = kL;
  std::vector<uint16_t> emitted;
  emitted.reserve(nq * kLanes);
  for (int64_t q = static_cast<int64_t>(nq) - 1; q >= 0; --q) {
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
void pack_lows(const std::vector<uint8_t> &sym, uint32_t dim, bool is_v, uint32_t t, uint32_t *lows) {
  const uint32_t groups = dim / 16;
  for (uint32_t g = 0; g < groups; ++g) {
    uint32_t n[2] = {0, 0}, c = 0;
    for (uint32_t qd = 0; qd < 4; ++qd)
      for (uint32_t i = 0; i < 4; ++i) {
        const uint32_t l = lane_sym(sym, dim, is_v, t, 4 * g + qd, i) & 63u;
        n[qd >> 1] |= (l & 15u) << (8 * i + 4 * (qd & 1));
        c |= (l >> 4) << (8 * i + 2 * qd);
      }
    lows[(g * 3 + 0) * kLanes + t] = n[0];
    lows[(g * 3 + 1) * kLanes + t] = n[1];
    lows[(g * 3 + 2) * kLanes + t] = c;
  }
}

uint64_t align16(uint64_t v) { return (v + 15) & ~uint64_t(15); }

}  // namespace

extern "C" uint64_t cf_kv_page_blob_max_bytes(uint32_t codec, uint32_t head_dim) {
  if (head_dim == 0 || head_dim % 16 != 0 || head_dim > CF_KV_MAX_HEAD_DIM) return 0;
  if (codec == CF_KV_CODEC_INT8) return 32 + 2ull * CF_KV_PAGE_TOKENS * head_dim;
  if (codec != CF_KV_CODEC_RANS_HYBRID) return 0;
  const uint64_t lows = 3ull * (head_dim / 16) * kLanes * 4;
  const uint64_t max_words = (static_cast<uint64_t>(head_dim / 4) * kLanes * kProbBits + 15) / 16 + kLanes;
  return align16(160 + 2 * lows + 2 * 2 * max_words);
}

extern "C" cf_status cf_kv_rans_page_histogram(const float *values, uint32_t token_count, uint32_t head_dim,
                                               uint64_t *hist256) {
  if (!values || !hist256 || token_count == 0 || token_count > CF_KV_PAGE_TOKENS || head_dim == 0 ||
      head_dim % 16 != 0 || head_dim > CF_KV_MAX_HEAD_DIM)
    return CF_ERR_INVALID_ARGUMENT;
  const Quant q = quantize_page(values, token_count, head_dim);
  for (uint32_t t = 0; t < kLanes; ++t)
    for (uint32_t qq = 0; qq < head_dim / 4; ++qq) {
      uint32_t j = 0;
      for (uint32_t i = 0; i < 4; ++i) j |= static_cast<uint32_t>(lane_sym(q.sym, head_dim, false, t, qq, i) >> 6) << (2 * i);
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
      const uint32_t lo = (f[j] - 1) | (c << 11) | (j << 22);
      const uint32_t hi = spread_highs(j);
      std::memcpy(out + 8 * slot, &lo, 4);
      std::memcpy(out + 8 * slot + 4, &hi, 4);
    }
    cum += f[j];
  }
  return CF_OK;
}

extern "C" cf_status cf_kv_encode_page(uint32_t codec, const float *keys, const float *values,
                                       uint32_t token_count, uint32_t head_dim, const uint8_t *k_table,
                                       const uint8_t *v_table, uint32_t k_table_index, uint32_t v_table_index,
                                       uint8_t *blob, uint64_t capacity, uint64_t *blob_bytes) {
  if (!keys || !values || !blob || !blob_bytes || token_count == 0 || token_count > CF_KV_PAGE_TOKENS ||
      head_dim == 0 || head_dim % 16 != 0 || head_dim > CF_KV_MAX_HEAD_DIM)
    return CF_ERR_INVALID_ARGUMENT;
  if (codec != CF_KV_CODEC_INT8 && codec != CF_KV_CODEC_RANS_HYBRID) return CF_ERR_UNSUPPORTED;
  if (codec == CF_KV_CODEC_RANS_HYBRID && (!k_table || !v_table)) return CF_ERR_INVALID_ARGUMENT;
  if (capacity < cf_kv_page_blob_max_bytes(codec, head_dim)) return CF_ERR_INVALID_ARGUMENT;

  const Quant qk = quantize_page(keys, token_count, head_dim);
  const Quant qv = quantize_page(values, token_count, head_dim);
  const uint32_t nq = head_dim / 4;
  cf_kv_rans_page_header h{};
  h.codec = codec;
  h.k_scale = qk.scale;
  h.v_scale = qv.scale;
  h.token_count = static_cast<uint16_t>(token_count);
  h.head_dim = static_cast<uint16_t>(head_dim);
  h.k_table = k_table_index;
  h.v_table = v_table_index;

  if (codec == CF_KV_CODEC_INT8) {
    uint8_t *p = blob + 32;
    for (int s = 0; s < 2; ++s) {
      const Quant &qq = s ? qv : qk;
      for (uint32_t q = 0; q < nq; ++q)
        for (uint32_t t = 0; t < kLanes; ++t)
          for (uint32_t i = 0; i < 4; ++i) *p++ = lane_sym(qq.sym, head_dim, s == 1, t, q, i);
    }
    std::memcpy(blob, &h, sizeof h);
    *blob_bytes = static_cast<uint64_t>(p - blob);
    return CF_OK;
  }

  Table tk, tv;
  if (!load_table(k_table, &tk) || !load_table(v_table, &tv)) return CF_ERR_INVALID_ARGUMENT;
  uint32_t states[2][kLanes];
  std::vector<uint16_t> words[2];
  const uint32_t nlow = 3 * (head_dim / 16) * kLanes;
  std::vector<uint32_t> lows(2 * nlow, 0u);
  for (int s = 0; s < 2; ++s) {
    const Quant &qq = s ? qv : qk;
    std::vector<uint8_t> joint(static_cast<size_t>(kLanes) * nq);
    for (uint32_t t = 0; t < kLanes; ++t) {
      for (uint32_t q = 0; q < nq; ++q) {
        uint32_t j = 0;
        for (uint32_t i = 0; i < 4; ++i) j |= static_cast<uint32_t>(lane_sym(qq.sym, head_dim, s == 1, t, q, i) >> 6) << (2 * i);
        joint[static_cast<size_t>(t) * nq + q] = static_cast<uint8_t>(j);
      }
      pack_lows(qq.sym, head_dim, s == 1, t, lows.data() + s * nlow);
    }
    rans_encode(s ? tv : tk, joint, nq, states[s], &words[s]);
  }
  h.k_word_count = static_cast<uint16_t>(words[0].size());
  h.v_word_count = static_cast<uint16_t>(words[1].size());
  uint64_t at = 0;
  std::memcpy(blob + at, &h, sizeof h);
  at += 32;
  std::memcpy(blob + at, states, sizeof states);
  at += sizeof states;
  std::memcpy(blob + at, lows.data(), lows.size() * 4);
  at += lows.size() * 4;
  for (int s = 0; s < 2; ++s) {
    std::memcpy(blob + at, words[s].data(), words[s].size() * 2);
    at += words[s].size() * 2;
  }
  const uint64_t end = align16(at);
  std::memset(blob + at, 0, end - at);
  *blob_bytes = end;
  return CF_OK;
}

// ---------------------------------------------------------------------------------------------------------------
// Batch encoder: `npages` pages stored page-major ([npages][16][D] fp32 for K and V), encoded in parallel with
// std::thread workers and packed back to back (16-byte aligned) into `pool` starting at byte `pool_at`.
// token_counts may be NULL (all pages full); heads may be NULL (all pages use table pair 0).
// offsets_out[p] receives the byte offset of page p divided by 16.
#include <atomic>
#include <thread>

extern "C" cf_status cf_kv_encode_pages(uint32_t codec, const float *keys, const float *values, uint64_t npages,
                                        const uint32_t *token_counts, uint32_t head_dim, const uint8_t *tables,
                                        const uint32_t *heads, uint8_t *pool, uint64_t pool_capacity,
                                        uint64_t pool_at, uint32_t *offsets_out, uint64_t *pool_end,
                                        uint32_t threads) {
  if (!keys || !values || !pool || !offsets_out || !pool_end || pool_at % 16 != 0) return CF_ERR_INVALID_ARGUMENT;
  if (codec == CF_KV_CODEC_RANS_HYBRID && !tables) return CF_ERR_INVALID_ARGUMENT;
  const uint64_t cap = cf_kv_page_blob_max_bytes(codec, head_dim);
  if (cap == 0) return CF_ERR_UNSUPPORTED;
  const uint64_t page_vals = static_cast<uint64_t>(CF_KV_PAGE_TOKENS) * head_dim;
  std::vector<uint8_t> tmp(npages * cap);
  std::vector<uint64_t> sizes(npages, 0);
  std::atomic<int> status{CF_OK};
  std::atomic<uint64_t> next{0};
  if (threads == 0) threads = std::max(1u, std::thread::hardware_concurrency());
  auto work = [&]() {
    for (;;) {
      const uint64_t p = next.fetch_add(1);
      if (p >= npages) return;
      const uint32_t tc = token_counts ? token_counts[p] : CF_KV_PAGE_TOKENS;
      const uint32_t h = heads ? heads[p] : 0;
      const uint8_t *kt = tables ? tables + static_cast<uint64_t>(2 * h) * CF_KV_RANS_TABLE_BYTES : nullptr;
      const uint8_t *vt = tables ? kt + CF_KV_RANS_TABLE_BYTES : nullptr;
      uint64_t sz = 0;
      const cf_status st = cf_kv_encode_page(codec, keys + p * page_vals, values + p * page_vals, tc, head_dim, kt, vt,
                                             2 * h, 2 * h + 1, tmp.data() + p * cap, cap, &sz);
      if (st != CF_OK) status = st;
      sizes[p] = sz;
    }
  };
  std::vector<std::thread> pool_threads;
  for (uint32_t i = 1; i < threads; ++i) pool_threads.emplace_back(work);
  work();
  for (auto &th : pool_threads) th.join();
  if (status != CF_OK) return static_cast<cf_status>(status.load());
  uint64_t at = pool_at;
  for (uint64_t p = 0; p < npages; ++p) {
    if (at + sizes[p] > pool_capacity || at / 16 > 0xFFFFFFFFull) return CF_ERR_INVALID_ARGUMENT;
    std::memcpy(pool + at, tmp.data() + p * cap, sizes[p]);
    offsets_out[p] = static_cast<uint32_t>(at / 16);
    at += sizes[p];
  }
  *pool_end = at;
  return CF_OK;
}
