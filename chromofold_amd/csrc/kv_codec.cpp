// kv_codec.cpp — host-side KV page-group encoder for the additive codecs of kv_codec_ext.h (INT8, RANS_HYBRID).
//
// The quantiser follows the convention of the reference's page encoder (reference
// src/runtime/kv_gpu_fixture.cpp:12-16: symmetric, qmax = 127, zero point 128, lrint of the IEEE fp32 quotient,
// clamp to [-(qmax+1), qmax]); the scale granularity is one absmax scale per page and head for K and for V (the
// benchmark configuration's "per-page-per-head absmax"). The entropy coder is this project's own design (the
// reference has no rANS KV codec): sign-magnitude values whose "big" bits (|q| >= 64) are coded 8 at a time with
// interleaved rANS (M = 2^11, 16-bit renormalisation, one chain of 64 lane states per stream running across a pair
// of groups), signs and 6-bit low parts stored raw, bit-sliced in rotated frames. The byte format is specified in
// include/chromofold/kv_codec_ext.h.
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
constexpr uint32_t kStates = 2 * kLanes * 4;        // K and V lane states of a chain start
constexpr uint32_t kFrame[8] = {0, 4, 2, 6, 1, 5, 3, 7};  // frame of quad k of a sign group
constexpr uint32_t kNWord[8] = {0, 0, 1, 1, 3, 3, 4, 4};  // word holding quad k's nibbles (N0 N1 C0 N2 N3 C1 S)

// quantised values q of one page [16, D] token-major (absent tokens 0) and its scale
// reference src/runtime/kv_gpu_fixture.cpp:12-16 (quantize) with one scale per page/head
float quantize_page(const float *x, uint32_t tokens, uint32_t dim, int8_t *qv) {
  float m = 0.0f;
  for (uint64_t i = 0; i < static_cast<uint64_t>(tokens) * dim; ++i) m = std::max(m, std::fabs(x[i]));
  const float scale = m == 0.0f ? 1.0f : m / 127.0f;
  std::fill(qv, qv + static_cast<size_t>(kPageTok) * dim, int8_t(0));
  for (uint32_t t = 0; t < tokens; ++t)
    for (uint32_t d = 0; d < dim; ++d) {
      const long r = std::lrint(x[static_cast<size_t>(t) * dim + d] / scale);
      qv[static_cast<size_t>(t) * dim + d] = static_cast<int8_t>(std::clamp(r, -128L, 127L));
    }
  return scale;
}

// value of lane L (page L/16, t = L%16), quad q, position i in the lane order of kv_codec_ext.h
// page_q: 4 pages of [16, D] values
inline int8_t lane_q(const int8_t *page_q, uint32_t dim, bool is_v, uint32_t L, uint32_t q, uint32_t i) {
  const int8_t *sym = page_q + static_cast<size_t>(L / 16) * kPageTok * dim;
  const uint32_t t = L % 16;
  if (!is_v) return sym[static_cast<size_t>(t) * dim + 4 * q + i];
  const uint32_t per_tq = dim / 16;
  const uint32_t tq = q / per_tq, di = q % per_tq;
  return sym[static_cast<size_t>(4 * tq + i) * dim + t + 16 * di];
}

inline uint32_t big(int v) { return (v >= 64 || v <= -64) ? 1u : 0u; }

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

// big bits of a joint symbol in the frames (0, 4) of a quad pair
uint32_t spread_bigs(uint32_t j) {
  uint32_t v = 0;
  for (uint32_t i = 0; i < 4; ++i) {
    v |= ((j >> i) & 1u) << (8 * i + 6);
    v |= ((j >> (4 + i)) & 1u) << ((8 * i + 10) % 32);
  }
  return v;
}

// A group's coding inputs per stream (K, V): the joint symbols [L][step] and the raw words [(7 s + w) * 64 + L].
struct GroupCode {
  std::vector<uint8_t> joint[2];
  std::vector<uint32_t> raw[2];
  bool codable = true;  // false when a value is -128 (sign-magnitude cannot hold it: the group is stored INT8)
};

void build_code(const int8_t *kq, const int8_t *vq, uint32_t dim, GroupCode *gc) {
  const uint32_t steps = dim / 8, sgroups = dim / 32;
  for (int s = 0; s < 2; ++s) {
    const int8_t *qv = s ? vq : kq;
    gc->joint[s].assign(static_cast<size_t>(kLanes) * steps, 0);
    gc->raw[s].assign(static_cast<size_t>(7) * sgroups * kLanes, 0u);
    for (uint32_t L = 0; L < kLanes; ++L) {
      for (uint32_t p = 0; p < steps; ++p) {
        uint32_t j = 0;
        for (uint32_t h = 0; h < 2; ++h)
          for (uint32_t i = 0; i < 4; ++i) {
            const int v = lane_q(qv, dim, s == 1, L, 2 * p + h, i);
            if (v == -128) gc->codable = false;
            j |= big(v) << (4 * h + i);
          }
        gc->joint[s][static_cast<size_t>(L) * steps + p] = static_cast<uint8_t>(j);
      }
      for (uint32_t sg = 0; sg < sgroups; ++sg) {
        uint32_t w[7] = {0, 0, 0, 0, 0, 0, 0};
        for (uint32_t k = 0; k < 8; ++k) {
          const uint32_t r = kFrame[k];
          for (uint32_t i = 0; i < 4; ++i) {
            const int v = lane_q(qv, dim, s == 1, L, 8 * sg + k, i);
            const uint32_t a = static_cast<uint32_t>(v < 0 ? -v : v) & 127u;
            for (uint32_t f = 0; f < 4; ++f) w[kNWord[k]] |= ((a >> f) & 1u) << ((8 * i + r + f) % 32);
            for (uint32_t f = 0; f < 2; ++f) w[k < 4 ? 2 : 5] |= ((a >> (4 + f)) & 1u) << ((8 * i + r + 4 + f) % 32);
            w[6] |= (v < 0 ? 1u : 0u) << ((8 * i + r + 7) % 32);
          }
        }
        for (uint32_t x = 0; x < 7; ++x) gc->raw[s][(7 * sg + x) * kLanes + L] = w[x];
      }
    }
  }
}

// Interleaved rANS encode of one stream over a chain of `n` groups (decode order: group 0's steps ascending, then
// group 1's; in each step all lanes decode and renormalisation reads go in ascending lane order). Writes the 64
// initial decoder states and each group's word stream in decode order.
void rans_encode_chain(const Table &tb, const std::vector<uint8_t> *const *joint, uint32_t n, uint32_t steps,
                       uint32_t *states, std::vector<uint16_t> *words) {
  uint32_t x[kLanes];
  for (uint32_t t = 0; t < kLanes; ++t) x[t] = kL;
  for (int g = static_cast<int>(n) - 1; g >= 0; --g) {
    std::vector<uint16_t> emitted;
    emitted.reserve(static_cast<size_t>(steps) * kLanes / 2);
    for (int64_t p = static_cast<int64_t>(steps) - 1; p >= 0; --p)
      for (int t = static_cast<int>(kLanes) - 1; t >= 0; --t) {
        const uint32_t s = (*joint[g])[static_cast<size_t>(t) * steps + p];
        const uint32_t f = tb.freq[s];
        const uint64_t x_max = static_cast<uint64_t>((kL >> kProbBits) << 16) * f;
        uint32_t v = x[t];
        if (v >= x_max) {  // one word always suffices: v >> 16 < 2^16 <= x_max
          emitted.push_back(static_cast<uint16_t>(v & 0xFFFFu));
          v >>= 16;
        }
        x[t] = ((v / f) << kProbBits) + (v % f) + tb.cum[s];
      }
    words[g].assign(emitted.rbegin(), emitted.rend());
  }
  for (uint32_t t = 0; t < kLanes; ++t) states[t] = x[t];
}

uint64_t align16(uint64_t v) { return (v + 15) & ~uint64_t(15); }

bool dim_ok(uint32_t codec, uint32_t d) {
  if (d == 0 || d > CF_KV_MAX_HEAD_DIM) return false;
  return codec == CF_KV_CODEC_RANS_HYBRID ? d % 32 == 0 : d % 16 == 0;
}

// One group's quantised pages, header fields and the pointers it was quantised from.
struct GroupIn {
  cf_kv_group_header h{};
  std::vector<int8_t> kq, vq;
};

cf_status prepare_group(const float *keys, const float *values, uint32_t page_count, const uint32_t *token_counts,
                        uint32_t head_dim, uint32_t k_table_index, uint32_t v_table_index, GroupIn *g) {
  if (!keys || !values || page_count == 0 || page_count > CF_KV_GROUP_PAGES) return CF_ERR_INVALID_ARGUMENT;
  const size_t page_vals = static_cast<size_t>(kPageTok) * head_dim;
  g->h = cf_kv_group_header{};
  g->h.head_dim = static_cast<uint16_t>(head_dim);
  g->h.page_count = static_cast<uint16_t>(page_count);
  g->h.k_table = k_table_index;
  g->h.v_table = v_table_index;
  g->kq.assign(CF_KV_GROUP_PAGES * page_vals, 0);
  g->vq.assign(CF_KV_GROUP_PAGES * page_vals, 0);
  for (uint32_t p = 0; p < CF_KV_GROUP_PAGES; ++p) {
    const uint32_t tc = p < page_count ? (token_counts ? token_counts[p] : kPageTok) : 0;
    if (p < page_count && (tc == 0 || tc > kPageTok)) return CF_ERR_INVALID_ARGUMENT;
    g->h.token_count[p] = static_cast<uint16_t>(tc);
    if (tc) {
      g->h.k_scale[p] = quantize_page(keys + p * page_vals, tc, head_dim, g->kq.data() + p * page_vals);
      g->h.v_scale[p] = quantize_page(values + p * page_vals, tc, head_dim, g->vq.data() + p * page_vals);
    } else {
      g->h.k_scale[p] = g->h.v_scale[p] = 1.0f;
    }
  }
  return CF_OK;
}

uint64_t write_int8(GroupIn &g, uint8_t *blob) {
  const uint32_t dim = g.h.head_dim, nq = dim / 4;
  g.h.codec = CF_KV_CODEC_INT8;
  g.h.chain = 0;
  g.h.word_count[0] = g.h.word_count[1] = 0;
  uint8_t *p = blob + kHeader;
  for (int s = 0; s < 2; ++s)
    for (uint32_t q = 0; q < nq; ++q)
      for (uint32_t L = 0; L < kLanes; ++L)
        for (uint32_t i = 0; i < 4; ++i)
          *p++ = static_cast<uint8_t>(lane_q(s ? g.vq.data() : g.kq.data(), dim, s == 1, L, q, i) + 128);
  std::memcpy(blob, &g.h, sizeof g.h);
  return static_cast<uint64_t>(p - blob);
}

uint64_t write_rans(GroupIn &g, const GroupCode &gc, const uint32_t *states /* 2 x 64, NULL: continues */,
                    const std::vector<uint16_t> *words /* K, V */, uint8_t *blob) {
  g.h.codec = CF_KV_CODEC_RANS_HYBRID;
  g.h.chain = states ? 1 : 0;
  g.h.word_count[0] = static_cast<uint16_t>(words[0].size());
  g.h.word_count[1] = static_cast<uint16_t>(words[1].size());
  uint64_t at = 0;
  std::memcpy(blob, &g.h, sizeof g.h);
  at += kHeader;
  if (states) {
    std::memcpy(blob + at, states, kStates);
    at += kStates;
  }
  for (int s = 0; s < 2; ++s) {
    std::memcpy(blob + at, gc.raw[s].data(), gc.raw[s].size() * 4);
    at += gc.raw[s].size() * 4;
  }
  for (int s = 0; s < 2; ++s) {
    std::memcpy(blob + at, words[s].data(), words[s].size() * 2);
    at += words[s].size() * 2;
  }
  const uint64_t end = align16(at);
  std::memset(blob + at, 0, end - at);
  return end;
}

// Encode a chain unit: group a alone, or groups a and b (b = the second group of a's pair). Raw fallback: a group
// holding -128 is written INT8 and its partner, if any, starts a chain of its own.
void encode_unit(uint32_t codec, GroupIn *a, GroupIn *b, const Table *tk, const Table *tv, uint8_t *blob_a,
                 uint8_t *blob_b, uint64_t *size_a, uint64_t *size_b) {
  if (codec == CF_KV_CODEC_INT8) {
    *size_a = write_int8(*a, blob_a);
    if (b) *size_b = write_int8(*b, blob_b);
    return;
  }
  const uint32_t dim = a->h.head_dim, steps = dim / 8;
  GroupCode ca, cb;
  build_code(a->kq.data(), a->vq.data(), dim, &ca);
  if (b) build_code(b->kq.data(), b->vq.data(), dim, &cb);
  auto alone = [&](GroupIn *g, GroupCode &c, uint8_t *blob) -> uint64_t {
    if (!c.codable) return write_int8(*g, blob);
    uint32_t st[2][kLanes];
    std::vector<uint16_t> w[2][1];
    for (int s = 0; s < 2; ++s) {
      const std::vector<uint8_t> *j[1] = {&c.joint[s]};
      rans_encode_chain(s ? *tv : *tk, j, 1, steps, st[s], w[s]);
    }
    const std::vector<uint16_t> words[2] = {w[0][0], w[1][0]};
    return write_rans(*g, c, &st[0][0], words, blob);
  };
  if (!b || !ca.codable || !cb.codable) {
    *size_a = alone(a, ca, blob_a);
    if (b) *size_b = alone(b, cb, blob_b);
    return;
  }
  uint32_t st[2][kLanes];
  std::vector<uint16_t> w[2][2];  // [stream][group]
  for (int s = 0; s < 2; ++s) {
    const std::vector<uint8_t> *j[2] = {&ca.joint[s], &cb.joint[s]};
    rans_encode_chain(s ? *tv : *tk, j, 2, steps, st[s], w[s]);
  }
  const std::vector<uint16_t> wa[2] = {w[0][0], w[1][0]}, wb[2] = {w[0][1], w[1][1]};
  *size_a = write_rans(*a, ca, &st[0][0], wa, blob_a);
  *size_b = write_rans(*b, cb, nullptr, wb, blob_b);
}

}  // namespace

extern "C" uint64_t cf_kv_group_blob_max_bytes(uint32_t codec, uint32_t head_dim) {
  if (!dim_ok(codec, head_dim)) return 0;
  const uint64_t int8 = kHeader + 2ull * CF_KV_GROUP_PAGES * kPageTok * head_dim;
  if (codec == CF_KV_CODEC_INT8) return int8;
  if (codec != CF_KV_CODEC_RANS_HYBRID) return 0;
  // header, 2 x 64 states, K and V raw words (7 bits per value), at most one word per lane and step
  const uint64_t raw = 2ull * 7 * (head_dim / 32) * kLanes * 4;
  return std::max<uint64_t>(int8, align16(kHeader + kStates + raw + 2ull * 16 * head_dim));
}

extern "C" cf_status cf_kv_rans_page_histogram(const float *values, uint32_t token_count, uint32_t head_dim,
                                               uint64_t *hist256) {
  if (!values || !hist256 || token_count == 0 || token_count > kPageTok ||
      !dim_ok(CF_KV_CODEC_RANS_HYBRID, head_dim))
    return CF_ERR_INVALID_ARGUMENT;
  std::vector<int8_t> qv(static_cast<size_t>(kPageTok) * head_dim);
  quantize_page(values, token_count, head_dim, qv.data());
  for (uint32_t t = 0; t < kPageTok; ++t)
    for (uint32_t p = 0; p < head_dim / 8; ++p) {
      uint32_t j = 0;
      for (uint32_t i = 0; i < 8; ++i) j |= big(qv[static_cast<size_t>(t) * head_dim + 8 * p + i]) << i;
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
      const uint32_t hi = spread_bigs(j);
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
  if (!keys || !values || !blob || !blob_bytes || page_count == 0 || page_count > CF_KV_GROUP_PAGES)
    return CF_ERR_INVALID_ARGUMENT;
  if (codec != CF_KV_CODEC_INT8 && codec != CF_KV_CODEC_RANS_HYBRID) return CF_ERR_UNSUPPORTED;
  if (!dim_ok(codec, head_dim)) return CF_ERR_INVALID_ARGUMENT;
  if (codec == CF_KV_CODEC_RANS_HYBRID && (!k_table || !v_table)) return CF_ERR_INVALID_ARGUMENT;
  if (capacity < cf_kv_group_blob_max_bytes(codec, head_dim)) return CF_ERR_INVALID_ARGUMENT;
  GroupIn g;
  const cf_status st = prepare_group(keys, values, page_count, token_counts, head_dim, k_table_index, v_table_index,
                                     &g);
  if (st != CF_OK) return st;
  Table tk, tv;
  if (codec == CF_KV_CODEC_RANS_HYBRID && (!load_table(k_table, &tk) || !load_table(v_table, &tv)))
    return CF_ERR_INVALID_ARGUMENT;
  uint64_t sz = 0;
  encode_unit(codec, &g, nullptr, &tk, &tv, blob, nullptr, &sz, nullptr);
  *blob_bytes = sz;
  return CF_OK;
}

extern "C" cf_status cf_kv_encode_groups(uint32_t codec, const float *keys, const float *values, uint64_t ngroups,
                                         const uint64_t *first_page, const uint32_t *page_counts,
                                         const uint32_t *token_counts, uint32_t head_dim, const uint8_t *tables,
                                         const uint32_t *heads, const uint8_t *continues, uint8_t *pool,
                                         uint64_t pool_capacity, uint64_t pool_at, uint32_t *offsets_out,
                                         uint64_t *pool_end, uint32_t threads) {
  if (!keys || !values || !first_page || !page_counts || !pool || !offsets_out || !pool_end || pool_at % 16 != 0)
    return CF_ERR_INVALID_ARGUMENT;
  if (codec != CF_KV_CODEC_INT8 && codec != CF_KV_CODEC_RANS_HYBRID) return CF_ERR_UNSUPPORTED;
  if (codec == CF_KV_CODEC_RANS_HYBRID && !tables) return CF_ERR_INVALID_ARGUMENT;
  const uint64_t cap = cf_kv_group_blob_max_bytes(codec, head_dim);
  if (cap == 0) return CF_ERR_UNSUPPORTED;
  // chain units: group i alone, or (i, i + 1) when group i + 1 continues it
  std::vector<uint64_t> units;
  for (uint64_t i = 0; i < ngroups; ++i) {
    const bool cont = continues && continues[i];
    if (cont) {
      if (i == 0 || (continues[i - 1]) || (heads && heads[i] != heads[i - 1])) return CF_ERR_INVALID_ARGUMENT;
      continue;
    }
    units.push_back(i);
  }
  const uint64_t page_vals = static_cast<uint64_t>(kPageTok) * head_dim;
  std::vector<uint8_t> tmp(ngroups * cap);
  std::vector<uint64_t> sizes(ngroups, 0);
  std::atomic<int> status{CF_OK};
  std::atomic<uint64_t> next{0};
  if (threads == 0) threads = std::max(1u, std::thread::hardware_concurrency());
  auto work = [&]() {
    Table tk, tv;
    uint32_t loaded = ~0u;
    for (;;) {
      const uint64_t u = next.fetch_add(1);
      if (u >= units.size()) return;
      const uint64_t i = units[u];
      const bool pair = i + 1 < ngroups && continues && continues[i + 1];
      const uint32_t h = heads ? heads[i] : 0;
      if (codec == CF_KV_CODEC_RANS_HYBRID && h != loaded) {
        const uint8_t *kt = tables + static_cast<uint64_t>(2 * h) * CF_KV_RANS_TABLE_BYTES;
        if (!load_table(kt, &tk) || !load_table(kt + CF_KV_RANS_TABLE_BYTES, &tv)) {
          status = CF_ERR_INVALID_ARGUMENT;
          return;
        }
        loaded = h;
      }
      GroupIn ga, gb;
      for (uint64_t k = i; k < i + (pair ? 2 : 1); ++k) {
        const uint64_t p0 = first_page[k];
        const cf_status st = prepare_group(keys + p0 * page_vals, values + p0 * page_vals, page_counts[k],
                                           token_counts ? token_counts + p0 : nullptr, head_dim, 2 * h, 2 * h + 1,
                                           k == i ? &ga : &gb);
        if (st != CF_OK) {
          status = st;
          return;
        }
      }
      encode_unit(codec, &ga, pair ? &gb : nullptr, &tk, &tv, tmp.data() + i * cap,
                  pair ? tmp.data() + (i + 1) * cap : nullptr, &sizes[i], pair ? &sizes[i + 1] : nullptr);
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

