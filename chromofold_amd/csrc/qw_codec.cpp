// qw_codec.cpp — host encoder of the cf_qw_matrix format (include/chromofold/chromofold_qw.h): int4 quantisation
// per (row, 64-column segment), per-band length-limited canonical Huffman, MSB-first segment-addressable packing.
// Plain C++ on the CPU (the offline weight-preparation step); the decode side is fused_matmul.hip.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <queue>
#include <vector>

#include "chromofold/chromofold_qw.h"

namespace {

uint64_t nseg_of(uint32_t cols) { return (static_cast<uint64_t>(cols) + CF_QW_SEG_COLS - 1) / CF_QW_SEG_COLS; }

// Huffman code lengths of 16 symbols, limited to CF_QW_MAX_CODE_LENGTH: lengths deeper than the limit are clamped,
// then the longest codes below the limit are lengthened (least frequent first) until the Kraft sum is <= 1.
void huffman_lengths16(const uint64_t *freq, uint8_t *len) {
  std::memset(len, 0, 16);
  std::vector<int> used;
  for (int s = 0; s < 16; ++s)
    if (freq[s]) used.push_back(s);
  if (used.empty()) return;
  if (used.size() == 1) {
    len[used[0]] = 1;
    return;
  }
  struct Node {
    uint64_t f;
    int id;
  };
  auto cmp = [](const Node &a, const Node &b) { return a.f != b.f ? a.f > b.f : a.id > b.id; };
  std::priority_queue<Node, std::vector<Node>, decltype(cmp)> pq(cmp);
  std::vector<int> parent(32, -1);
  int next = 16;
  for (int s : used) pq.push({freq[s], s});
  while (pq.size() > 1) {
    const Node a = pq.top();
    pq.pop();
    const Node b = pq.top();
    pq.pop();
    parent[a.id] = parent[b.id] = next;
    pq.push({a.f + b.f, next++});
  }
  for (int s : used) {
    int d = 0;
    for (int v = s; parent[v] >= 0; v = parent[v]) ++d;
    len[s] = static_cast<uint8_t>(std::min<int>(d, CF_QW_MAX_CODE_LENGTH));
  }
  auto kraft_over = [&] {
    uint64_t k = 0;
    for (int s : used) k += uint64_t(1) << (CF_QW_MAX_CODE_LENGTH - len[s]);
    return k > (uint64_t(1) << CF_QW_MAX_CODE_LENGTH);
  };
  while (kraft_over()) {
    int pick = -1;
    for (int s : used)
      if (len[s] < CF_QW_MAX_CODE_LENGTH &&
          (pick < 0 || len[s] > len[pick] || (len[s] == len[pick] && freq[s] < freq[pick])))
        pick = s;
    ++len[pick];
  }
}

// canonical codes in (length, symbol) order
void canonical16(const uint8_t *len, uint32_t *code) {
  uint32_t c = 0;
  int prev = 0;
  for (int l = 1; l <= static_cast<int>(CF_QW_MAX_CODE_LENGTH); ++l)
    for (int s = 0; s < 16; ++s)
      if (len[s] == l) {
        c <<= (l - prev);
        prev = l;
        code[s] = c++;
      }
}

}  // namespace

extern "C" cf_status cf_qw_quantize_int4(const float *w, uint32_t rows, uint32_t cols, uint8_t *sym, float *scales) {
  if (!w || !sym || !scales || rows == 0 || cols == 0) return CF_ERR_INVALID_ARGUMENT;
  const uint64_t ns = nseg_of(cols);
  for (uint64_t r = 0; r < rows; ++r)
    for (uint64_t s = 0; s < ns; ++s) {
      const uint64_t c0 = s * CF_QW_SEG_COLS, c1 = std::min<uint64_t>(cols, c0 + CF_QW_SEG_COLS);
      float amax = 0.f;
      for (uint64_t c = c0; c < c1; ++c) amax = std::max(amax, std::fabs(w[r * cols + c]));
      const float sc = (amax > 0.f && std::isfinite(amax)) ? amax / 7.0f : 1.0f;
      scales[r * ns + s] = sc;
      for (uint64_t c = c0; c < c1; ++c) {
        const float q = std::nearbyint(w[r * cols + c] / sc);  // round half to even
        sym[r * cols + c] = static_cast<uint8_t>(std::clamp(q, -8.0f, 7.0f) + 8.0f);
      }
    }
  return CF_OK;
}

extern "C" uint64_t cf_qw_huffman_plan(const uint8_t *sym, uint32_t rows, uint32_t cols, uint8_t *code_lengths) {
  if (!sym || !code_lengths || rows == 0 || cols == 0) return 0;
  const uint64_t bands = (rows + CF_QW_BAND_ROWS - 1) / CF_QW_BAND_ROWS;
  uint64_t bits = 0;
  for (uint64_t b = 0; b < bands; ++b) {
    uint64_t freq[16] = {};
    const uint64_t r0 = b * CF_QW_BAND_ROWS, r1 = std::min<uint64_t>(rows, r0 + CF_QW_BAND_ROWS);
    for (uint64_t i = r0 * cols; i < r1 * cols; ++i) {
      if (sym[i] > 15) return 0;
      ++freq[sym[i]];
    }
    huffman_lengths16(freq, code_lengths + b * 16);
    for (int s = 0; s < 16; ++s) bits += freq[s] * code_lengths[b * 16 + s];
  }
  return (bits + 31) / 32 + 2;  // two words of padding cover the decoder's lookahead past the last code
}

extern "C" cf_status cf_qw_huffman_encode(const uint8_t *sym, uint32_t rows, uint32_t cols,
                                          const uint8_t *code_lengths, uint32_t *words, uint64_t word_capacity,
                                          uint32_t *seg_offsets) {
  if (!sym || !code_lengths || !words || !seg_offsets || rows == 0 || cols == 0) return CF_ERR_INVALID_ARGUMENT;
  const uint64_t ns = nseg_of(cols);
  std::memset(words, 0, word_capacity * 4);
  uint64_t bit = 0;
  for (uint64_t r = 0; r < rows; ++r) {
    const uint8_t *len = code_lengths + (r / CF_QW_BAND_ROWS) * 16;
    uint32_t code[16] = {};
    canonical16(len, code);
    for (uint64_t s = 0; s < ns; ++s) {
      if (bit > 0xFFFFFFFFull) return CF_ERR_UNSUPPORTED;
      seg_offsets[r * ns + s] = static_cast<uint32_t>(bit);
      const uint64_t c0 = s * CF_QW_SEG_COLS, c1 = std::min<uint64_t>(cols, c0 + CF_QW_SEG_COLS);
      for (uint64_t c = c0; c < c1; ++c) {
        const uint8_t v = sym[r * cols + c];
        const int l = v < 16 ? len[v] : 0;
        if (l == 0) return CF_ERR_INVALID_ARGUMENT;  // symbol without a code in this band
        if ((bit + l + 31) / 32 + 1 > word_capacity) return CF_ERR_INVALID_ARGUMENT;
        for (int i = l - 1; i >= 0; --i, ++bit)  // MSB first
          if ((code[v] >> i) & 1u) words[bit >> 5] |= 1u << (31 - (bit & 31));
      }
    }
  }
  return CF_OK;
}

// ------------------------------------------------------------------------------------------------ rANS (pairs)
namespace {

constexpr uint32_t kProbM = 1u << CF_QW_RANS_PROB_BITS;  // 4096
constexpr uint32_t kRansL = 1u << 16;                    // lane states live in [2^16, 2^32)

struct RansGeom {
  uint64_t bands, nstripes, nchunks;
};

RansGeom rans_geom(uint32_t rows, uint32_t cols) {
  RansGeom g;
  g.bands = (rows + CF_QW_BAND_ROWS - 1) / CF_QW_BAND_ROWS;
  g.nstripes = (static_cast<uint64_t>(cols) + CF_QW_STRIPE_COLS - 1) / CF_QW_STRIPE_COLS;
  g.nchunks = (g.nstripes + CF_QW_CHUNK_STRIPES - 1) / CF_QW_CHUNK_STRIPES;
  return g;
}

// The pair lane l decodes at step t of stripe `stripe` in band b (the column order of chromofold_qw.h).
inline uint32_t rans_pair(const uint8_t *sym, uint32_t rows, uint32_t cols, uint8_t zero, uint64_t b,
                          uint64_t stripe, int l, int t) {
  const int g = l >> 4, r = l & 15;
  const uint64_t row = b * CF_QW_BAND_ROWS + r;
  const uint64_t c = stripe * CF_QW_STRIPE_COLS + 64 * (t >> 3) + 16 * g + 4 * ((t >> 1) & 3) + 2 * (t & 1);
  const auto at = [&](uint64_t col) -> uint32_t { return row < rows && col < cols ? sym[row * cols + col] : zero; };
  return at(c) | (at(c + 1) << 4);
}

// Counts -> frequencies summing to 4096: largest remainder, then every present pair raised to >= 1 by taking from
// the largest frequencies (ties: lower symbol first).
void normalise_pairs(const uint64_t *cnt, uint16_t *freq) {
  uint64_t total = 0;
  for (int s = 0; s < 256; ++s) total += cnt[s];
  int64_t f[256];
  uint64_t rem[256];
  int64_t sum = 0;
  for (int s = 0; s < 256; ++s) {
    f[s] = static_cast<int64_t>(cnt[s] * kProbM / total);
    rem[s] = cnt[s] * kProbM % total;
    sum += f[s];
  }
  std::vector<int> order;
  for (int s = 0; s < 256; ++s)
    if (cnt[s]) order.push_back(s);
  std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return rem[a] > rem[b]; });
  for (size_t i = 0; sum < kProbM; i = (i + 1) % order.size()) {
    ++f[order[i]];
    ++sum;
  }
  for (int s = 0; s < 256; ++s)
    if (cnt[s] && f[s] == 0) {
      f[s] = 1;
      ++sum;
    }
  while (sum > kProbM) {
    int pick = -1;
    for (int s = 0; s < 256; ++s)
      if (f[s] > 1 && (pick < 0 || f[s] > f[pick])) pick = s;
    --f[pick];
    --sum;
  }
  for (int s = 0; s < 256; ++s) freq[s] = static_cast<uint16_t>(f[s]);
}

// Encodes one stripe: the 64 lane states (in) are 2^16, out the decoder's initial states; `out` receives the
// stream's 16-bit words in decoding order. Returns false for a pair without frequency.
bool rans_encode_stripe(const uint8_t *sym, uint32_t rows, uint32_t cols, uint8_t zero, uint64_t b, uint64_t stripe,
                        const uint16_t *freq, const uint32_t *cum, uint32_t *x, std::vector<uint16_t> &out) {
  out.clear();
  for (int l = 0; l < 64; ++l) x[l] = kRansL;
  // decoding runs t = 0..31 with lanes in increasing order, so encoding runs backwards: t = 31..0, lanes 63..0,
  // and the emitted words are reversed at the end
  for (int t = 31; t >= 0; --t)
    for (int l = 63; l >= 0; --l) {
      const uint32_t s = rans_pair(sym, rows, cols, zero, b, stripe, l, t);
      const uint32_t f = freq[s];
      if (f == 0) return false;
      const uint64_t xmax = static_cast<uint64_t>(kRansL >> CF_QW_RANS_PROB_BITS << 16) * f;
      if (x[l] >= xmax) {
        out.push_back(static_cast<uint16_t>(x[l] & 0xFFFFu));
        x[l] >>= 16;
      }
      x[l] = (x[l] / f) * kProbM + x[l] % f + cum[s];
    }
  std::reverse(out.begin(), out.end());
  return true;
}

}  // namespace

extern "C" cf_status cf_qw_rans_plan(const uint8_t *sym, uint32_t rows, uint32_t cols, uint8_t zero,
                                     uint16_t *cum_out, uint32_t *chunk_words, uint32_t *last_words) {
  if (!sym || !cum_out || !chunk_words || !last_words || rows == 0 || cols == 0 || zero > 15)
    return CF_ERR_INVALID_ARGUMENT;
  const RansGeom g = rans_geom(rows, cols);
  for (uint64_t i = 0; i < static_cast<uint64_t>(rows) * cols; ++i)
    if (sym[i] > 15) return CF_ERR_INVALID_ARGUMENT;
  uint64_t full_max = 0, last_max = 0;
  std::vector<uint16_t> words;
  for (uint64_t b = 0; b < g.bands; ++b) {
    uint64_t cnt[256] = {};
    for (uint64_t st = 0; st < g.nstripes; ++st)
      for (int t = 0; t < 32; ++t)
        for (int l = 0; l < 64; ++l) ++cnt[rans_pair(sym, rows, cols, zero, b, st, l, t)];
    uint16_t f[256];
    normalise_pairs(cnt, f);
    uint32_t cum[256], c = 0;
    for (int s = 0; s < 256; ++s) {
      cum[s] = c;
      cum_out[b * 256 + s] = static_cast<uint16_t>(c);
      c += f[s];
    }
    for (uint64_t ch = 0; ch < g.nchunks; ++ch) {
      uint64_t slot = 0;
      uint32_t x[64];
      for (uint64_t st = ch * CF_QW_CHUNK_STRIPES; st < std::min<uint64_t>(g.nstripes, (ch + 1) * CF_QW_CHUNK_STRIPES);
           ++st) {
        if (!rans_encode_stripe(sym, rows, cols, zero, b, st, f, cum, x, words)) return CF_ERR_INVALID_ARGUMENT;
        slot += words.size();
      }
      uint64_t &mx = ch + 1 == g.nchunks ? last_max : full_max;
      mx = std::max(mx, slot);
    }
  }
  const uint64_t cw = (full_max + 7) / 8 * 8, lw = std::max<uint64_t>(8, (last_max + 7) / 8 * 8);
  if (cw > CF_QW_MAX_CHUNK_WORDS || lw > CF_QW_MAX_CHUNK_WORDS) return CF_ERR_UNSUPPORTED;
  *chunk_words = static_cast<uint32_t>(cw);
  *last_words = static_cast<uint32_t>(lw);
  return CF_OK;
}

extern "C" cf_status cf_qw_rans_encode(const uint8_t *sym, uint32_t rows, uint32_t cols, uint8_t zero,
                                       const uint16_t *cum_in, uint32_t chunk_words, uint32_t last_words,
                                       uint32_t *words, uint64_t word_capacity, uint32_t *offsets, uint32_t *states) {
  if (!sym || !cum_in || !words || !offsets || !states || rows == 0 || cols == 0 || zero > 15)
    return CF_ERR_INVALID_ARGUMENT;
  const RansGeom g = rans_geom(rows, cols);
  if (chunk_words % 8 != 0 || chunk_words > CF_QW_MAX_CHUNK_WORDS || (g.nchunks > 1 && chunk_words == 0))
    return CF_ERR_INVALID_ARGUMENT;
  if (last_words == 0 || last_words % 8 != 0 || last_words > CF_QW_MAX_CHUNK_WORDS) return CF_ERR_INVALID_ARGUMENT;
  const uint64_t band_words = (g.nchunks - 1) * chunk_words + last_words;
  if (word_capacity < g.bands * band_words / 2) return CF_ERR_INVALID_ARGUMENT;
  std::memset(words, 0, word_capacity * 4);
  uint16_t *w16 = reinterpret_cast<uint16_t *>(words);  // little-endian: 16-bit word 2i + 1 is the high half
  std::vector<uint16_t> stream;
  for (uint64_t b = 0; b < g.bands; ++b) {
    const uint16_t *cb = cum_in + b * 256;
    uint16_t f[256];
    uint32_t cum[256];
    if (cb[0] != 0) return CF_ERR_INVALID_ARGUMENT;
    for (int s = 0; s < 256; ++s) {
      const uint32_t next = s < 255 ? cb[s + 1] : kProbM;
      if (next < cb[s]) return CF_ERR_INVALID_ARGUMENT;
      cum[s] = cb[s];
      f[s] = static_cast<uint16_t>(next - cb[s]);
    }
    for (uint64_t ch = 0; ch < g.nchunks; ++ch) {
      uint16_t *slot = w16 + b * band_words + ch * chunk_words;
      const uint64_t cap = ch + 1 == g.nchunks ? last_words : chunk_words;
      uint64_t at = 0;
      for (uint64_t st = ch * CF_QW_CHUNK_STRIPES; st < std::min<uint64_t>(g.nstripes, (ch + 1) * CF_QW_CHUNK_STRIPES);
           ++st) {
        uint32_t *x = states + (b * g.nstripes + st) * 64;
        if (!rans_encode_stripe(sym, rows, cols, zero, b, st, f, cum, x, stream)) return CF_ERR_INVALID_ARGUMENT;
        if (at + stream.size() > cap) return CF_ERR_INVALID_ARGUMENT;
        offsets[b * g.nstripes + st] = static_cast<uint32_t>(at);
        std::copy(stream.begin(), stream.end(), slot + at);
        at += stream.size();
      }
    }
  }
  return CF_OK;
}
