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
