// oracle_seal.cpp — CPU restatement of the reference's int4 nibble-page sealing and of attention over such pages.
// TEST INFRASTRUCTURE ONLY (see oracle/__init__.py): the product library never links this file.
//
//   or_nib_seal       reference src/cuda/device_kv_seal_attention.cu:72-113 (finite_scan, quantize_int4,
//                     pack_nibbles): per block of block_size values scale = absmax / 7 (1.0 for an all-zero block),
//                     q = rint(x / scale) clamped to [-8, 7] (saturations counted), symbol q + 8, two symbols per
//                     byte with the even index in the low nibble; NaN/Inf values are counted and the page rejected.
//   or_nib_attention  reference src/cuda/device_kv_seal_attention.cu:116-187 (reference_attention): query token t
//                     at position P = query_begin + t and query head h use kv head h / gqa; key position p counts
//                     when p <= P and (window == 0 or p + window > P); softmax over the visible keys of the sealed
//                     pages (in table order) then the active page; decoded value (symbol - 8) * scale[i / block];
//                     no visible key -> 0. Accumulated in double with the maximum subtracted (two-pass, not online).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <vector>

extern "C" int or_nib_seal(const float *x, uint32_t values, uint32_t block_size, uint8_t *payload, float *scales,
                           uint64_t *saturated, uint64_t *nan_count, uint64_t *inf_count) {
  uint64_t nan = 0, inf = 0, sat = 0;
  for (uint32_t i = 0; i < values; ++i) {
    if (std::isnan(x[i])) ++nan;
    if (std::isinf(x[i])) ++inf;
  }
  *nan_count = nan;
  *inf_count = inf;
  if (nan || inf) return -1;
  const uint32_t blocks = (values + block_size - 1) / block_size;
  for (uint32_t b = 0; b < blocks; ++b) {
    float amax = 0.0f;
    const uint32_t end = std::min<uint64_t>(uint64_t(b + 1) * block_size, values);
    for (uint32_t i = b * block_size; i < end; ++i) amax = std::fmax(amax, std::fabs(x[i]));
    scales[b] = amax > 0.0f ? amax / 7.0f : 1.0f;
  }
  for (uint32_t i = 0; i < (values + 1) / 2; ++i) payload[i] = 0;
  for (uint32_t i = 0; i < values; ++i) {
    const float q = std::nearbyint(x[i] / scales[i / block_size]);  // round half to even (default rounding mode)
    int qi = static_cast<int>(q);
    if (qi < -8) { qi = -8; ++sat; }
    if (qi > 7) { qi = 7; ++sat; }
    const uint8_t sym = static_cast<uint8_t>(qi + 8);
    payload[i / 2] |= (i & 1) ? static_cast<uint8_t>(sym << 4) : sym;
  }
  *saturated = sat;
  return 0;
}

static double nib_value(const uint8_t *payload, const float *scales, uint64_t i, uint32_t block_size) {
  const uint8_t byte = payload[i / 2];
  const int sym = (i & 1) ? (byte >> 4) : (byte & 0x0f);
  return double(sym - 8) * double(scales[i / block_size]);
}

// pages: npages entries of (key payload, value payload, key scales, value scales, token_begin, token_count);
// active: fp32 [active_count, kv_heads, head_dim] (may be null when active_count == 0);
// q: fp32 [q_tokens, kv_heads * gqa, head_dim]; out: fp32 of the same shape.
extern "C" void or_nib_attention(uint32_t npages, const uint8_t *const *kp, const uint8_t *const *vp,
                                 const float *const *ks, const float *const *vs, const uint32_t *tbegin,
                                 const uint32_t *tcount, uint32_t block_size, const float *ak, const float *av,
                                 uint32_t abegin, uint32_t acount, const float *q, uint32_t q_tokens,
                                 uint32_t query_begin, uint32_t kv_heads, uint32_t gqa, uint32_t head_dim,
                                 float softmax_scale, uint32_t window, float *out) {
  const uint32_t qh = kv_heads * gqa;
  std::vector<double> score, kvec(head_dim), acc(head_dim);
  std::vector<std::pair<int, uint32_t>> keys;  // (page index or -1 for active, token)
  for (uint32_t t = 0; t < q_tokens; ++t) {
    const uint64_t P = uint64_t(query_begin) + t;
    auto visible = [&](uint64_t p) { return p <= P && (window == 0 || p + window > P); };
    keys.clear();
    for (uint32_t pg = 0; pg < npages; ++pg)
      for (uint32_t tok = 0; tok < tcount[pg]; ++tok)
        if (visible(uint64_t(tbegin[pg]) + tok)) keys.push_back({int(pg), tok});
    for (uint32_t tok = 0; tok < acount; ++tok)
      if (visible(uint64_t(abegin) + tok)) keys.push_back({-1, tok});
    for (uint32_t h = 0; h < qh; ++h) {
      const uint32_t kh = h / gqa;
      const float *qrow = q + (uint64_t(t) * qh + h) * head_dim;
      float *orow = out + (uint64_t(t) * qh + h) * head_dim;
      if (keys.empty()) {
        for (uint32_t d = 0; d < head_dim; ++d) orow[d] = 0.0f;
        continue;
      }
      score.assign(keys.size(), 0.0);
      double mx = -INFINITY;
      for (size_t k = 0; k < keys.size(); ++k) {
        const auto [pg, tok] = keys[k];
        const uint64_t base = (uint64_t(tok) * kv_heads + kh) * head_dim;
        double s = 0.0;
        for (uint32_t d = 0; d < head_dim; ++d) {
          const double kv = pg < 0 ? double(ak[base + d]) : nib_value(kp[pg], ks[pg], base + d, block_size);
          s += double(qrow[d]) * kv;
        }
        score[k] = s * softmax_scale;
        mx = std::fmax(mx, score[k]);
      }
      double den = 0.0;
      acc.assign(head_dim, 0.0);
      for (size_t k = 0; k < keys.size(); ++k) {
        const auto [pg, tok] = keys[k];
        const uint64_t base = (uint64_t(tok) * kv_heads + kh) * head_dim;
        const double w = std::exp(score[k] - mx);
        den += w;
        for (uint32_t d = 0; d < head_dim; ++d) {
          const double vv = pg < 0 ? double(av[base + d]) : nib_value(vp[pg], vs[pg], base + d, block_size);
          acc[d] += w * vv;
        }
      }
      for (uint32_t d = 0; d < head_dim; ++d) orow[d] = static_cast<float>(acc[d] / den);
    }
  }
}
