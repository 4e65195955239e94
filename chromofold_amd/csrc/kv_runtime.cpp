// kv_runtime.cpp — host-side page/layout validation, resident-byte accounting and the double-precision online
// softmax state of include/chromofold/kv_runtime.h. Pure host code (no device calls).
//
// Semantics (status codes, order of checks, overflow handling) follow reference src/runtime/kv_runtime.cpp:41-254:
// malformed input -> CF_ERR_INVALID_ARGUMENT, arithmetic that would overflow 64 bits -> CF_ERR_UNSUPPORTED.
#include <cmath>
#include <cstring>
#include <limits>

#include "chromofold/kv_runtime.h"

namespace {

// checked u64 arithmetic: false on overflow
bool add_ok(uint64_t a, uint64_t b, uint64_t *out) {
  if (a > std::numeric_limits<uint64_t>::max() - b) return false;
  *out = a + b;
  return true;
}
bool mul_ok(uint64_t a, uint64_t b, uint64_t *out) {
  if (a != 0 && b > std::numeric_limits<uint64_t>::max() / a) return false;
  *out = a * b;
  return true;
}
// a counted array is either empty or has storage
bool present(const void *p, uint64_t n) { return n == 0 || p != nullptr; }

}  // namespace

// reference kv_runtime.cpp:41-74
extern "C" cf_status cf_kv_validate_page(const cf_kv_page_view *pg) {
  if (!pg || pg->struct_size != sizeof(cf_kv_page_view) || pg->abi_version != CF_KV_RUNTIME_ABI_VERSION)
    return CF_ERR_INVALID_ARGUMENT;
  if (!(pg->flags & CF_KV_PAGE_FLAG_SEALED) || pg->token_count == 0 || pg->head_dim == 0 ||
      pg->head_dim > CF_KV_MAX_HEAD_DIM || pg->block_size == 0)
    return CF_ERR_INVALID_ARGUMENT;
  const bool streams_ok = present(pg->k_words, pg->k_word_count) && pg->k_word_count != 0 &&
                          present(pg->v_words, pg->v_word_count) && pg->v_word_count != 0 &&
                          present(pg->k_block_offsets, pg->k_block_count) && pg->k_block_count != 0 &&
                          present(pg->v_block_offsets, pg->v_block_count) && pg->v_block_count != 0 &&
                          present(pg->k_lut, pg->k_lut_count) && pg->k_lut_count != 0 &&
                          present(pg->v_lut, pg->v_lut_count) && pg->v_lut_count != 0 &&
                          present(pg->k_scales, pg->k_scale_count) && present(pg->v_scales, pg->v_scale_count);
  if (!streams_ok) return CF_ERR_INVALID_ARGUMENT;
  if (pg->k_scale_count != pg->head_dim || pg->v_scale_count != pg->token_count) return CF_ERR_INVALID_ARGUMENT;
  uint64_t values = 0;
  if (!mul_ok(pg->token_count, pg->head_dim, &values)) return CF_ERR_UNSUPPORTED;
  const uint64_t blocks = (values + pg->block_size - 1) / pg->block_size;
  if (pg->k_block_count < blocks || pg->v_block_count < blocks) return CF_ERR_INVALID_ARGUMENT;
  if (pg->token_begin > std::numeric_limits<uint32_t>::max() - pg->token_count) return CF_ERR_INVALID_ARGUMENT;
  return CF_OK;
}

// reference kv_runtime.cpp:76-120
extern "C" cf_status cf_kv_validate_layout(const cf_kv_cache_layout *ly) {
  if (!ly || ly->struct_size != sizeof(cf_kv_cache_layout) || ly->abi_version != CF_KV_RUNTIME_ABI_VERSION ||
      ly->layer_count == 0 || ly->kv_head_count == 0 || ly->head_dim == 0 || ly->head_dim > CF_KV_MAX_HEAD_DIM ||
      ly->page_capacity_tokens == 0 || ly->active_element_bytes == 0 || ly->active_element_bytes > 8 ||
      ly->active_token_count > ly->page_capacity_tokens || (ly->page_count != 0 && ly->pages == nullptr))
    return CF_ERR_INVALID_ARGUMENT;
  uint64_t active = 0, bytes = 0;
  if (!mul_ok(ly->active_token_count, ly->layer_count, &active) || !mul_ok(active, ly->kv_head_count, &active) ||
      !mul_ok(active, ly->head_dim, &active) || !mul_ok(active, ly->active_element_bytes, &bytes))
    return CF_ERR_UNSUPPORTED;
  if (ly->active_k_bytes < bytes || ly->active_v_bytes < bytes) return CF_ERR_INVALID_ARGUMENT;
  for (uint64_t i = 0; i < ly->page_count; ++i) {
    const cf_kv_page_view &a = ly->pages[i];
    const cf_status st = cf_kv_validate_page(&a);
    if (st != CF_OK) return st;
    if (a.layer >= ly->layer_count || a.kv_head >= ly->kv_head_count || a.head_dim != ly->head_dim ||
        a.token_count > ly->page_capacity_tokens || a.token_begin + a.token_count > ly->active_token_begin)
      return CF_ERR_INVALID_ARGUMENT;
    for (uint64_t j = i + 1; j < ly->page_count; ++j) {  // sealed pages of one (layer, head) may not overlap
      const cf_kv_page_view &b = ly->pages[j];
      if (b.layer != a.layer || b.kv_head != a.kv_head) continue;
      const uint64_t a_end = static_cast<uint64_t>(a.token_begin) + a.token_count;
      const uint64_t b_end = static_cast<uint64_t>(b.token_begin) + b.token_count;
      if (a.token_begin < b_end && b.token_begin < a_end) return CF_ERR_INVALID_ARGUMENT;
    }
  }
  return CF_OK;
}

// reference kv_runtime.cpp:122-140
extern "C" cf_status cf_kv_page_resident_bytes(const cf_kv_page_view *pg, uint64_t *out) {
  if (!out) return CF_ERR_INVALID_ARGUMENT;
  const cf_status st = cf_kv_validate_page(pg);
  if (st != CF_OK) return st;
  const uint64_t counts[8] = {pg->k_word_count, pg->v_word_count, pg->k_block_count, pg->v_block_count,
                              pg->k_lut_count,  pg->v_lut_count,  pg->k_scale_count, pg->v_scale_count};
  uint64_t total = 0;
  for (uint64_t c : counts) {  // every element is 4 bytes (u32 words, i32 offsets / LUT entries, f32 scales)
    uint64_t b = 0;
    if (!mul_ok(c, 4, &b) || !add_ok(total, b, &total)) return CF_ERR_UNSUPPORTED;
  }
  *out = total;
  return CF_OK;
}

// reference kv_runtime.cpp:142-177
extern "C" cf_status cf_kv_cache_memory_stats(const cf_kv_cache_layout *ly, cf_kv_memory_stats *out) {
  if (!out) return CF_ERR_INVALID_ARGUMENT;
  const cf_status st = cf_kv_validate_layout(ly);
  if (st != CF_OK) return st;
  cf_kv_memory_stats s{};
  s.page_count = ly->page_count;
  s.active_tokens = ly->active_token_count;
  if (!add_ok(ly->active_k_bytes, ly->active_v_bytes, &s.active_payload_bytes) ||
      !mul_ok(ly->page_count, sizeof(cf_kv_page_view), &s.sealed_descriptor_bytes))
    return CF_ERR_UNSUPPORTED;
  for (uint64_t i = 0; i < ly->page_count; ++i) {
    uint64_t b = 0;
    if (cf_kv_page_resident_bytes(&ly->pages[i], &b) != CF_OK || !add_ok(s.sealed_payload_bytes, b, &s.sealed_payload_bytes) ||
        !add_ok(s.sealed_tokens, ly->pages[i].token_count, &s.sealed_tokens))
      return CF_ERR_UNSUPPORTED;
  }
  uint64_t total = 0;
  if (!add_ok(s.sealed_payload_bytes, s.sealed_descriptor_bytes, &total) ||
      !add_ok(total, s.active_payload_bytes, &total))
    return CF_ERR_UNSUPPORTED;
  s.total_resident_bytes = total;
  *out = s;
  return CF_OK;
}

// reference kv_runtime.cpp:179-191
extern "C" cf_status cf_online_softmax_init(cf_online_softmax_state *st, double *weighted, uint32_t dim) {
  if (!st || !weighted || dim == 0 || dim > CF_KV_MAX_HEAD_DIM) return CF_ERR_INVALID_ARGUMENT;
  st->max_score = -std::numeric_limits<double>::infinity();
  st->exp_sum = 0.0;
  st->weighted_values = weighted;
  st->dim = dim;
  st->initialized = 0;
  std::memset(weighted, 0, sizeof(double) * dim);
  return CF_OK;
}

// reference kv_runtime.cpp:193-217: first value initialises (max = score, sum = 1); later ones rescale by the
// running maximum
extern "C" cf_status cf_online_softmax_accumulate(cf_online_softmax_state *st, double score, const float *value) {
  if (!st || !st->weighted_values || !value || st->dim == 0 || !std::isfinite(score)) return CF_ERR_INVALID_ARGUMENT;
  if (!st->initialized) {
    st->max_score = score;
    st->exp_sum = 1.0;
    for (uint32_t d = 0; d < st->dim; ++d) st->weighted_values[d] = value[d];
    st->initialized = 1;
    return CF_OK;
  }
  const double mx = score > st->max_score ? score : st->max_score;
  const double a = std::exp(st->max_score - mx), b = std::exp(score - mx);
  st->exp_sum = st->exp_sum * a + b;
  for (uint32_t d = 0; d < st->dim; ++d) st->weighted_values[d] = st->weighted_values[d] * a + value[d] * b;
  st->max_score = mx;
  return CF_OK;
}

// reference kv_runtime.cpp:219-243: merging split-context partial states (the flash-decoding combine)
extern "C" cf_status cf_online_softmax_merge(cf_online_softmax_state *dst, const cf_online_softmax_state *src) {
  if (!dst || !src || !dst->weighted_values || !src->weighted_values || dst->dim == 0 || dst->dim != src->dim)
    return CF_ERR_INVALID_ARGUMENT;
  if (!src->initialized) return CF_OK;
  if (!dst->initialized) {
    dst->max_score = src->max_score;
    dst->exp_sum = src->exp_sum;
    dst->initialized = 1;
    std::memcpy(dst->weighted_values, src->weighted_values, sizeof(double) * dst->dim);
    return CF_OK;
  }
  const double mx = src->max_score > dst->max_score ? src->max_score : dst->max_score;
  const double a = std::exp(dst->max_score - mx), b = std::exp(src->max_score - mx);
  dst->exp_sum = dst->exp_sum * a + src->exp_sum * b;
  for (uint32_t d = 0; d < dst->dim; ++d)
    dst->weighted_values[d] = dst->weighted_values[d] * a + src->weighted_values[d] * b;
  dst->max_score = mx;
  return CF_OK;
}

// reference kv_runtime.cpp:245-254
extern "C" cf_status cf_online_softmax_finalize(const cf_online_softmax_state *st, float *out) {
  if (!st || !out || !st->weighted_values || !st->initialized || st->dim == 0 || !std::isfinite(st->exp_sum) ||
      st->exp_sum <= 0.0)
    return CF_ERR_INVALID_ARGUMENT;
  for (uint32_t d = 0; d < st->dim; ++d) out[d] = static_cast<float>(st->weighted_values[d] / st->exp_sum);
  return CF_OK;
}
