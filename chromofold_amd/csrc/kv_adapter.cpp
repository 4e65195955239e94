// kv_adapter.cpp — the llama.cpp paged-KV adapter (include/chromofold/chromofold_kv_adapter.h) and the host encoder
// of the reference's fixed-width page format. Host C++ over the HIP runtime; attention goes through the seam
// cf_kv_paged_attention_async (kv_legacy.hip) with its decode-shape route off (that route takes rANS pages only).
//
// Behaviour follows reference integrations/llama.cpp/chromofold_kv_adapter.cpp:21-236 and
// src/runtime/compressed_kv_cache.cu:66-210: per (layer, kv head) a host fp32 active tail that must grow
// contiguously, pages sealed every page_size tokens with the fixture codec (int4 or int8, K per-channel / V
// per-token scales), flush() seals partial tails, the attention view = sealed pages + the active tail interleaved
// [tokens, kv_heads, head_dim] (tails must be aligned across heads), sequence 0 only (seq_cp reports the missing
// shared-page table, seq_shift only accepts 0), errors as -1 + last_error.
//
// Memory layout, MI355X side: the reference allocates eight device arrays per page and re-uploads the whole
// descriptor array and the tail on every attention call. Here each layer owns ONE device arena of page payloads
// (K/V words and scales, 16-byte aligned slices) that grows by doubling, the degenerate LUT and the block offsets
// of full pages are stored once per adapter and shared by every page, the device descriptor array is rebuilt only
// when pages were added or the arena moved, and the device tail only when the tail changed.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "chromofold/chromofold_kv_adapter.h"
#include "chromofold/kv_codec_ext.h"
#include "kv_seam_route.hpp"
#include "chromofold/kv_cuda.h"

extern "C" cf_status cf_kv_encode_fixed_page(uint32_t bits, const float *keys, const float *values,
                                             uint32_t token_count, uint32_t head_dim, uint32_t block,
                                             uint32_t *k_words, uint32_t *v_words, float *k_scales, float *v_scales,
                                             int32_t *block_offsets) {
  if ((bits != 4 && bits != 8) || !keys || !values || token_count == 0 || head_dim == 0 || block == 0 || !k_words ||
      !v_words || !k_scales || !v_scales || !block_offsets)
    return CF_ERR_INVALID_ARGUMENT;
  const int qmax = (1 << (bits - 1)) - 1, zp = 1 << (bits - 1);
  const uint64_t n = static_cast<uint64_t>(token_count) * head_dim;
  for (uint64_t i = 0; i < n; ++i)
    if (!std::isfinite(keys[i]) || !std::isfinite(values[i])) return CF_ERR_INVALID_ARGUMENT;
  for (uint32_t d = 0; d < head_dim; ++d) {
    float m = 0.f;
    for (uint32_t t = 0; t < token_count; ++t) m = std::max(m, std::fabs(keys[static_cast<uint64_t>(t) * head_dim + d]));
    k_scales[d] = m == 0.f ? 1.f : m / static_cast<float>(qmax);
  }
  for (uint32_t t = 0; t < token_count; ++t) {
    float m = 0.f;
    for (uint32_t d = 0; d < head_dim; ++d) m = std::max(m, std::fabs(values[static_cast<uint64_t>(t) * head_dim + d]));
    v_scales[t] = m == 0.f ? 1.f : m / static_cast<float>(qmax);
  }
  const uint64_t nwords = (n * bits + 31) / 32;
  std::memset(k_words, 0, nwords * 4);
  std::memset(v_words, 0, nwords * 4);
  auto sym = [&](float x, float s) {  // lrint: round half to even in the default rounding mode
    const long q = std::lrint(x / s);
    return static_cast<uint32_t>(std::clamp<long>(q, -(qmax + 1), qmax) + zp);
  };
  for (uint64_t i = 0; i < n; ++i) {
    const uint32_t t = static_cast<uint32_t>(i / head_dim), d = static_cast<uint32_t>(i % head_dim);
    const uint64_t bit = i * bits;
    const uint32_t shift = (32u - bits) - static_cast<uint32_t>(bit & 31u);  // MSB-first inside each word
    k_words[bit >> 5] |= sym(keys[i], k_scales[d]) << shift;
    v_words[bit >> 5] |= sym(values[i], v_scales[t]) << shift;
  }
  for (uint64_t b = 0; b * block < n; ++b) block_offsets[b] = static_cast<int32_t>(b * block * bits);
  return CF_OK;
}

namespace {

constexpr uint32_t kBlock = 64;  // symbols per block offset (the reference cache's encoder setting)

size_t align16(size_t v) { return (v + 15) & ~size_t(15); }

void hip_check(hipError_t e, const char *what) {
  if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// grow-only device buffer; growing keeps the first `keep` bytes
struct DeviceBuffer {
  void *ptr = nullptr;
  size_t cap = 0;
  DeviceBuffer() = default;
  DeviceBuffer(const DeviceBuffer &) = delete;
  DeviceBuffer &operator=(const DeviceBuffer &) = delete;
  DeviceBuffer(DeviceBuffer &&o) noexcept : ptr(o.ptr), cap(o.cap) {
    o.ptr = nullptr;
    o.cap = 0;
  }
  DeviceBuffer &operator=(DeviceBuffer &&o) noexcept {
    std::swap(ptr, o.ptr);
    std::swap(cap, o.cap);
    return *this;
  }
  ~DeviceBuffer() {
    if (ptr) (void)hipFree(ptr);
  }
  // true when the buffer moved
  bool reserve(size_t bytes, size_t keep, hipStream_t s) {
    if (bytes <= cap) return false;
    const size_t nc = std::max({bytes, cap * 2, size_t(1) << 20});
    void *np = nullptr;
    hip_check(hipMalloc(&np, nc), "device allocation");
    if (keep && ptr) {
      hip_check(hipMemcpyAsync(np, ptr, keep, hipMemcpyDeviceToDevice, s), "device copy");
      hip_check(hipStreamSynchronize(s), "stream synchronize");
    }
    if (ptr) hip_check(hipFree(ptr), "device free");
    ptr = np;
    cap = nc;
    return true;
  }
  template <typename T>
  T *at(size_t off) const {
    return reinterpret_cast<T *>(static_cast<uint8_t *>(ptr) + off);
  }
};

struct Page {  // one sealed page of one kv head: payload slices inside the layer arena
  uint32_t kv_head, token_begin, token_count;
  size_t k_words, v_words, k_scales, v_scales, boff;  // byte offsets in the arena (boff: own offsets, partial pages)
  bool own_boff;
  uint64_t bytes;  // payload bytes of this page
};

struct Tail {
  uint32_t token_begin = 0;
  std::vector<float> k, v;
};

struct Layer {
  DeviceBuffer arena, desc, tail_k, tail_v;
  size_t used = 0;
  std::vector<Page> pages;
  std::vector<cf_kv_device_page> host_desc;
  std::vector<float> tail_stage_k, tail_stage_v;
  bool desc_dirty = true, tail_dirty = true;
  uint32_t tail_tokens = 0, tail_begin = 0;
  std::vector<Tail> tails;
};

}  // namespace

struct cf_llama_kv_adapter {
  cf_llama_kv_options opt{};
  uint32_t bits = 4;
  std::vector<Layer> layers;
  DeviceBuffer shared;  // LUT [2^bits] + block offsets of a full page
  size_t shared_lut = 0, shared_boff = 0;
  DeviceBuffer host_q, host_out;  // scratch of cf_llama_kv_attention_host
  uint64_t appended = 0, sealed_tokens = 0;
  std::string last_error;
};

namespace {

template <typename Op>
int guarded(cf_llama_kv_adapter *a, Op &&op) {
  if (a == nullptr) return -1;
  try {
    op();
    a->last_error.clear();
    return 0;
  } catch (const std::exception &e) {
    a->last_error = e.what();
    return -1;
  } catch (...) {
    a->last_error = "unknown ChromoFold KV error";
    return -1;
  }
}

void reset(cf_llama_kv_adapter *a) {
  for (Layer &L : a->layers) {
    L.used = 0;
    L.pages.clear();
    L.host_desc.clear();
    L.desc_dirty = L.tail_dirty = true;
    L.tail_tokens = L.tail_begin = 0;
    for (Tail &t : L.tails) t = Tail{};
  }
  a->appended = a->sealed_tokens = 0;
}

void init_shared(cf_llama_kv_adapter *a, hipStream_t s) {
  const uint32_t levels = 1u << a->bits;
  const uint64_t n = static_cast<uint64_t>(a->opt.page_size) * a->opt.head_dim;
  const uint64_t nb = (n + kBlock - 1) / kBlock;
  std::vector<int32_t> lut(levels), boff(nb);
  for (uint32_t i = 0; i < levels; ++i) lut[i] = static_cast<int32_t>(i | (a->bits << 8));
  for (uint64_t b = 0; b < nb; ++b) boff[b] = static_cast<int32_t>(b * kBlock * a->bits);
  a->shared_lut = 0;
  a->shared_boff = align16(4ull * levels);
  a->shared.reserve(a->shared_boff + 4 * nb, 0, s);
  hip_check(hipMemcpy(a->shared.at<void>(a->shared_lut), lut.data(), 4ull * levels, hipMemcpyHostToDevice), "upload");
  hip_check(hipMemcpy(a->shared.at<void>(a->shared_boff), boff.data(), 4 * nb, hipMemcpyHostToDevice), "upload");
}

// encode tokens [0, count) of a head's tail as one page and append it to the layer arena
void seal(cf_llama_kv_adapter *a, Layer &L, uint32_t head, uint32_t count, hipStream_t s) {
  if (!a->shared.cap) init_shared(a, s);
  Tail &tl = L.tails[head];
  const uint32_t hd = a->opt.head_dim;
  const uint64_t n = static_cast<uint64_t>(count) * hd;
  const uint64_t nw = (n * a->bits + 31) / 32, nb = (n + kBlock - 1) / kBlock;
  std::vector<uint32_t> kw(nw), vw(nw);
  std::vector<float> ks(hd), vs(count);
  std::vector<int32_t> boff(nb);
  if (cf_kv_encode_fixed_page(a->bits, tl.k.data(), tl.v.data(), count, hd, kBlock, kw.data(), vw.data(), ks.data(),
                              vs.data(), boff.data()) != CF_OK)
    throw std::invalid_argument("invalid quantization input");
  Page p{};
  p.kv_head = head;
  p.token_begin = tl.token_begin;
  p.token_count = count;
  p.own_boff = count != a->opt.page_size;
  size_t at = L.used;
  p.k_words = at;
  at = align16(at + 4 * nw);
  p.v_words = at;
  at = align16(at + 4 * nw);
  p.k_scales = at;
  at = align16(at + 4ull * hd);
  p.v_scales = at;
  at = align16(at + 4ull * count);
  p.boff = at;
  if (p.own_boff) at = align16(at + 4 * nb);
  p.bytes = at - L.used;
  if (L.arena.reserve(at, L.used, s)) L.desc_dirty = true;  // every page pointer moved
  auto put = [&](size_t off, const void *src, size_t bytes) {
    hip_check(hipMemcpyAsync(L.arena.at<void>(off), src, bytes, hipMemcpyHostToDevice, s), "upload");
  };
  put(p.k_words, kw.data(), 4 * nw);
  put(p.v_words, vw.data(), 4 * nw);
  put(p.k_scales, ks.data(), 4ull * hd);
  put(p.v_scales, vs.data(), 4ull * count);
  if (p.own_boff) put(p.boff, boff.data(), 4 * nb);
  hip_check(hipStreamSynchronize(s), "stream synchronize");  // the host staging vectors die here
  L.used = at;
  L.pages.push_back(p);
  L.desc_dirty = true;
  tl.k.erase(tl.k.begin(), tl.k.begin() + n);
  tl.v.erase(tl.v.begin(), tl.v.begin() + n);
  tl.token_begin += count;
  L.tail_dirty = true;
  a->sealed_tokens += count;
}

void seal_full(cf_llama_kv_adapter *a, Layer &L, uint32_t head, hipStream_t s) {
  while (L.tails[head].k.size() / a->opt.head_dim >= a->opt.page_size) seal(a, L, head, a->opt.page_size, s);
}

void refresh_descriptors(cf_llama_kv_adapter *a, Layer &L, hipStream_t s) {
  if (!L.desc_dirty) return;
  L.host_desc.resize(L.pages.size());
  for (size_t i = 0; i < L.pages.size(); ++i) {
    const Page &p = L.pages[i];
    cf_kv_device_page &d = L.host_desc[i];
    d = cf_kv_device_page{};
    const int32_t *boff = p.own_boff ? L.arena.at<const int32_t>(p.boff) : a->shared.at<const int32_t>(a->shared_boff);
    const int32_t *lut = a->shared.at<const int32_t>(a->shared_lut);
    d.k_words = L.arena.at<const uint32_t>(p.k_words);
    d.k_block_offsets = boff;
    d.k_lut = lut;
    d.k_scales = L.arena.at<const float>(p.k_scales);
    d.v_words = L.arena.at<const uint32_t>(p.v_words);
    d.v_block_offsets = boff;
    d.v_lut = lut;
    d.v_scales = L.arena.at<const float>(p.v_scales);
    d.token_begin = p.token_begin;
    d.token_count = p.token_count;
    d.head_dim = a->opt.head_dim;
    d.block_size = kBlock;
    d.k_max_code_length = d.v_max_code_length = a->bits;
    d.zero_point = 1u << (a->bits - 1);
    d.kv_head = p.kv_head;
    d.fixed_code_length = a->bits;
  }
  if (!L.host_desc.empty()) {
    const size_t bytes = L.host_desc.size() * sizeof(cf_kv_device_page);
    L.desc.reserve(bytes, 0, s);
    hip_check(hipMemcpyAsync(L.desc.ptr, L.host_desc.data(), bytes, hipMemcpyHostToDevice, s), "upload");
  }
  L.desc_dirty = false;
}

void refresh_tail(cf_llama_kv_adapter *a, Layer &L, hipStream_t s) {
  if (!L.tail_dirty) return;
  const uint32_t hd = a->opt.head_dim, kvh = a->opt.kv_head_count;
  const uint32_t tokens = static_cast<uint32_t>(L.tails[0].k.size() / hd);
  for (uint32_t h = 0; h < kvh; ++h)
    if (L.tails[h].k.size() / hd != tokens || (tokens && L.tails[h].token_begin != L.tails[0].token_begin))
      throw std::runtime_error("KV active tails are not aligned across heads");
  L.tail_tokens = tokens;
  L.tail_begin = L.tails[0].token_begin;
  if (tokens) {
    const size_t n = static_cast<size_t>(tokens) * kvh * hd;
    L.tail_stage_k.resize(n);
    L.tail_stage_v.resize(n);
    for (uint32_t h = 0; h < kvh; ++h)
      for (uint32_t t = 0; t < tokens; ++t) {
        std::memcpy(&L.tail_stage_k[(static_cast<size_t>(t) * kvh + h) * hd], &L.tails[h].k[static_cast<size_t>(t) * hd],
                    4ull * hd);
        std::memcpy(&L.tail_stage_v[(static_cast<size_t>(t) * kvh + h) * hd], &L.tails[h].v[static_cast<size_t>(t) * hd],
                    4ull * hd);
      }
    L.tail_k.reserve(4 * n, 0, s);
    L.tail_v.reserve(4 * n, 0, s);
    hip_check(hipMemcpyAsync(L.tail_k.ptr, L.tail_stage_k.data(), 4 * n, hipMemcpyHostToDevice, s), "upload");
    hip_check(hipMemcpyAsync(L.tail_v.ptr, L.tail_stage_v.data(), 4 * n, hipMemcpyHostToDevice, s), "upload");
  }
  L.tail_dirty = false;
}

}  // namespace

extern "C" int cf_llama_kv_options_validate(const cf_llama_kv_options *o) {
  if (o == nullptr || o->struct_size != sizeof(cf_llama_kv_options)) return -1;
  if (o->backend == CF_LLAMA_KV_BACKEND_DENSE) return 0;
  if (o->backend != CF_LLAMA_KV_BACKEND_CHROMOFOLD || o->layer_count == 0 || o->kv_head_count == 0 ||
      o->query_head_count == 0 || o->head_dim == 0 || o->page_size == 0 || o->gqa_group_size == 0 ||
      o->query_head_count != o->kv_head_count * o->gqa_group_size)
    return -1;
  return 0;
}

extern "C" cf_llama_kv_adapter *cf_llama_kv_create(const cf_llama_kv_options *o) {
  if (cf_llama_kv_options_validate(o) != 0 || o->backend != CF_LLAMA_KV_BACKEND_CHROMOFOLD) return nullptr;
  if (o->head_dim > CF_KV_MAX_HEAD_DIM) return nullptr;  // the cache's own configuration limit
  try {
    auto a = std::make_unique<cf_llama_kv_adapter>();
    a->opt = *o;
    a->bits = o->kv_bits == 8 ? 8u : 4u;
    a->layers.resize(o->layer_count);
    for (Layer &L : a->layers) L.tails.resize(o->kv_head_count);
    return a.release();  // no device work until the first page is sealed
  } catch (...) {
    return nullptr;
  }
}

extern "C" void cf_llama_kv_destroy(cf_llama_kv_adapter *a) { delete a; }

extern "C" int cf_llama_kv_append(cf_llama_kv_adapter *a, uint32_t layer, uint32_t kv_head, uint32_t token_begin,
                                  const float *keys, const float *values, uint32_t token_count, void *stream) {
  return guarded(a, [&] {
    if (keys == nullptr || values == nullptr || token_count == 0) throw std::invalid_argument("invalid KV append");
    if (layer >= a->opt.layer_count || kv_head >= a->opt.kv_head_count)
      throw std::out_of_range("KV layer/head out of range");
    Layer &L = a->layers[layer];
    Tail &t = L.tails[kv_head];
    const uint32_t hd = a->opt.head_dim;
    const uint32_t active = static_cast<uint32_t>(t.k.size() / hd);
    if (active == 0)
      t.token_begin = token_begin;
    else if (token_begin != t.token_begin + active)
      throw std::invalid_argument("KV append must be logically contiguous");
    const size_t n = static_cast<size_t>(token_count) * hd;
    t.k.insert(t.k.end(), keys, keys + n);
    t.v.insert(t.v.end(), values, values + n);
    a->appended += token_count;
    L.tail_dirty = true;
    seal_full(a, L, kv_head, static_cast<hipStream_t>(stream));
  });
}

extern "C" int cf_llama_kv_attention(cf_llama_kv_adapter *a, uint32_t layer, const float *queries_device,
                                     float *output_device, uint32_t query_count, uint32_t query_head_count,
                                     uint32_t gqa_group_size, uint32_t query_token_begin, float softmax_scale,
                                     uint32_t causal_window, void *stream) {
  return guarded(a, [&] {
    if (queries_device == nullptr || output_device == nullptr || gqa_group_size == 0 || query_head_count == 0 ||
        query_head_count % gqa_group_size != 0)
      throw std::invalid_argument("invalid ChromoFold attention request");
    if (layer >= a->opt.layer_count) throw std::out_of_range("KV layer out of range");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    Layer &L = a->layers[layer];
    refresh_descriptors(a, L, s);
    refresh_tail(a, L, s);
    cf_kv_paged_attention_desc d{};
    d.struct_size = sizeof(d);
    d.abi_version = CF_KV_CUDA_ABI_VERSION;
    d.pages = L.pages.empty() ? nullptr : static_cast<const cf_kv_device_page *>(L.desc.ptr);
    d.page_count = static_cast<uint32_t>(L.pages.size());
    d.kv_head_count = query_head_count / gqa_group_size;
    d.query_head_count = query_head_count;
    d.gqa_group_size = gqa_group_size;
    d.active_k = L.tail_tokens ? static_cast<const float *>(L.tail_k.ptr) : nullptr;
    d.active_v = L.tail_tokens ? static_cast<const float *>(L.tail_v.ptr) : nullptr;
    d.active_token_begin = L.tail_tokens ? L.tail_begin : 0;
    d.active_token_count = L.tail_tokens;
    d.queries = queries_device;
    d.output = output_device;
    d.query_token_begin = query_token_begin;
    d.query_count = query_count;
    d.head_dim = a->opt.head_dim;
    d.causal_window = causal_window;
    d.softmax_scale = softmax_scale;
    if (cfkv::seam_paged_attention(&d, stream, false) != CF_OK)  // fixed-width pages: the route never takes them
      throw std::runtime_error("ChromoFold paged attention launch rejected");
  });
}

extern "C" int cf_llama_kv_attention_host(cf_llama_kv_adapter *a, uint32_t layer, const float *queries_host,
                                          float *output_host, uint32_t query_count, uint32_t query_head_count,
                                          uint32_t gqa_group_size, uint32_t query_token_begin, float softmax_scale,
                                          uint32_t causal_window, void *stream) {
  return guarded(a, [&] {
    if (queries_host == nullptr || output_host == nullptr) throw std::invalid_argument("null host attention buffer");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const size_t bytes = static_cast<size_t>(query_count) * query_head_count * a->opt.head_dim * sizeof(float);
    a->host_q.reserve(bytes, 0, s);
    a->host_out.reserve(bytes, 0, s);
    hip_check(hipMemcpyAsync(a->host_q.ptr, queries_host, bytes, hipMemcpyHostToDevice, s), "upload");
    if (cf_llama_kv_attention(a, layer, static_cast<const float *>(a->host_q.ptr), static_cast<float *>(a->host_out.ptr),
                              query_count, query_head_count, gqa_group_size, query_token_begin, softmax_scale,
                              causal_window, stream) != 0)
      throw std::runtime_error(a->last_error.empty() ? "attention failed" : a->last_error);
    hip_check(hipMemcpyAsync(output_host, a->host_out.ptr, bytes, hipMemcpyDeviceToHost, s), "download");
    hip_check(hipStreamSynchronize(s), "stream synchronize");
  });
}

extern "C" int cf_llama_kv_flush(cf_llama_kv_adapter *a, void *stream) {
  return guarded(a, [&] {
    const hipStream_t s = static_cast<hipStream_t>(stream);
    for (Layer &L : a->layers)
      for (uint32_t h = 0; h < a->opt.kv_head_count; ++h) {
        const uint32_t tokens = static_cast<uint32_t>(L.tails[h].k.size() / a->opt.head_dim);
        if (tokens) seal(a, L, h, tokens, s);
      }
  });
}

extern "C" int cf_llama_kv_seq_rm(cf_llama_kv_adapter *a, uint64_t sequence_id) {
  return guarded(a, [&] {
    if (sequence_id != 0) throw std::invalid_argument("current ChromoFold cache supports sequence 0 only");
    reset(a);
  });
}

extern "C" int cf_llama_kv_seq_cp(cf_llama_kv_adapter *a, uint64_t source_id, uint64_t destination_id) {
  return guarded(a, [&] {
    if (source_id == destination_id) return;
    throw std::runtime_error("sequence copy requires the forthcoming shared-page table");
  });
}

extern "C" int cf_llama_kv_seq_shift(cf_llama_kv_adapter *a, uint64_t sequence_id, int32_t delta) {
  return guarded(a, [&] {
    if (sequence_id != 0 || delta != 0) throw std::runtime_error("non-zero context shift is not implemented");
  });
}

extern "C" int cf_llama_kv_clear(cf_llama_kv_adapter *a) {
  return guarded(a, [&] { reset(a); });
}

extern "C" int cf_llama_kv_get_stats(const cf_llama_kv_adapter *a, cf_llama_kv_stats *st) {
  if (a == nullptr || st == nullptr) return -1;
  cf_llama_kv_stats r{};
  r.appended_tokens = a->appended;
  r.sealed_tokens = a->sealed_tokens;
  for (const Layer &L : a->layers) {
    r.sealed_pages += L.pages.size();
    for (const Page &p : L.pages) r.compressed_bytes += p.bytes;
    for (const Tail &t : L.tails) {
      r.active_tokens += t.k.size() / a->opt.head_dim;
      r.dense_active_bytes += (t.k.size() + t.v.size()) * sizeof(float);
    }
  }
  if (r.sealed_pages) r.compressed_bytes += a->shared.cap ? a->shared_boff + 4 * ((static_cast<uint64_t>(a->opt.page_size) *
                                                                                   a->opt.head_dim + kBlock - 1) / kBlock)
                                                          : 0;  // the shared LUT + block offsets, once
  r.descriptor_bytes = r.sealed_pages * sizeof(cf_kv_device_page);
  *st = r;
  return 0;
}

extern "C" const char *cf_llama_kv_last_error(const cf_llama_kv_adapter *a) {
  return a == nullptr ? "invalid ChromoFold KV adapter" : a->last_error.c_str();
}
