// seal_engine.cpp — the device seal engine (cf_device_seal_*) and the device KV dataplane (cf_device_kv_*,
// cf_device_tensor_validate) over int4 nibble pages.
//
// Reference behaviour followed: include/chromofold/device_kv_seal_attention.h and
// src/cuda/device_kv_seal_attention.cu:196-373 (config checks, the seal transaction with its states, fault points
// and rollback, attention argument checks, counters); include/chromofold/device_kv_dataplane.h and
// src/cuda/device_kv_dataplane.cu:111-247 (view validation, append checks and dtype conversion).
//
// Differences by design (MI355X build):
//   - pages are slots of a device arena (slabs that never move) instead of four allocations per page; the slot of a
//     failed seal is reused, and clear returns every slot to the arena instead of freeing it;
//   - the K and V finite scans and block scales run as ONE launch, quantisation and packing of both streams as ONE
//     more (the launch counters count these launches); the one stream synchronisation stays between them, so a page
//     holding NaN/Inf is rejected before anything is quantised, as in the reference;
//   - the layer's page table grows by doubling and each seal uploads only the new descriptor;
//   - attention is the batched split-context kernel of nibble_kv.hip;
//   - head_dim must be a multiple of 8 and at most 256 (create fails otherwise);
//   - the dataplane is connected: its seal and attention entry points work (the reference's always fail), on an
//     internal engine with block_size 32.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "chromofold/device_kv_dataplane.h"
#include "chromofold/device_kv_seal_attention.h"
#include "nibble_kv.hpp"
#include "page_arena.hpp"

namespace {

using cfnib::DeviceBuffer;

struct HipError : std::runtime_error {
  using std::runtime_error::runtime_error;
};

void hip_check(hipError_t e, const char *what) {
  if (e != hipSuccess) throw HipError(std::string(what) + ": " + hipGetErrorString(e));
}

struct SealLayer {
  DeviceBuffer active_k, active_v;
  uint32_t active_begin = 0, active_count = 0;
  uint32_t state = CF_SEAL_ACTIVE_FILLING;
  std::vector<cf_device_page_descriptor> pages;
  std::vector<char *> slots;
  DeviceBuffer table;  // device cf_device_page_descriptor[capacity]
  uint32_t capacity = 0;
  uint64_t generation = 0;
};

// Pinned host memory for the status read-back (allocated once).
struct PinnedStatus {
  cfnib::SealStatus *p = nullptr;
  ~PinnedStatus() {
    if (p) (void)hipHostFree(p);
  }
};

bool seal_config_ok(const cf_device_seal_config &c) {
  return c.layer_count && c.kv_head_count && c.query_head_count && c.head_dim && c.page_size && c.block_size &&
         c.query_head_count == c.kv_head_count * c.gqa_group_size && cfnib::head_dim_supported(c.head_dim) &&
         uint64_t(c.page_size) * c.kv_head_count * c.head_dim < (uint64_t(1) << 31);
}

}  // namespace

struct cf_device_seal_engine {
  cf_device_seal_config config{};
  std::vector<SealLayer> layers;
  cf_device_seal_counters counters{};
  uint32_t fault = CF_SEAL_FAULT_NONE;
  std::string error;
  cfnib::PageArena arena;
  DeviceBuffer status;  // one SealStatus
  PinnedStatus host_status;
  cfnib::AttnRunner runner;

  uint32_t values() const { return config.page_size * config.kv_head_count * config.head_dim; }
  uint32_t blocks() const { return (values() + config.block_size - 1u) / config.block_size; }
  uint64_t payload_bytes() const { return (uint64_t(values()) + 1u) / 2u; }
  static uint64_t a256(uint64_t b) { return (b + 255u) & ~uint64_t(255); }
  // slot layout: K payload | V payload | K scales | V scales, each 256-byte aligned
  uint64_t slot_bytes() const { return 2 * a256(payload_bytes()) + 2 * a256(uint64_t(blocks()) * 4u); }

  void refresh_owned() {
    counters.descriptor_bytes = 0;
    for (const auto &l : layers) counters.descriptor_bytes += l.table.bytes;
    counters.workspace_bytes = runner.workspace_bytes() + status.bytes;
    counters.peak_owned_bytes = std::max(counters.peak_owned_bytes,
                                         counters.compressed_bytes + counters.descriptor_bytes + counters.workspace_bytes);
  }
};

namespace {

// Allocates the layer's fp32 active page once.
void ensure_active(cf_device_seal_engine *e, SealLayer &layer) {
  const uint64_t bytes = uint64_t(e->values()) * sizeof(float);
  if (!layer.active_k.ptr) hip_check(layer.active_k.allocate(bytes), "active K allocation");
  if (!layer.active_v.ptr) hip_check(layer.active_v.allocate(bytes), "active V allocation");
}

int seal_layer(cf_device_seal_engine *e, uint32_t layer_index, hipStream_t stream) {
  SealLayer &layer = e->layers[layer_index];
  e->counters.seal_attempts++;
  if (layer.active_count != e->config.page_size || layer.state != CF_SEAL_ACTIVE_FULL) {
    e->error = "layer does not contain a full active page";
    e->counters.seal_failures++;
    return -1;
  }
  char *slot = nullptr;
  try {
    auto inject = [&](uint32_t point) {
      if (e->fault == point) throw std::runtime_error("injected transactional seal failure");
    };
    const uint32_t values = e->values();
    const uint32_t blocks = e->blocks();
    const uint64_t payload = e->payload_bytes();
    inject(CF_SEAL_FAULT_CANDIDATE_ALLOC);
    hip_check(e->arena.acquire(&slot), "page arena");
    uint8_t *kp = reinterpret_cast<uint8_t *>(slot);
    uint8_t *vp = kp + cf_device_seal_engine::a256(payload);
    float *ks = reinterpret_cast<float *>(vp + cf_device_seal_engine::a256(payload));
    float *vs = reinterpret_cast<float *>(reinterpret_cast<char *>(ks) + cf_device_seal_engine::a256(uint64_t(blocks) * 4u));
    if (!e->status.ptr) hip_check(e->status.allocate(sizeof(cfnib::SealStatus)), "status allocation");
    if (!e->host_status.p)
      hip_check(hipHostMalloc(reinterpret_cast<void **>(&e->host_status.p), sizeof(cfnib::SealStatus)),
                "pinned status allocation");
    auto *status = e->status.as<cfnib::SealStatus>();

    layer.state = CF_SEAL_VALIDATING;
    hip_check(cfnib::launch_clear_status(status, 1, stream), "clear seal status");
    hip_check(cfnib::launch_block_scales(layer.active_k.as<float>(), layer.active_v.as<float>(), values,
                                         e->config.block_size, ks, vs, status, stream),
              "finite validation launch");
    e->counters.finite_validation_launches++;
    e->counters.values_scanned += uint64_t(values) * 2u;
    inject(CF_SEAL_FAULT_FINITE_VALIDATION);
    hip_check(hipMemcpyAsync(e->host_status.p, status, sizeof(cfnib::SealStatus), hipMemcpyDeviceToHost, stream),
              "read finite counters");
    hip_check(hipStreamSynchronize(stream), "finite validation sync");
    const cfnib::SealStatus st = *e->host_status.p;
    e->counters.nan_values += st.nan_values;
    e->counters.inf_values += st.inf_values;
    if (st.nan_values || st.inf_values) {
      e->counters.invalid_pages_rejected++;
      throw std::runtime_error("active page contains NaN or Inf");
    }

    layer.state = CF_SEAL_QUANTIZING;
    inject(CF_SEAL_FAULT_SCALE_ALLOC);
    hip_check(cfnib::launch_pack(layer.active_k.as<float>(), layer.active_v.as<float>(), values, e->config.block_size,
                                 ks, vs, kp, vp, status, stream),
              "int4 quantization launch");
    e->counters.quantization_launches++;
    e->counters.values_quantized += uint64_t(values) * 2u;
    inject(CF_SEAL_FAULT_QUANTIZE_LAUNCH);

    layer.state = CF_SEAL_PACKING;  // the quantisation launch packs as it goes
    inject(CF_SEAL_FAULT_PAYLOAD_ALLOC);
    e->counters.packing_launches++;
    e->counters.symbols_packed += uint64_t(values) * 2u;
    e->counters.payload_bytes_written += payload * 2u;
    inject(CF_SEAL_FAULT_PACK_LAUNCH);

    cf_device_page_descriptor d{};
    d.key_payload = kp;
    d.value_payload = vp;
    d.key_scales = ks;
    d.value_scales = vs;
    d.token_begin = layer.active_begin;
    d.token_count = layer.active_count;
    d.kv_head_count = e->config.kv_head_count;
    d.head_dim = e->config.head_dim;
    d.block_size = e->config.block_size;
    d.blocks_per_page = blocks;
    d.key_payload_bytes = payload;
    d.value_payload_bytes = payload;
    d.resident_bytes = 2u * payload + 2u * uint64_t(blocks) * sizeof(float);
    d.generation = layer.generation + 1u;
    e->counters.descriptor_validations++;
    inject(CF_SEAL_FAULT_DESCRIPTOR_VALIDATE);

    layer.state = CF_SEAL_PUBLISHING;
    const uint32_t needed = static_cast<uint32_t>(layer.pages.size() + 1u);
    if (needed > layer.capacity) {
      inject(CF_SEAL_FAULT_PAGE_TABLE_GROW);
      uint32_t next = std::max<uint32_t>(4u, layer.capacity * 2u);
      while (next < needed) next *= 2u;
      DeviceBuffer grown;
      hip_check(grown.allocate(uint64_t(next) * sizeof(cf_device_page_descriptor)), "page table growth");
      if (!layer.pages.empty())
        hip_check(hipMemcpyAsync(grown.ptr, layer.table.ptr, layer.pages.size() * sizeof(cf_device_page_descriptor),
                                 hipMemcpyDeviceToDevice, stream),
                  "page table copy");
      hip_check(hipStreamSynchronize(stream), "page table growth sync");  // earlier launches may read the old table
      layer.table = std::move(grown);
      layer.capacity = next;
      e->counters.page_table_reallocations++;
    }
    inject(CF_SEAL_FAULT_ACTIVE_REPLACEMENT);
    inject(CF_SEAL_FAULT_DESCRIPTOR_PUBLISH);
    layer.pages.push_back(d);
    layer.slots.push_back(slot);
    slot = nullptr;  // owned by the layer from here on
    hip_check(hipMemcpyAsync(layer.table.as<cf_device_page_descriptor>() + (layer.pages.size() - 1u),
                             &layer.pages.back(), sizeof(cf_device_page_descriptor), hipMemcpyHostToDevice, stream),
              "publish descriptor");
    layer.active_begin += layer.active_count;
    layer.active_count = 0;
    layer.generation++;
    layer.state = CF_SEAL_ACTIVE_FILLING;
    e->counters.descriptor_publications++;
    e->counters.page_table_generation = layer.generation;
    e->counters.seal_successes++;
    e->counters.compressed_bytes += d.resident_bytes;
    e->refresh_owned();
    e->error.clear();
    return 0;
  } catch (const std::exception &ex) {
    layer.state = CF_SEAL_ACTIVE_FULL;
    e->error = ex.what();
    e->counters.seal_failures++;
    if (dynamic_cast<const HipError *>(&ex)) e->counters.cuda_errors++;
    e->arena.release(slot);
    return -1;
  }
}

int engine_attention(cf_device_seal_engine *e, uint32_t layer_index, const cf_device_tensor_view *query, void *output,
                     uint32_t output_type, uint64_t ots, uint64_t ohs, uint64_t oes, uint32_t query_begin,
                     float softmax_scale, uint32_t window, hipStream_t stream) {
  try {
    SealLayer &layer = e->layers[layer_index];
    if (query->head_count != e->config.query_head_count || query->head_dim != e->config.head_dim)
      throw std::runtime_error("query topology mismatch");
    if (ots < uint64_t(query->head_count - 1u) * ohs + uint64_t(query->head_dim - 1u) * oes +
                  cfnib::scalar_bytes(output_type))
      throw std::runtime_error("output stride is too small");
    cfnib::AttnRequest r{};
    r.query = *query;
    r.output = output;
    r.output_type = output_type;
    r.o_token_stride = ots;
    r.o_head_stride = ohs;
    r.o_elem_stride = oes;
    r.pages = layer.table.as<const cf_device_page_descriptor>();
    r.page_count = static_cast<uint32_t>(layer.pages.size());
    r.active_k = layer.active_count ? layer.active_k.as<const float>() : nullptr;
    r.active_v = layer.active_count ? layer.active_v.as<const float>() : nullptr;
    r.active_begin = layer.active_begin;
    r.active_count = layer.active_count;
    r.query_begin = query_begin;
    r.window = window;
    r.softmax_scale = softmax_scale;
    r.block_size = e->config.block_size;
    const cfnib::AttnShape sh{e->config.kv_head_count, e->config.query_head_count, e->config.gqa_group_size,
                              e->config.head_dim, e->config.page_size};
    std::string err;
    const hipError_t st = e->runner.run({r}, sh, stream, err);
    if (st != hipSuccess) throw HipError(err.empty() ? std::string("compressed attention launch: ") + hipGetErrorString(st) : err);
    e->counters.compressed_attention_launches++;
    e->counters.sealed_pages_consumed += layer.pages.size();
    for (const auto &p : layer.pages)
      e->counters.sealed_values_consumed += uint64_t(p.token_count) * e->config.kv_head_count * e->config.head_dim * 2u;
    e->counters.active_values_consumed += uint64_t(layer.active_count) * e->config.kv_head_count * e->config.head_dim * 2u;
    if (query->scalar_type != CF_DEVICE_F32) e->counters.query_conversion_launches++;
    if (output_type != CF_DEVICE_F32) e->counters.output_conversion_launches++;
    e->refresh_owned();
    e->error.clear();
    return 0;
  } catch (const std::exception &ex) {
    e->error = ex.what();
    e->counters.cuda_errors++;
    return -1;
  }
}

void engine_clear(cf_device_seal_engine *e, hipStream_t stream) {
  bool device_state = e->arena.reserved_bytes() != 0;
  for (const auto &l : e->layers) device_state = device_state || l.table.ptr;
  if (device_state) (void)hipStreamSynchronize(stream);  // launches in flight may still read the slots and tables
  for (auto &layer : e->layers) {
    for (char *s : layer.slots) e->arena.release(s);
    layer.slots.clear();
    layer.pages.clear();
    layer.table.reset();
    layer.capacity = 0;
    layer.active_begin = layer.active_count = 0;
    layer.state = CF_SEAL_ACTIVE_FILLING;
    layer.generation = 0;
  }
  e->counters.compressed_bytes = 0;
  e->counters.descriptor_bytes = 0;
}

}  // namespace

// ================================================================================================= seal engine
extern "C" cf_device_seal_engine *cf_device_seal_create(const cf_device_seal_config *config) {
  if (!config || !seal_config_ok(*config)) return nullptr;
  try {
    auto e = std::make_unique<cf_device_seal_engine>();
    e->config = *config;
    e->layers.resize(config->layer_count);
    e->arena.set_slot_bytes(e->slot_bytes());
    return e.release();
  } catch (...) {
    return nullptr;
  }
}

extern "C" void cf_device_seal_destroy(cf_device_seal_engine *e, void *stream) {
  if (!e) return;
  bool device_state = e->status.ptr || e->arena.reserved_bytes() || e->runner.workspace_bytes();
  for (const auto &l : e->layers) device_state = device_state || l.active_k.ptr || l.table.ptr;
  if (device_state) (void)hipStreamSynchronize(static_cast<hipStream_t>(stream));  // in-flight work reads it
  delete e;
}

extern "C" int cf_device_seal_stage_active_page(cf_device_seal_engine *e, uint32_t layer_index, uint32_t token_begin,
                                                const float *k, const float *v, uint32_t token_count, void *stream) {
  if (!e || layer_index >= e->layers.size() || !k || !v || !token_count || token_count > e->config.page_size) return -1;
  try {
    SealLayer &layer = e->layers[layer_index];
    ensure_active(e, layer);
    const uint64_t used = uint64_t(token_count) * e->config.kv_head_count * e->config.head_dim * sizeof(float);
    hipStream_t s = static_cast<hipStream_t>(stream);
    hip_check(hipMemcpyAsync(layer.active_k.ptr, k, used, hipMemcpyDeviceToDevice, s), "stage active K");
    hip_check(hipMemcpyAsync(layer.active_v.ptr, v, used, hipMemcpyDeviceToDevice, s), "stage active V");
    layer.active_begin = token_begin;
    layer.active_count = token_count;
    layer.state = token_count == e->config.page_size ? CF_SEAL_ACTIVE_FULL : CF_SEAL_ACTIVE_FILLING;
    e->error.clear();
    return 0;
  } catch (const std::exception &ex) {
    e->error = ex.what();
    e->counters.cuda_errors++;
    return -1;
  }
}

extern "C" int cf_device_seal_full_page_async(cf_device_seal_engine *e, uint32_t layer_index, void *stream) {
  if (!e || layer_index >= e->layers.size()) return -1;
  return seal_layer(e, layer_index, static_cast<hipStream_t>(stream));
}

extern "C" int cf_device_seal_attention_async(cf_device_seal_engine *e, uint32_t layer_index,
                                              const cf_device_tensor_view *query, void *output, uint32_t output_type,
                                              uint64_t ots, uint64_t ohs, uint64_t oes, uint32_t query_begin,
                                              float softmax_scale, uint32_t window, void *stream) {
  if (!e || layer_index >= e->layers.size() || cf_device_tensor_validate(query) != 0 || !output ||
      !cfnib::scalar_bytes(output_type))
    return -1;
  return engine_attention(e, layer_index, query, output, output_type, ots, ohs, oes, query_begin, softmax_scale,
                          window, static_cast<hipStream_t>(stream));
}

extern "C" int cf_device_seal_clear_async(cf_device_seal_engine *e, void *stream) {
  if (!e) return -1;
  engine_clear(e, static_cast<hipStream_t>(stream));
  return 0;
}

extern "C" int cf_device_seal_set_fault(cf_device_seal_engine *e, uint32_t fault) {
  if (!e || fault > CF_SEAL_FAULT_ACTIVE_REPLACEMENT) return -1;
  e->fault = fault;
  return 0;
}

extern "C" int cf_device_seal_get_state(const cf_device_seal_engine *e, uint32_t layer, uint32_t *state) {
  if (!e || layer >= e->layers.size() || !state) return -1;
  *state = e->layers[layer].state;
  return 0;
}

extern "C" int cf_device_seal_get_counters(const cf_device_seal_engine *e, cf_device_seal_counters *counters) {
  if (!e || !counters) return -1;
  *counters = e->counters;
  return 0;
}

extern "C" const char *cf_device_seal_last_error(const cf_device_seal_engine *e) {
  return e ? e->error.c_str() : "null seal engine";
}

extern "C" int cf_device_seal_get_pages(const cf_device_seal_engine *e, uint32_t layer,
                                        cf_device_page_descriptor *out, uint32_t capacity, uint32_t *count) {
  if (!e || layer >= e->layers.size() || !count || (capacity && !out)) return -1;
  const auto &pages = e->layers[layer].pages;
  *count = static_cast<uint32_t>(pages.size());
  const size_t n = std::min<size_t>(capacity, pages.size());
  if (n) std::memcpy(out, pages.data(), n * sizeof(cf_device_page_descriptor));
  return 0;
}

// ================================================================================================= dataplane
extern "C" int cf_device_tensor_validate(const cf_device_tensor_view *view) {
  if (!view || !view->data || view->token_count == 0 || view->head_count == 0 || view->head_dim == 0) return -1;
  const uint64_t width = cfnib::scalar_bytes(view->scalar_type);
  if (width == 0 || view->element_stride_bytes < width) return -1;
  const uint64_t head_span = uint64_t(view->head_dim - 1u) * view->element_stride_bytes + width;
  if (view->head_stride_bytes < head_span) return -1;
  if (view->token_stride_bytes < uint64_t(view->head_count - 1u) * view->head_stride_bytes + head_span) return -1;
  return 0;
}

struct cf_device_kv_dataplane {
  cf_device_kv_config config{};
  cf_device_kv_counters counters{};
  std::string error;
  cf_device_seal_engine *engine = nullptr;
  ~cf_device_kv_dataplane() {
    if (engine) cf_device_seal_destroy(engine, nullptr);
  }
  void refresh() {
    const cf_device_seal_counters &s = engine->counters;
    counters.quantization_launches = s.quantization_launches;
    counters.seal_attempts = s.seal_attempts;
    counters.seal_successes = s.seal_successes;
    counters.seal_failures = s.seal_failures;
    counters.descriptor_publications = s.descriptor_publications;
    counters.compressed_attention_launches = s.compressed_attention_launches;
    counters.sealed_values_consumed = s.sealed_values_consumed;
    counters.active_values_consumed = s.active_values_consumed;
    counters.compressed_bytes = s.compressed_bytes;
    counters.descriptor_bytes = s.descriptor_bytes;
    counters.workspace_bytes = s.workspace_bytes;
    counters.active_bytes = 0;
    for (const auto &l : engine->layers) counters.active_bytes += l.active_k.bytes + l.active_v.bytes;
    counters.peak_owned_bytes = std::max(counters.peak_owned_bytes, counters.active_bytes + counters.compressed_bytes +
                                                                        counters.descriptor_bytes +
                                                                        counters.workspace_bytes);
  }
};

extern "C" cf_device_kv_dataplane *cf_device_kv_create(const cf_device_kv_config *config) {
  if (!config || !config->layer_count || !config->kv_head_count || !config->query_head_count || !config->head_dim ||
      !config->page_size || !config->gqa_group_size ||
      config->query_head_count != config->kv_head_count * config->gqa_group_size)
    return nullptr;
  cf_device_seal_config sc{};
  sc.layer_count = config->layer_count;
  sc.kv_head_count = config->kv_head_count;
  sc.query_head_count = config->query_head_count;
  sc.head_dim = config->head_dim;
  sc.page_size = config->page_size;
  sc.gqa_group_size = config->gqa_group_size;
  sc.block_size = 32;
  sc.use_async_allocator = config->use_async_allocator;
  try {
    auto dp = std::make_unique<cf_device_kv_dataplane>();
    dp->config = *config;
    dp->engine = cf_device_seal_create(&sc);
    if (!dp->engine) return nullptr;
    return dp.release();
  } catch (...) {
    return nullptr;
  }
}

extern "C" void cf_device_kv_destroy(cf_device_kv_dataplane *dp, void *stream) {
  if (!dp) return;
  cf_device_seal_destroy(dp->engine, stream);
  dp->engine = nullptr;
  delete dp;
}

extern "C" int cf_device_kv_append_async(cf_device_kv_dataplane *dp, uint32_t layer_index, uint32_t token_begin,
                                         const cf_device_tensor_view *keys, const cf_device_tensor_view *values,
                                         void *stream) {
  if (!dp || layer_index >= dp->config.layer_count || cf_device_tensor_validate(keys) != 0 ||
      cf_device_tensor_validate(values) != 0)
    return -1;
  try {
    if (keys->token_count != values->token_count || keys->head_count != values->head_count ||
        keys->head_dim != values->head_dim || keys->head_count != dp->config.kv_head_count ||
        keys->head_dim != dp->config.head_dim)
      throw std::runtime_error("device K/V topology mismatch");
    SealLayer &layer = dp->engine->layers[layer_index];
    if (layer.active_count != 0 && token_begin != layer.active_begin + layer.active_count)
      throw std::runtime_error("non-contiguous device token append");
    if (layer.active_count + keys->token_count > dp->config.page_size)
      throw std::runtime_error("append crosses active page boundary; seal before retry");
    ensure_active(dp->engine, layer);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (layer.active_count == 0) layer.active_begin = token_begin;
    const uint64_t n = uint64_t(keys->token_count) * keys->head_count * keys->head_dim;
    for (const cf_device_tensor_view *src : {keys, values}) {
      float *dst = (src == keys) ? layer.active_k.as<float>() : layer.active_v.as<float>();
      hip_check(cfnib::launch_convert(*src, dst, layer.active_count, s), "device KV conversion launch");
      if (src->scalar_type == CF_DEVICE_F16) dp->counters.fp16_values_converted += n;
      else if (src->scalar_type == CF_DEVICE_BF16) dp->counters.bf16_values_converted += n;
      else dp->counters.fp32_values_copied += n;
    }
    layer.active_count += keys->token_count;
    layer.state = layer.active_count == dp->config.page_size ? CF_SEAL_ACTIVE_FULL : CF_SEAL_ACTIVE_FILLING;
    dp->counters.device_append_calls++;
    dp->counters.device_values_appended += n * 2u;
    dp->refresh();
    dp->error.clear();
    return 0;
  } catch (const std::exception &ex) {
    dp->error = ex.what();
    dp->counters.cuda_errors++;
    return -1;
  }
}

extern "C" int cf_device_kv_seal_full_pages_async(cf_device_kv_dataplane *dp, void *stream) {
  if (!dp) return -1;
  for (uint32_t i = 0; i < dp->config.layer_count; ++i) {
    if (dp->engine->layers[i].active_count != dp->config.page_size) continue;
    if (seal_layer(dp->engine, i, static_cast<hipStream_t>(stream)) != 0) {
      dp->error = dp->engine->error;
      dp->refresh();
      return -1;
    }
  }
  dp->refresh();
  dp->error.clear();
  return 0;
}

extern "C" int cf_device_kv_attention_async(cf_device_kv_dataplane *dp, uint32_t layer_index, const float *query,
                                            float *output, uint32_t query_token_count, uint32_t query_token_begin,
                                            float softmax_scale, uint32_t causal_window, void *stream) {
  if (!dp || layer_index >= dp->config.layer_count || !query || !output || !query_token_count) return -1;
  const uint32_t qh = dp->config.query_head_count, d = dp->config.head_dim;
  cf_device_tensor_view q{};
  q.data = query;
  q.scalar_type = CF_DEVICE_F32;
  q.token_count = query_token_count;
  q.head_count = qh;
  q.head_dim = d;
  q.element_stride_bytes = 4;
  q.head_stride_bytes = uint64_t(d) * 4u;
  q.token_stride_bytes = uint64_t(qh) * d * 4u;
  const int rc = engine_attention(dp->engine, layer_index, &q, output, CF_DEVICE_F32, q.token_stride_bytes,
                                  q.head_stride_bytes, 4, query_token_begin, softmax_scale, causal_window,
                                  static_cast<hipStream_t>(stream));
  if (rc != 0) {
    dp->error = dp->engine->error;
    dp->counters.cuda_errors++;
  } else {
    dp->error.clear();
  }
  dp->refresh();
  return rc;
}

extern "C" int cf_device_kv_clear_async(cf_device_kv_dataplane *dp, void *stream) {
  if (!dp) return -1;
  engine_clear(dp->engine, static_cast<hipStream_t>(stream));
  dp->refresh();
  return 0;
}

extern "C" int cf_device_kv_get_counters(const cf_device_kv_dataplane *dp, cf_device_kv_counters *counters) {
  if (!dp || !counters) return -1;
  *counters = dp->counters;
  return 0;
}

extern "C" const char *cf_device_kv_last_error(const cf_device_kv_dataplane *dp) {
  return dp ? dp->error.c_str() : "null device KV dataplane";
}
