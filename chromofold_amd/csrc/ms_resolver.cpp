// ms_resolver.cpp — multi-sequence device page tables over shared, refcounted int4 nibble pages (cf_ms_cuda_*).
//
// Reference behaviour followed: include/chromofold/multisequence_cuda_resolver.h and
// src/cuda/multisequence_cuda_resolver.cu:197-497 — config checks, sequence create/remove/cancel, page
// publication with one logical reference, copy sharing every page (+1 logical reference) and copying the active
// tail, per-item snapshots holding in-flight references until the batch's completion event, reclamation of retired
// pages once no reference of either kind is left, audit and counters.
//
// Differences by design (MI355X build):
//   - a batch runs as ONE split-context attention launch over all items (+ one merge launch) from a device item
//     table; the reference launches one single-thread-per-(head, token) kernel per item;
//   - one completion event per batch (not per item) releases the batch's in-flight references;
//   - copying onto an existing destination releases the destination's old page references (the reference drops
//     the old state without releasing them, which leaves those pages' reference counts too high for its own audit);
//   - shift rewrites the affected device page tables (the reference only bumps a generation, so attention kept
//     reading the old positions) and rejects a shift that would make a position negative;
//   - items must match the config's query head count and head_dim, and page payload/scale pointers must be
//     4-byte aligned with the config's kv_head_count and head_dim (checked at publication).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "chromofold/multisequence_cuda_resolver.h"
#include "nibble_kv.hpp"
#include "page_arena.hpp"

namespace {

using cfnib::DeviceBuffer;

void hip_check(hipError_t e, const char *what) {
  if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

struct ArenaPage {
  uint64_t id = 0;
  uint64_t seal_generation = 0;
  cf_device_page_descriptor descriptor{};
  uint64_t resident_bytes = 0;
  uint32_t holders = 0;
  uint32_t batch_holds = 0;
  bool retired = false;
};

struct PageSpan {
  uint64_t page_id = 0;
  int64_t logical_begin = 0;
};

struct LayerTable {
  std::vector<PageSpan> pages;
  DeviceBuffer table;  // device cf_device_page_descriptor[capacity]
  uint32_t capacity = 0;
  uint64_t table_generation = 0;
  DeviceBuffer active_k, active_v;
  uint32_t active_begin = 0, active_count = 0;
  uint64_t active_generation = 0;
  uint32_t block_size = 0;  // the block size of every page of the layer
  bool vector_only = false;  // mixed block sizes, or payloads not 16-byte aligned: the VALU attention kernel
};

struct SeqRecord {
  int64_t id = 0;
  std::vector<LayerTable> layers;
  uint64_t topology_generation = 1;
  bool dispatchable = true;
};

struct PendingBatch {
  hipEvent_t event = nullptr;
  std::vector<uint64_t> page_ids;  // one entry per in-flight reference taken by the batch
};

bool aligned4(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }
bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

struct cf_ms_cuda_resolver {
  cf_ms_cuda_config config{};
  mutable std::mutex mutex;
  std::map<int64_t, SeqRecord> sequences;
  std::unordered_map<uint64_t, ArenaPage> pages;
  std::vector<PendingBatch> pending;
  uint64_t next_page_id = 1;
  cf_ms_cuda_counters counters{};
  std::string error;
  cfnib::AttnRunner runner;

  uint64_t active_bytes() const { return uint64_t(config.page_size) * config.kv_head_count * config.head_dim * 4u; }

  // Rewrites the layer's device page table from its references (logical begins) — stream ordered.
  void refresh_table(LayerTable &layer, hipStream_t stream) {
    std::vector<cf_device_page_descriptor> host;
    host.reserve(layer.pages.size());
    for (const auto &ref : layer.pages) {
      auto it = pages.find(ref.page_id);
      if (it == pages.end() || it->second.retired) throw std::runtime_error("sequence references unavailable shared page");
      cf_device_page_descriptor d = it->second.descriptor;
      d.token_begin = static_cast<uint32_t>(ref.logical_begin);
      host.push_back(d);
    }
    if (host.size() > layer.capacity) {
      uint32_t cap = std::max<uint32_t>(4u, layer.capacity * 2u);
      while (cap < host.size()) cap *= 2u;
      if (layer.table.ptr) hip_check(hipStreamSynchronize(stream), "page table growth sync");
      hip_check(layer.table.allocate(uint64_t(cap) * sizeof(cf_device_page_descriptor)), "page table allocation");
      layer.capacity = cap;
      ++counters.descriptor_table_rebuilds;
    }
    if (!host.empty())
      hip_check(hipMemcpyAsync(layer.table.ptr, host.data(), host.size() * sizeof(cf_device_page_descriptor),
                               hipMemcpyHostToDevice, stream),
                "publish sequence descriptors");
    ++layer.table_generation;
    ++counters.descriptor_tables_built;
  }

  void drop_logical_ref(uint64_t page_id) {
    auto it = pages.find(page_id);
    if (it == pages.end() || it->second.holders == 0) throw std::runtime_error("page logical reference underflow");
    ArenaPage &p = it->second;
    if (--p.holders == 0) {
      p.retired = true;
      ++counters.pages_retired;
      counters.pending_reclamation_bytes += p.resident_bytes;
      counters.pending_reclamation_bytes_peak =
          std::max(counters.pending_reclamation_bytes_peak, counters.pending_reclamation_bytes);
    }
  }

  void release_sequence(SeqRecord &seq) {
    for (auto &layer : seq.layers)
      for (const auto &ref : layer.pages) drop_logical_ref(ref.page_id);
  }

  void release_in_flight(const std::vector<uint64_t> &ids) {
    for (uint64_t id : ids) {
      auto it = pages.find(id);
      if (it == pages.end() || it->second.batch_holds == 0) throw std::runtime_error("snapshot reference underflow");
      --it->second.batch_holds;
      --counters.in_flight_page_references;
    }
  }
};

extern "C" cf_ms_cuda_resolver *cf_ms_cuda_create(const cf_ms_cuda_config *config) {
  if (!config || !config->layer_count || !config->kv_head_count || !config->query_head_count || !config->head_dim ||
      !config->page_size || !config->gqa_group_size ||
      config->query_head_count != config->kv_head_count * config->gqa_group_size ||
      !cfnib::head_dim_supported(config->head_dim))
    return nullptr;
  try {
    auto r = std::make_unique<cf_ms_cuda_resolver>();
    r->config = *config;
    return r.release();
  } catch (...) {
    return nullptr;
  }
}

extern "C" void cf_ms_cuda_destroy(cf_ms_cuda_resolver *r, void *stream) {
  if (!r) return;
  bool device_state = !r->pending.empty() || r->runner.workspace_bytes();
  for (const auto &[id, seq] : r->sequences)
    for (const auto &l : seq.layers) device_state = device_state || l.table.ptr || l.active_k.ptr;
  if (device_state) (void)hipStreamSynchronize(static_cast<hipStream_t>(stream));  // in-flight batches read them
  for (auto &p : r->pending)
    if (p.event) (void)hipEventDestroy(p.event);
  delete r;
}

extern "C" int cf_ms_cuda_sequence_create(cf_ms_cuda_resolver *r, int64_t sequence_id) {
  if (!r) return -1;
  std::lock_guard<std::mutex> guard(r->mutex);
  try {
    if (r->sequences.count(sequence_id)) throw std::runtime_error("sequence already exists");
    SeqRecord s;
    s.id = sequence_id;
    s.layers.resize(r->config.layer_count);
    r->sequences.emplace(sequence_id, std::move(s));
    r->error.clear();
    return 0;
  } catch (const std::exception &ex) {
    r->error = ex.what();
    return -1;
  }
}

extern "C" int cf_ms_cuda_publish_page_async(cf_ms_cuda_resolver *r, const cf_ms_page_publication *pub, void *stream) {
  if (!r || !pub) return -1;
  std::lock_guard<std::mutex> guard(r->mutex);
  try {
    auto seq = r->sequences.find(pub->sequence_id);
    if (seq == r->sequences.end() || pub->layer >= seq->second.layers.size())
      throw std::runtime_error("publication target is invalid");
    const cf_device_page_descriptor &d = pub->descriptor;
    if (!d.key_payload || !d.value_payload || !d.key_scales || !d.value_scales)
      throw std::runtime_error("publication descriptor is incomplete");
    if (d.kv_head_count != r->config.kv_head_count || d.head_dim != r->config.head_dim || !d.block_size ||
        d.token_count > r->config.page_size)
      throw std::runtime_error("publication descriptor does not match the resolver topology");
    if (!aligned4(d.key_payload) || !aligned4(d.value_payload) || !aligned4(d.key_scales) || !aligned4(d.value_scales))
      throw std::runtime_error("publication descriptor storage is not 4-byte aligned");
    ArenaPage page;
    page.id = r->next_page_id++;
    page.seal_generation = pub->seal_generation;
    page.descriptor = d;
    page.resident_bytes = pub->resident_bytes;
    page.holders = 1;
    r->pages.emplace(page.id, page);
    LayerTable &layer = seq->second.layers[pub->layer];
    const uint32_t bs_before = layer.block_size;
    const bool vector_before = layer.vector_only;
    if (layer.pages.empty()) layer.block_size = d.block_size;
    else if (layer.block_size != d.block_size) layer.vector_only = true;
    if (!aligned16(d.key_payload) || !aligned16(d.value_payload)) layer.vector_only = true;
    layer.pages.push_back({page.id, int64_t(d.token_begin)});
    try {
      r->refresh_table(layer, static_cast<hipStream_t>(stream));
    } catch (...) {
      layer.pages.pop_back();
      layer.block_size = bs_before;
      layer.vector_only = vector_before;
      r->pages.erase(page.id);
      throw;
    }
    ++seq->second.topology_generation;
    ++r->counters.pages_registered;
    r->error.clear();
    return 0;
  } catch (const std::exception &ex) {
    ++r->counters.page_registration_failures;
    r->error = ex.what();
    return -1;
  }
}

extern "C" int cf_ms_cuda_stage_active_async(cf_ms_cuda_resolver *r, int64_t sequence_id, uint32_t layer_index,
                                             uint32_t token_begin, const float *keys, const float *values,
                                             uint32_t token_count, void *stream) {
  if (!r || !keys || !values || !token_count || token_count > r->config.page_size) return -1;
  std::lock_guard<std::mutex> guard(r->mutex);
  try {
    auto seq = r->sequences.find(sequence_id);
    if (seq == r->sequences.end() || layer_index >= seq->second.layers.size())
      throw std::runtime_error("active target is invalid");
    LayerTable &layer = seq->second.layers[layer_index];
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (!layer.active_k.ptr) hip_check(layer.active_k.allocate(r->active_bytes()), "active K allocation");
    if (!layer.active_v.ptr) hip_check(layer.active_v.allocate(r->active_bytes()), "active V allocation");
    const uint64_t used = uint64_t(token_count) * r->config.kv_head_count * r->config.head_dim * sizeof(float);
    hip_check(hipMemcpyAsync(layer.active_k.ptr, keys, used, hipMemcpyDeviceToDevice, s), "stage sequence active K");
    hip_check(hipMemcpyAsync(layer.active_v.ptr, values, used, hipMemcpyDeviceToDevice, s), "stage sequence active V");
    layer.active_begin = token_begin;
    layer.active_count = token_count;
    ++layer.active_generation;
    r->error.clear();
    return 0;
  } catch (const std::exception &ex) {
    ++r->counters.cuda_errors;
    r->error = ex.what();
    return -1;
  }
}

extern "C" int cf_ms_cuda_copy_sequence_async(cf_ms_cuda_resolver *r, int64_t source_id, int64_t destination_id,
                                              void *stream) {
  if (!r || source_id == destination_id) return -1;
  std::lock_guard<std::mutex> guard(r->mutex);
  std::vector<uint64_t> acquired;
  try {
    auto src = r->sequences.find(source_id);
    if (src == r->sequences.end()) throw std::runtime_error("source sequence is missing");
    hipStream_t s = static_cast<hipStream_t>(stream);
    SeqRecord cand;
    cand.id = destination_id;
    cand.layers.resize(r->config.layer_count);
    for (uint32_t li = 0; li < r->config.layer_count; ++li) {
      const LayerTable &from = src->second.layers[li];
      LayerTable &to = cand.layers[li];
      to.pages = from.pages;
      to.block_size = from.block_size;
      to.vector_only = from.vector_only;
      for (const auto &ref : to.pages) {
        ++r->pages.at(ref.page_id).holders;
        acquired.push_back(ref.page_id);
      }
      if (from.active_count) {
        hip_check(to.active_k.allocate(r->active_bytes()), "active K allocation");
        hip_check(to.active_v.allocate(r->active_bytes()), "active V allocation");
        hip_check(hipMemcpyAsync(to.active_k.ptr, from.active_k.ptr, r->active_bytes(), hipMemcpyDeviceToDevice, s),
                  "copy active K");
        hip_check(hipMemcpyAsync(to.active_v.ptr, from.active_v.ptr, r->active_bytes(), hipMemcpyDeviceToDevice, s),
                  "copy active V");
        to.active_begin = from.active_begin;
        to.active_count = from.active_count;
        to.active_generation = from.active_generation + 1u;
        ++r->counters.copy_on_write_tail_copies;
      }
      r->refresh_table(to, s);
    }
    auto old = r->sequences.find(destination_id);
    if (old != r->sequences.end()) {
      hip_check(hipStreamSynchronize(s), "copy destination sync");  // launches may still read its tables
      r->release_sequence(old->second);
      r->sequences.erase(old);
    }
    r->sequences.emplace(destination_id, std::move(cand));
    r->error.clear();
    return 0;
  } catch (const std::exception &ex) {
    for (uint64_t id : acquired) {
      auto it = r->pages.find(id);
      if (it != r->pages.end() && it->second.holders) --it->second.holders;
    }
    ++r->counters.cuda_errors;
    r->error = ex.what();
    return -1;
  }
}

extern "C" int cf_ms_cuda_shift_sequence(cf_ms_cuda_resolver *r, int64_t sequence_id, uint32_t begin, uint32_t end,
                                         int32_t delta) {
  if (!r || end < begin) return -1;
  std::lock_guard<std::mutex> guard(r->mutex);
  try {
    auto seq = r->sequences.find(sequence_id);
    if (seq == r->sequences.end()) throw std::runtime_error("sequence is missing");
    // validate every page first so that a rejected shift changes nothing
    for (const auto &layer : seq->second.layers)
      for (const auto &ref : layer.pages) {
        const int64_t ref_end = ref.logical_begin + r->config.page_size;
        if (ref.logical_begin >= begin && ref_end <= end) {
          if (ref.logical_begin + delta < 0) throw std::runtime_error("shift produces a negative token position");
        } else if (ref.logical_begin < end && ref_end > begin) {
          throw std::runtime_error("shift intersects part of an immutable page");
        }
      }
    bool moved = false;
    for (auto &layer : seq->second.layers) {
      bool layer_moved = false;
      for (auto &ref : layer.pages) {
        const int64_t ref_end = ref.logical_begin + r->config.page_size;
        if (ref.logical_begin >= begin && ref_end <= end && delta != 0) {
          ref.logical_begin += delta;
          layer_moved = true;
        }
      }
      if (layer_moved) {
        r->refresh_table(layer, nullptr);
        moved = true;
      }
    }
    if (moved) hip_check(hipStreamSynchronize(nullptr), "shift table upload");
    ++seq->second.topology_generation;
    r->error.clear();
    return 0;
  } catch (const std::exception &ex) {
    r->error = ex.what();
    return -1;
  }
}

extern "C" int cf_ms_cuda_execute_batch_async(cf_ms_cuda_resolver *r, const cf_ms_batch_item *items,
                                              uint32_t item_count, void *stream) {
  if (!r || !items || !item_count) return -1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  std::lock_guard<std::mutex> guard(r->mutex);
  std::vector<uint64_t> taken;
  try {
    std::vector<cfnib::AttnRequest> reqs(item_count);
    for (uint32_t i = 0; i < item_count; ++i) {
      const cf_ms_batch_item &it = items[i];
      if (cf_device_tensor_validate(&it.query) != 0 || !it.output || !cfnib::scalar_bytes(it.output_type))
        throw std::runtime_error("invalid batch tensor");
      if (it.query.head_count != r->config.query_head_count || it.query.head_dim != r->config.head_dim)
        throw std::runtime_error("batch query topology mismatch");
      auto seq = r->sequences.find(it.sequence_id);
      if (seq == r->sequences.end() || !seq->second.dispatchable)
        throw std::runtime_error("sequence is unavailable for dispatch");
      if (it.layer >= seq->second.layers.size()) throw std::runtime_error("layer out of range");
      const LayerTable &layer = seq->second.layers[it.layer];
      for (const auto &ref : layer.pages) {
        ++r->pages.at(ref.page_id).batch_holds;
        ++r->counters.in_flight_page_references;
        taken.push_back(ref.page_id);
      }
      ++r->counters.snapshots_acquired;
      cfnib::AttnRequest &q = reqs[i];
      q.query = it.query;
      q.output = it.output;
      q.output_type = it.output_type;
      q.o_token_stride = it.output_token_stride_bytes;
      q.o_head_stride = it.output_head_stride_bytes;
      q.o_elem_stride = it.output_element_stride_bytes;
      q.pages = layer.table.as<const cf_device_page_descriptor>();
      q.page_count = static_cast<uint32_t>(layer.pages.size());
      q.active_k = layer.active_count ? layer.active_k.as<const float>() : nullptr;
      q.active_v = layer.active_count ? layer.active_v.as<const float>() : nullptr;
      q.active_begin = layer.active_begin;
      q.active_count = layer.active_count;
      q.query_begin = it.query_token_begin;
      q.window = it.causal_window;
      q.softmax_scale = it.softmax_scale;
      q.block_size = layer.vector_only ? 0u : layer.block_size;
    }
    ++r->counters.server_batches_received;
    r->counters.tokens_per_batch_peak = std::max<uint64_t>(r->counters.tokens_per_batch_peak, item_count);
    const cfnib::AttnShape sh{r->config.kv_head_count, r->config.query_head_count, r->config.gqa_group_size,
                              r->config.head_dim, r->config.page_size};
    std::string err;
    const hipError_t st = r->runner.run(reqs, sh, s, err);
    if (st != hipSuccess)
      throw std::runtime_error(err.empty() ? std::string("multi-sequence attention launch: ") + hipGetErrorString(st)
                                           : err);
    ++r->counters.sequence_attention_launches;
    for (uint32_t i = 0; i < item_count; ++i) {
      if (items[i].query.token_count == 1) ++r->counters.decode_items;
      else ++r->counters.prefill_items;
    }
    PendingBatch pb;
    hip_check(hipEventCreateWithFlags(&pb.event, hipEventDisableTiming), "create batch completion event");
    const hipError_t rec = hipEventRecord(pb.event, s);
    if (rec != hipSuccess) {
      (void)hipEventDestroy(pb.event);
      hip_check(rec, "record batch completion event");
    }
    pb.page_ids = std::move(taken);
    taken.clear();
    r->pending.push_back(std::move(pb));
    ++r->counters.snapshot_release_events;
    ++r->counters.compressed_batches_executed;
    r->error.clear();
    return 0;
  } catch (const std::exception &ex) {
    try {
      r->release_in_flight(taken);
    } catch (...) {
    }
    ++r->counters.cuda_errors;
    r->error = ex.what();
    return -1;
  }
}

extern "C" int cf_ms_cuda_cancel_sequence_async(cf_ms_cuda_resolver *r, int64_t sequence_id, void *) {
  if (!r) return -1;
  std::lock_guard<std::mutex> guard(r->mutex);
  auto seq = r->sequences.find(sequence_id);
  if (seq == r->sequences.end()) return -1;
  seq->second.dispatchable = false;
  ++r->counters.cancellation_requests;
  return 0;
}

extern "C" int cf_ms_cuda_sequence_remove_async(cf_ms_cuda_resolver *r, int64_t sequence_id, void *stream) {
  if (!r) return -1;
  std::lock_guard<std::mutex> guard(r->mutex);
  try {
    auto seq = r->sequences.find(sequence_id);
    if (seq == r->sequences.end()) throw std::runtime_error("sequence is missing");
    hip_check(hipStreamSynchronize(static_cast<hipStream_t>(stream)), "remove sync");  // its tables may be in use
    r->release_sequence(seq->second);
    r->sequences.erase(seq);
    r->error.clear();
    return 0;
  } catch (const std::exception &ex) {
    r->error = ex.what();
    return -1;
  }
}

extern "C" int cf_ms_cuda_reclaim_async(cf_ms_cuda_resolver *r, void *) {
  if (!r) return -1;
  std::lock_guard<std::mutex> guard(r->mutex);
  try {
    for (auto it = r->pending.begin(); it != r->pending.end();) {
      const hipError_t q = hipEventQuery(it->event);
      if (q == hipErrorNotReady) {
        ++it;
        continue;
      }
      hip_check(q, "query batch completion event");
      r->release_in_flight(it->page_ids);
      ++r->counters.snapshots_released;
      (void)hipEventDestroy(it->event);
      it = r->pending.erase(it);
    }
    for (auto it = r->pages.begin(); it != r->pages.end();) {
      if (it->second.retired && it->second.holders == 0 && it->second.batch_holds == 0) {
        r->counters.pending_reclamation_bytes -= it->second.resident_bytes;
        ++r->counters.pages_reclaimed;
        it = r->pages.erase(it);
      } else {
        ++it;
      }
    }
    r->error.clear();
    return 0;
  } catch (const std::exception &ex) {
    ++r->counters.cuda_errors;
    r->error = ex.what();
    return -1;
  }
}

extern "C" int cf_ms_cuda_audit(const cf_ms_cuda_resolver *r) {
  if (!r) return -1;
  std::lock_guard<std::mutex> guard(r->mutex);
  std::unordered_map<uint64_t, uint64_t> observed;
  for (const auto &[id, seq] : r->sequences) {
    if (id != seq.id) return -1;
    for (const auto &layer : seq.layers)
      for (const auto &ref : layer.pages) {
        auto p = r->pages.find(ref.page_id);
        if (p == r->pages.end() || p->second.retired) return -1;
        ++observed[ref.page_id];
      }
  }
  for (const auto &[id, page] : r->pages) {
    auto o = observed.find(id);
    const uint64_t n = o == observed.end() ? 0u : o->second;
    if (!page.retired && page.holders != n) return -1;
    if (page.retired && (page.holders != 0 || n != 0)) return -1;
  }
  return r->counters.cross_sequence_contamination == 0 && r->counters.dense_fallback_launches == 0 ? 0 : -1;
}

extern "C" int cf_ms_cuda_get_counters(const cf_ms_cuda_resolver *r, cf_ms_cuda_counters *counters) {
  if (!r || !counters) return -1;
  std::lock_guard<std::mutex> guard(r->mutex);
  *counters = r->counters;
  return 0;
}

extern "C" const char *cf_ms_cuda_last_error(const cf_ms_cuda_resolver *r) {
  return r ? r->error.c_str() : "null multi-sequence CUDA resolver";
}
