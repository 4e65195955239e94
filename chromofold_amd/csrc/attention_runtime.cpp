// attention_runtime.cpp — batched decode attention over caller-held int4 nibble pages (cf_attention_runtime_*).
//
// Reference behaviour followed: include/chromofold/production_attention.h and src/cuda/production_attention.cu —
// config checks of create (:153-162), argument checks, the reference-mode refusal and the counters of execute
// (:173-215), compare's refusal (:217-227), invalidate / counters / last error (:229-246). The attention itself
// (the reference's optimized_decode_kernel, :59-139) is served by the nibble-page split-context kernel with the
// request flags that give the reference's item semantics: two's-complement nibbles, blocks counted per
// (token, KV head) row, no causal bound and an inclusive window bound, NULL pages skipped, one query token.
//
// Differences by design (MI355X build):
//   - all items of a call run in one attention launch plus one merge launch, from a device item table in a
//     runtime-owned workspace grown on demand (the reference allocates and frees a table per call);
//   - items are checked before anything is launched: a NULL query/output, or a NULL page table / active tail with
//     a non-zero count, fails the call (the reference's kernel would read through the NULL pointer);
//   - head_dim must be a multiple of 8 and at most 256, checked at create.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "chromofold/production_attention.h"
#include "nibble_kv.hpp"

struct cf_attention_runtime {
  cf_attention_runtime_config config{};
  mutable std::mutex mutex;
  cf_attention_counters counters{};
  cfnib::AttnRunner runner;
  std::string error;
};

extern "C" cf_attention_runtime *cf_attention_runtime_create(const cf_attention_runtime_config *config) {
  if (!config || !config->layer_count || !config->query_head_count || !config->kv_head_count || !config->head_dim)
    return nullptr;
  if (config->query_head_count != config->kv_head_count * config->gqa_group_size) return nullptr;
  if (!cfnib::head_dim_supported(config->head_dim)) return nullptr;
  try {
    auto *r = new cf_attention_runtime();
    r->config = *config;
    return r;
  } catch (...) {
    return nullptr;
  }
}

extern "C" void cf_attention_runtime_destroy(cf_attention_runtime *runtime, void *stream) {
  if (!runtime) return;
  if (stream) (void)hipStreamSynchronize(static_cast<hipStream_t>(stream));  // launches may still read the workspace
  delete runtime;
}

extern "C" int cf_attention_execute_async(cf_attention_runtime *runtime, const cf_attention_batch_item *items,
                                          uint32_t item_count, void *stream) {
  if (!runtime || !items || !item_count) return -1;
  std::lock_guard<std::mutex> guard(runtime->mutex);
  cf_attention_runtime &r = *runtime;
  if (r.config.mode == CF_ATTENTION_REFERENCE) {
    r.error = "CF_ATTENTION_REFERENCE has no kernel in this library: use CF_ATTENTION_OPTIMIZED";
    ++r.counters.reference_launches;
    return -1;
  }
  try {
    std::vector<cfnib::AttnRequest> reqs(item_count);
    for (uint32_t i = 0; i < item_count; ++i) {
      const cf_attention_batch_item &it = items[i];
      if (!it.query.data || !it.output) throw std::invalid_argument("batch item with a NULL query or output");
      if (it.sealed_page_count && !it.sealed_pages)
        throw std::invalid_argument("batch item with sealed pages but no page table");
      if (it.active_token_count && (!it.active_keys || !it.active_values))
        throw std::invalid_argument("batch item with active tokens but no active keys/values");
      cfnib::AttnRequest &q = reqs[i];
      q.query = it.query;
      q.query.token_count = 1;  // one query token per item; its token stride is never used
      q.output = it.output;
      q.output_type = it.output_type;
      q.o_token_stride = it.output_token_stride_bytes;
      q.o_head_stride = it.output_head_stride_bytes;
      q.o_elem_stride = it.output_element_stride_bytes;
      q.pages = it.sealed_pages;
      q.page_count = it.sealed_page_count;
      q.active_k = it.active_token_count ? it.active_keys : nullptr;
      q.active_v = it.active_token_count ? it.active_values : nullptr;
      q.active_begin = it.active_token_begin;
      q.active_count = it.active_token_count;
      q.query_begin = it.query_token_begin;
      q.window = it.causal_window;
      q.softmax_scale = it.softmax_scale;
      q.block_size = 0;  // read per page
      q.flags = cfnib::kSignedNibbles | cfnib::kOpenWindow | cfnib::kRowBlocks;
    }
    const cfnib::AttnShape sh{r.config.kv_head_count, r.config.query_head_count, r.config.gqa_group_size,
                              r.config.head_dim, r.config.page_size};
    const uint64_t before = r.runner.workspace_bytes();
    std::string err;
    const hipError_t st = r.runner.run(reqs, sh, static_cast<hipStream_t>(stream), err);
    const uint64_t after = r.runner.workspace_bytes();
    if (after != before) {
      ++r.counters.allocation_count;
      ++r.counters.pool_misses;
    } else {
      ++r.counters.pool_hits;
    }
    r.counters.peak_reserved_bytes = std::max(r.counters.peak_reserved_bytes, after);
    if (st != hipSuccess)
      throw std::runtime_error(err.empty() ? std::string("attention launch: ") + hipGetErrorString(st) : err);
    ++r.counters.optimized_launches;
    ++r.counters.decode_launches;
    if (item_count > 1) {
      ++r.counters.grouped_batches;
      r.counters.grouped_items += item_count;
      r.counters.kernel_launches_avoided += item_count - 1;
    }
    r.error.clear();
    return 0;
  } catch (const std::invalid_argument &e) {
    r.error = e.what();
    return -1;
  } catch (const std::exception &e) {
    ++r.counters.cuda_errors;
    r.error = e.what();
    return -1;
  }
}

extern "C" int cf_attention_compare_async(cf_attention_runtime *runtime, const cf_attention_batch_item *,
                                          uint32_t item_count, float max_abs_error, float mean_abs_error, void *) {
  if (!runtime || !item_count || max_abs_error <= 0.0f || mean_abs_error <= 0.0f) return -1;
  std::lock_guard<std::mutex> guard(runtime->mutex);
  runtime->error = "comparison needs reference and optimized output buffers, which this call does not take";
  return -1;
}

extern "C" int cf_attention_invalidate_graphs(cf_attention_runtime *runtime) {
  if (!runtime) return -1;
  std::lock_guard<std::mutex> guard(runtime->mutex);
  ++runtime->counters.graph_invalidations;  // no graphs are captured here: nothing else to drop
  return 0;
}

extern "C" int cf_attention_get_counters(const cf_attention_runtime *runtime, cf_attention_counters *counters) {
  if (!runtime || !counters) return -1;
  std::lock_guard<std::mutex> guard(runtime->mutex);
  *counters = runtime->counters;
  return 0;
}

extern "C" const char *cf_attention_last_error(const cf_attention_runtime *runtime) {
  return runtime ? runtime->error.c_str() : "runtime is null";
}
