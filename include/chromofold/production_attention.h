/* production_attention.h — batched decode attention over caller-held int4 nibble pages: one request per batch
 * item, each with its own page table, active fp32 tail, query view and output view.
 *
 * Drop-in for reference include/chromofold/production_attention.h (mode :11-14, tuning :16-24, config :26-38,
 * batch item :40-58, counters :60-87, entry points :89-105): struct layouts and signatures are the reference's.
 * cf_attention_runtime_create returns NULL for an invalid config; the other calls return 0 on success and -1 on
 * failure, with the message in cf_attention_last_error.
 *
 * Semantics of cf_attention_execute_async (reference src/cuda/production_attention.cu:59-139, kept exactly):
 *   - one query token per item: query head h reads query.data + h * query.head_stride_bytes
 *     + d * query.element_stride_bytes (query.token_count and token_stride_bytes are not read), scalar type
 *     query.scalar_type (F16 / BF16, anything else read as F32); the output row goes to
 *     output + h * output_head_stride_bytes + d * output_element_stride_bytes in output_type (same rule);
 *   - query head h reads KV head h / gqa_group_size;
 *   - a page's K (and V) values are [token][kv_head_count][head_dim] (the config's KV heads and head_dim), two
 *     per byte with the even index in the low nibble, each a TWO'S-COMPLEMENT int4 (nibble n is n for n < 8,
 *     n - 16 otherwise) times the scale of its block; blocks are counted per (token, KV head) row:
 *     scale index = (token * kv_head_count + kv_head) * ceil(page.head_dim / page.block_size) + d / block_size;
 *   - a page with a NULL payload or scale pointer is skipped (so is one with block_size 0 here);
 *   - token at absolute position p (page token_begin + index, or active_token_begin + index) is attended unless
 *     causal_window > 0 and p + causal_window < query_token_begin: there is NO upper (causal) bound, and the
 *     window bound is inclusive — unlike the sealed-page dataplane and resolver (p <= q and p + w > q);
 *   - sealed pages in table order, then the active tail (fp32 [token][kv_head_count][head_dim]); softmax with the
 *     score times softmax_scale; a row with nothing attended is written as zeros.
 *   - sequence_id and layer are not read.
 * CF_ATTENTION_REFERENCE mode has no kernel (the call fails and counts a reference launch), as in the reference;
 * cf_attention_compare_async validates its arguments and fails, as in the reference.
 *
 * MI355X build: every item of a call runs from one device item table in at most three launches (the reference:
 * one 32-thread block per (item, query head) reading K and V once per query head): with head_dim 128, a
 * matrix-core kernel reads every page whose payloads are 16-byte aligned, whose block_size is a multiple of 32 and
 * which holds at most page_size tokens; a VALU kernel reads the other pages (each page is tested on the device by
 * both kernels, so the host never reads the page table) and the active tail; a merge kernel combines the
 * context splits. head_dim must be a multiple of 8 and at most 256 (create returns NULL otherwise); payload and scale
 * pointers must be 4-byte aligned. The item table and split partials live in a runtime-owned device workspace
 * grown on demand (allocation_count / pool_* count its growth); calls on one runtime must be ordered on one stream.
 * The tuning fields, cuda_device, use_async_allocator and block_size are accepted and not used; page_size only
 * sets the page length the matrix-core kernel plans for (longer pages go to the VALU kernel).
 */
#ifndef CHROMOFOLD_PRODUCTION_ATTENTION_H
#define CHROMOFOLD_PRODUCTION_ATTENTION_H

#include <stdint.h>

#include "chromofold/device_kv_seal_attention.h"
#include "chromofold/multisequence_cuda_resolver.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef enum cf_attention_kernel_mode {
  CF_ATTENTION_REFERENCE = 0,
  CF_ATTENTION_OPTIMIZED = 1
} cf_attention_kernel_mode;

typedef struct cf_attention_tuning {
  uint32_t threads_per_block;
  uint32_t warps_per_block;
  uint32_t heads_per_block;
  uint32_t pages_per_work_unit;
  uint32_t vector_width;
  uint32_t enable_cuda_graphs;
  uint32_t enable_async_sealing;
} cf_attention_tuning;

typedef struct cf_attention_runtime_config {
  uint32_t layer_count;
  uint32_t query_head_count;
  uint32_t kv_head_count;
  uint32_t head_dim;
  uint32_t page_size;
  uint32_t block_size;
  uint32_t gqa_group_size;
  uint32_t cuda_device;
  uint32_t use_async_allocator;
  cf_attention_kernel_mode mode;
  cf_attention_tuning tuning;
} cf_attention_runtime_config;

/* One decode request; every pointer is device memory (sealed_pages is a device array of descriptors). */
typedef struct cf_attention_batch_item {
  int64_t sequence_id;
  uint32_t layer;
  cf_device_tensor_view query;
  void *output;
  uint32_t output_type;
  uint64_t output_token_stride_bytes;
  uint64_t output_head_stride_bytes;
  uint64_t output_element_stride_bytes;
  uint32_t query_token_begin;
  float softmax_scale;
  uint32_t causal_window;
  const cf_device_page_descriptor *sealed_pages;
  uint32_t sealed_page_count;
  const float *active_keys;
  const float *active_values;
  uint32_t active_token_begin;
  uint32_t active_token_count;
} cf_attention_batch_item;

typedef struct cf_attention_counters {
  uint64_t reference_launches;
  uint64_t optimized_launches;
  uint64_t decode_launches;
  uint64_t prefill_launches;
  uint64_t grouped_batches;
  uint64_t grouped_items;
  uint64_t kernel_launches_avoided;
  uint64_t graph_captures;
  uint64_t graph_replays;
  uint64_t graph_invalidations;
  uint64_t graph_replay_failures;
  uint64_t async_seal_submissions;
  uint64_t async_seal_overlaps;
  uint64_t descriptor_bytes_read;
  uint64_t compressed_payload_bytes_read;
  uint64_t scale_bytes_read;
  uint64_t allocation_count;
  uint64_t pool_hits;
  uint64_t pool_misses;
  uint64_t peak_reserved_bytes;
  uint64_t peak_live_bytes;
  uint64_t numerical_failures;
  uint64_t cross_sequence_contamination;
  uint64_t dense_fallback_launches;
  uint64_t cuda_errors;
} cf_attention_counters;

typedef struct cf_attention_runtime cf_attention_runtime;

/* reference production_attention.h:89 */
cf_attention_runtime *cf_attention_runtime_create(const cf_attention_runtime_config *config);
/* reference production_attention.h:90; waits for `stream` (when not NULL) before freeing the workspace */
void cf_attention_runtime_destroy(cf_attention_runtime *runtime, void *stream);
/* reference production_attention.h:91-94 */
int cf_attention_execute_async(cf_attention_runtime *runtime, const cf_attention_batch_item *items,
                               uint32_t item_count, void *stream);
/* reference production_attention.h:95-100 */
int cf_attention_compare_async(cf_attention_runtime *runtime, const cf_attention_batch_item *items,
                               uint32_t item_count, float max_abs_error, float mean_abs_error, void *stream);
/* reference production_attention.h:101 */
int cf_attention_invalidate_graphs(cf_attention_runtime *runtime);
/* reference production_attention.h:102 */
int cf_attention_get_counters(const cf_attention_runtime *runtime, cf_attention_counters *counters);
/* reference production_attention.h:103 */
const char *cf_attention_last_error(const cf_attention_runtime *runtime);

#ifdef __cplusplus
}
#endif

#endif /* CHROMOFOLD_PRODUCTION_ATTENTION_H */
