/* device_kv_seal_attention.h — transactional device sealing of fp32 active pages into int4 nibble pages, and
 * attention over them.
 *
 * Drop-in for reference include/chromofold/device_kv_seal_attention.h (states :11-19, fault points :21-33,
 * cf_device_page_descriptor :35-50 (88 B), counters :52-82, config :84-93, entry points :97-121). Functions return
 * 0 on success and -1 on failure (message in cf_device_seal_last_error); cf_device_seal_create returns NULL for an
 * invalid config.
 *
 * Page format (reference src/cuda/device_kv_seal_attention.cu:80-113): the page's K (and V) values, flattened as
 * [token][kv_head][dim], are cut into blocks of block_size values; each block has scale = absmax / 7 (1 when the
 * block is all zero); value i is stored as the 4-bit symbol clamp(rint(x / scale), -8, 7) + 8, two per byte, even
 * index in the low nibble. Decoded value = (symbol - 8) * scale[i / block_size].
 *
 * Transaction (reference :244-334): ACTIVE_FULL -> VALIDATING -> QUANTIZING -> PACKING -> PUBLISHING ->
 * ACTIVE_FILLING. A failure at any step (a page holding NaN/Inf, a device error, or the injected fault point)
 * publishes nothing and returns the layer to ACTIVE_FULL with its active page intact.
 *
 * MI355X build: pages live in slabs of a per-engine device arena (no allocation per page; slots of failed seals
 * are reused); the finite scan, block scales, quantisation and packing run as two kernels with one stream
 * synchronisation; attention is one batched split-context kernel plus a merge over the layer's page table.
 * The active page is fp32 [page_size, kv_head_count, head_dim]; head_dim must be a multiple of 8, at most 256.
 */
#ifndef CHROMOFOLD_DEVICE_KV_SEAL_ATTENTION_H
#define CHROMOFOLD_DEVICE_KV_SEAL_ATTENTION_H

#include <stdint.h>

#include "chromofold/device_kv_dataplane.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef enum cf_device_seal_state {
  CF_SEAL_ACTIVE_FILLING = 0,
  CF_SEAL_ACTIVE_FULL = 1,
  CF_SEAL_VALIDATING = 2,
  CF_SEAL_QUANTIZING = 3,
  CF_SEAL_PACKING = 4,
  CF_SEAL_PUBLISHING = 5,
  CF_SEAL_FAILED = 6,
} cf_device_seal_state;

typedef enum cf_device_seal_fault {
  CF_SEAL_FAULT_NONE = 0,
  CF_SEAL_FAULT_CANDIDATE_ALLOC = 1,
  CF_SEAL_FAULT_FINITE_VALIDATION = 2,
  CF_SEAL_FAULT_SCALE_ALLOC = 3,
  CF_SEAL_FAULT_QUANTIZE_LAUNCH = 4,
  CF_SEAL_FAULT_PAYLOAD_ALLOC = 5,
  CF_SEAL_FAULT_PACK_LAUNCH = 6,
  CF_SEAL_FAULT_DESCRIPTOR_VALIDATE = 7,
  CF_SEAL_FAULT_PAGE_TABLE_GROW = 8,
  CF_SEAL_FAULT_DESCRIPTOR_PUBLISH = 9,
  CF_SEAL_FAULT_ACTIVE_REPLACEMENT = 10,
} cf_device_seal_fault;

/* One sealed page (all KV heads of token_count tokens). Payloads hold ceil(values / 2) bytes, scale arrays
 * blocks_per_page floats, values = token_count * kv_head_count * head_dim. */
typedef struct cf_device_page_descriptor {
  const uint8_t *key_payload;
  const uint8_t *value_payload;
  const float *key_scales;
  const float *value_scales;
  uint32_t token_begin;
  uint32_t token_count;
  uint32_t kv_head_count;
  uint32_t head_dim;
  uint32_t block_size;
  uint32_t blocks_per_page;
  uint64_t key_payload_bytes;
  uint64_t value_payload_bytes;
  uint64_t resident_bytes;
  uint64_t generation;
} cf_device_page_descriptor;

typedef struct cf_device_seal_counters {
  uint64_t seal_attempts;
  uint64_t seal_successes;
  uint64_t seal_failures;
  uint64_t finite_validation_launches;
  uint64_t values_scanned;
  uint64_t nan_values;
  uint64_t inf_values;
  uint64_t invalid_pages_rejected;
  uint64_t quantization_launches;
  uint64_t values_quantized;
  uint64_t saturation_count;
  uint64_t packing_launches;
  uint64_t symbols_packed;
  uint64_t payload_bytes_written;
  uint64_t descriptor_validations;
  uint64_t descriptor_publications;
  uint64_t page_table_reallocations;
  uint64_t page_table_generation;
  uint64_t compressed_attention_launches;
  uint64_t sealed_pages_consumed;
  uint64_t sealed_values_consumed;
  uint64_t active_values_consumed;
  uint64_t query_conversion_launches;
  uint64_t output_conversion_launches;
  uint64_t cuda_errors;
  uint64_t compressed_bytes;
  uint64_t descriptor_bytes;
  uint64_t workspace_bytes;
  uint64_t peak_owned_bytes;
} cf_device_seal_counters;

typedef struct cf_device_seal_config {
  uint32_t layer_count;
  uint32_t kv_head_count;
  uint32_t query_head_count;
  uint32_t head_dim;
  uint32_t page_size;
  uint32_t gqa_group_size;
  uint32_t block_size;
  uint32_t use_async_allocator;
} cf_device_seal_config;

typedef struct cf_device_seal_engine cf_device_seal_engine;

cf_device_seal_engine *cf_device_seal_create(const cf_device_seal_config *config);
void cf_device_seal_destroy(cf_device_seal_engine *engine, void *stream);
/* Replaces the layer's active page with token_count tokens (device fp32 [token_count, kv_heads, head_dim]). */
int cf_device_seal_stage_active_page(cf_device_seal_engine *engine, uint32_t layer, uint32_t token_begin,
                                     const float *active_k, const float *active_v, uint32_t token_count, void *stream);
/* Seals the layer's full active page (the transaction above). Synchronises `stream` once. */
int cf_device_seal_full_page_async(cf_device_seal_engine *engine, uint32_t layer, void *stream);
/* Attention of `query` (query_head_count heads) over the layer's sealed pages and active page; output element
 * (t, h, d) at byte offset t * output_token_stride + h * output_head_stride + d * output_element_stride, of
 * output_scalar_type. Key position p is used by query token t when p <= query_token_begin + t and, with a
 * window w > 0, p + w > query_token_begin + t. */
int cf_device_seal_attention_async(cf_device_seal_engine *engine, uint32_t layer, const cf_device_tensor_view *query,
                                   void *output, uint32_t output_scalar_type, uint64_t output_token_stride_bytes,
                                   uint64_t output_head_stride_bytes, uint64_t output_element_stride_bytes,
                                   uint32_t query_token_begin, float softmax_scale, uint32_t causal_window,
                                   void *stream);
int cf_device_seal_clear_async(cf_device_seal_engine *engine, void *stream);
int cf_device_seal_set_fault(cf_device_seal_engine *engine, uint32_t fault);
int cf_device_seal_get_state(const cf_device_seal_engine *engine, uint32_t layer, uint32_t *state);
int cf_device_seal_get_counters(const cf_device_seal_engine *engine, cf_device_seal_counters *counters);
const char *cf_device_seal_last_error(const cf_device_seal_engine *engine);

/* ADDITIVE (no counterpart in the reference): copies the layer's published page descriptors (device pointers
 * into the engine's arena, valid until clear/destroy) into `out` (capacity entries) and stores the layer's page
 * count in *count. Lets a caller hand sealed pages to cf_ms_cuda_publish_page_async. */
int cf_device_seal_get_pages(const cf_device_seal_engine *engine, uint32_t layer, cf_device_page_descriptor *out,
                             uint32_t capacity, uint32_t *count);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* CHROMOFOLD_DEVICE_KV_SEAL_ATTENTION_H */
