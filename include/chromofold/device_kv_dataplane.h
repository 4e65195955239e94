/* device_kv_dataplane.h — device tensor views and the single-sequence device KV dataplane.
 *
 * Drop-in for reference include/chromofold/device_kv_dataplane.h (types at :11-61, entry points at :63-89): the
 * scalar-type codes, cf_device_tensor_view (56 B), the config and counter structs and every signature are the
 * reference's. The functions return 0 on success and -1 on failure, with the message in cf_device_kv_last_error.
 *
 * Behind the API (HIP, gfx950): appends convert f16/bf16/f32 strided views into an fp32 active page in one
 * kernel; cf_device_kv_seal_full_pages_async seals every full active page into int4 nibble pages (the same format
 * and kernels as device_kv_seal_attention.h) and cf_device_kv_attention_async runs the batched nibble-page
 * attention kernel. The reference leaves those two unconnected (reference src/cuda/device_kv_dataplane.cu:204-220
 * always fail); here they work, with the same argument checks in front.
 */
#ifndef CHROMOFOLD_DEVICE_KV_DATAPLANE_H
#define CHROMOFOLD_DEVICE_KV_DATAPLANE_H

#include <stdint.h>

#include "chromofold/kv_cuda.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef enum cf_device_scalar_type {
  CF_DEVICE_F16 = 1,
  CF_DEVICE_BF16 = 2,
  CF_DEVICE_F32 = 3,
} cf_device_scalar_type;

/* A strided [token_count, head_count, head_dim] device tensor; strides in bytes. */
typedef struct cf_device_tensor_view {
  const void *data;
  uint32_t scalar_type; /* cf_device_scalar_type */
  uint32_t token_count;
  uint32_t head_count;
  uint32_t head_dim;
  uint64_t token_stride_bytes;
  uint64_t head_stride_bytes;
  uint64_t element_stride_bytes;
  int32_t device_ordinal;
} cf_device_tensor_view;

typedef struct cf_device_kv_config {
  uint32_t layer_count;
  uint32_t kv_head_count;
  uint32_t query_head_count;
  uint32_t head_dim;
  uint32_t page_size;
  uint32_t gqa_group_size;
  uint32_t use_async_allocator;
} cf_device_kv_config;

typedef struct cf_device_kv_counters {
  uint64_t device_append_calls;
  uint64_t device_values_appended;
  uint64_t fp16_values_converted;
  uint64_t bf16_values_converted;
  uint64_t fp32_values_copied;
  uint64_t quantization_launches;
  uint64_t huffman_pack_launches;
  uint64_t seal_attempts;
  uint64_t seal_successes;
  uint64_t seal_failures;
  uint64_t descriptor_publications;
  uint64_t compressed_attention_launches;
  uint64_t sealed_values_consumed;
  uint64_t active_values_consumed;
  uint64_t query_conversion_launches;
  uint64_t output_conversion_launches;
  uint64_t dense_fallback_launches;
  uint64_t cuda_errors;
  uint64_t active_bytes;
  uint64_t compressed_bytes;
  uint64_t descriptor_bytes;
  uint64_t workspace_bytes;
  uint64_t retired_pending_bytes;
  uint64_t peak_owned_bytes;
} cf_device_kv_counters;

typedef struct cf_device_kv_dataplane cf_device_kv_dataplane;

/* 0 when the view is usable: data set, non-zero extents, a known scalar type, and strides that do not overlap
 * (element >= width, head >= span of one head row, token >= span of one token). reference
 * src/cuda/device_kv_dataplane.cu:111-120 */
int cf_device_tensor_validate(const cf_device_tensor_view *view);

cf_device_kv_dataplane *cf_device_kv_create(const cf_device_kv_config *config);
void cf_device_kv_destroy(cf_device_kv_dataplane *dataplane, void *stream);
/* Appends token_count tokens at token_begin to the layer's active page (contiguous with what it holds; the page
 * may not overflow page_size: seal first). */
int cf_device_kv_append_async(cf_device_kv_dataplane *dataplane, uint32_t layer, uint32_t token_begin,
                              const cf_device_tensor_view *keys, const cf_device_tensor_view *values, void *stream);
/* Seals every layer whose active page is full into an int4 nibble page (synchronises the stream once per page to
 * check the page for NaN/Inf before publishing). */
int cf_device_kv_seal_full_pages_async(cf_device_kv_dataplane *dataplane, void *stream);
/* Attention of query [query_token_count, query_head_count, head_dim] (fp32, contiguous) over the layer's sealed
 * pages and active page; output fp32 of the same shape. Causal at query_token_begin + t, optional window. */
int cf_device_kv_attention_async(cf_device_kv_dataplane *dataplane, uint32_t layer, const float *query, float *output,
                                 uint32_t query_token_count, uint32_t query_token_begin, float softmax_scale,
                                 uint32_t causal_window, void *stream);
int cf_device_kv_clear_async(cf_device_kv_dataplane *dataplane, void *stream);
int cf_device_kv_get_counters(const cf_device_kv_dataplane *dataplane, cf_device_kv_counters *counters);
const char *cf_device_kv_last_error(const cf_device_kv_dataplane *dataplane);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* CHROMOFOLD_DEVICE_KV_DATAPLANE_H */
