/* chromofold_kv_adapter.h — the llama.cpp paged-KV adapter (cf_llama_kv_*), exported by libchromofold.
 *
 * Same types, functions, argument meaning and return convention as the reference's
 * integrations/llama.cpp/chromofold_kv_adapter.h:1-89 (int 0 = ok, -1 = error with cf_llama_kv_last_error(),
 * create() returns NULL for the dense backend or invalid options). `stream` is a hipStream_t passed as void*;
 * `keys`/`values` of cf_llama_kv_append are HOST arrays [token_count, head_dim] (as in the reference);
 * queries/output of cf_llama_kv_attention are device arrays [query_count, query_head_count, head_dim].
 * The adapter is not thread-safe (as the reference's).
 */
#ifndef CHROMOFOLD_KV_ADAPTER_H
#define CHROMOFOLD_KV_ADAPTER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum cf_llama_kv_backend {
  CF_LLAMA_KV_BACKEND_DENSE = 0,
  CF_LLAMA_KV_BACKEND_CHROMOFOLD = 1,
} cf_llama_kv_backend;

typedef struct cf_llama_kv_options {
  uint32_t struct_size;
  cf_llama_kv_backend backend;
  uint32_t layer_count;
  uint32_t kv_head_count;
  uint32_t query_head_count;
  uint32_t head_dim;
  uint32_t page_size;
  uint32_t gqa_group_size;
  uint32_t kv_bits; /* 8 -> int8 pages; 0 or 4 -> int4 pages (default) */
} cf_llama_kv_options;

typedef struct cf_llama_kv_stats {
  uint64_t appended_tokens;
  uint64_t sealed_tokens;
  uint64_t sealed_pages;
  uint64_t active_tokens;
  uint64_t dense_active_bytes;
  uint64_t compressed_bytes;
  uint64_t descriptor_bytes;
} cf_llama_kv_stats;

typedef struct cf_llama_kv_adapter cf_llama_kv_adapter;

/* reference chromofold_kv_adapter.h:40-42 */
int cf_llama_kv_options_validate(const cf_llama_kv_options *options);
cf_llama_kv_adapter *cf_llama_kv_create(const cf_llama_kv_options *options);
void cf_llama_kv_destroy(cf_llama_kv_adapter *adapter);

/* Append token_count tokens of one (layer, kv head) at token_begin (must continue the head's active tail); full
 * pages are sealed (quantised, packed, uploaded) as they complete. reference chromofold_kv_adapter.h:44-51 */
int cf_llama_kv_append(cf_llama_kv_adapter *adapter, uint32_t layer, uint32_t kv_head, uint32_t token_begin,
                       const float *keys, const float *values, uint32_t token_count, void *stream);

/* Attention of one layer over its sealed pages + active tail through cf_kv_paged_attention_async.
 * reference chromofold_kv_adapter.h:56-66 */
int cf_llama_kv_attention(cf_llama_kv_adapter *adapter, uint32_t layer, const float *queries_device,
                          float *output_device, uint32_t query_count, uint32_t query_head_count,
                          uint32_t gqa_group_size, uint32_t query_token_begin, float softmax_scale,
                          uint32_t causal_window, void *stream);

/* Host-memory twin of cf_llama_kv_attention (synchronous). reference chromofold_kv_adapter.h:70-80 */
int cf_llama_kv_attention_host(cf_llama_kv_adapter *adapter, uint32_t layer, const float *queries_host,
                               float *output_host, uint32_t query_count, uint32_t query_head_count,
                               uint32_t gqa_group_size, uint32_t query_token_begin, float softmax_scale,
                               uint32_t causal_window, void *stream);

/* reference chromofold_kv_adapter.h:82-89 */
int cf_llama_kv_flush(cf_llama_kv_adapter *adapter, void *stream);
int cf_llama_kv_seq_rm(cf_llama_kv_adapter *adapter, uint64_t sequence_id);
int cf_llama_kv_seq_cp(cf_llama_kv_adapter *adapter, uint64_t source_id, uint64_t destination_id);
int cf_llama_kv_seq_shift(cf_llama_kv_adapter *adapter, uint64_t sequence_id, int32_t delta);
int cf_llama_kv_clear(cf_llama_kv_adapter *adapter);
int cf_llama_kv_get_stats(const cf_llama_kv_adapter *adapter, cf_llama_kv_stats *stats);
const char *cf_llama_kv_last_error(const cf_llama_kv_adapter *adapter);

#ifdef __cplusplus
}
#endif

#endif /* CHROMOFOLD_KV_ADAPTER_H */
