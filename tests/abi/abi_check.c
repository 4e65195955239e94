/* abi_check.c — compiled by tests/test_abi.py with plain `gcc -std=c99` against the public headers and linked
 * with libchromofold.so: the public headers are valid C, every declaration links, and the NULL-argument contract
 * holds (each call below is rejected on the host before any device call, so no GPU is needed). Prints one line per
 * check; exit status 0 = all passed. */
#include <stdio.h>
#include <string.h>

#include "chromofold/chromofold.h"
#include "chromofold/chromofold_extra.h"
#include "chromofold/chromofold_index.h"
#include "chromofold/chromofold_kv_adapter.h"
#include "chromofold/chromofold_qw.h"
#include "chromofold/chromofold_search.h"
#include "chromofold/device_kv_dataplane.h"
#include "chromofold/device_kv_seal_attention.h"
#include "chromofold/multisequence_cuda_resolver.h"
#include "chromofold/production_attention.h"
#include "chromofold/kv_codec_ext.h"
#include "chromofold/kv_cuda.h"
#include "chromofold/kv_runtime.h"
#include "chromofold/chromofold_measure.h"

static int failures = 0;

static void expect(const char *what, int got, int want) {
  printf("%-40s %d %s\n", what, got, got == want ? "ok" : "FAIL");
  if (got != want) ++failures;
}

int main(void) {
  cf_wavelet_view wv;
  cf_rrrw_view rv;
  cf_fm_view fv;
  memset(&wv, 0, sizeof wv);
  memset(&rv, 0, sizeof rv);
  memset(&fv, 0, sizeof fv);
  const int INV = CF_ERR_INVALID_ARGUMENT;
  printf("sizeof cf_wavelet_view %zu\n", sizeof(cf_wavelet_view));
  printf("sizeof cf_rrrw_view %zu\n", sizeof(cf_rrrw_view));
  printf("sizeof cf_fm_view %zu\n", sizeof(cf_fm_view));
  printf("sizeof cf_kv_device_page %zu\n", sizeof(cf_kv_device_page));
  printf("sizeof cf_kv_paged_attention_desc %zu\n", sizeof(cf_kv_paged_attention_desc));
  printf("sizeof cf_kv_batched_desc %zu\n", sizeof(cf_kv_batched_desc));
  printf("sizeof cf_qw_matrix %zu\n", sizeof(cf_qw_matrix));
  /* chromofold.h */
  expect("cf_access_async", cf_access_async(wv, NULL, NULL, 1, NULL), INV);
  expect("cf_rank_async", cf_rank_async(wv, NULL, NULL, NULL, 1, NULL), INV);
  expect("cf_embedding_gather_async", cf_embedding_gather_async(wv, NULL, 1, NULL, NULL, 1, NULL), INV);
  expect("cf_kv_attn_fused_async", cf_kv_attn_fused_async(NULL, NULL, NULL, 0, NULL, NULL, NULL, 0, NULL, NULL,
                                                          NULL, NULL, 0, 0, 0, 0, 0, 0, 0.0f, NULL), INV);
  expect("cf_kv_attn_dense_async", cf_kv_attn_dense_async(NULL, NULL, NULL, 0, NULL, NULL, NULL, 0, NULL, NULL,
                                                          NULL, NULL, NULL, NULL, 0, 0, 0, 0, 0, 0, 0.0f, NULL), INV);
  /* chromofold_search.h */
  expect("cf_rrrw_access_async", cf_rrrw_access_async(rv, NULL, NULL, 1, NULL), INV);
  expect("cf_rrrw_rank_async", cf_rrrw_rank_async(rv, NULL, NULL, NULL, 1, NULL), INV);
  expect("cf_fm_count_async", cf_fm_count_async(fv, NULL, NULL, NULL, NULL, 1, NULL), INV);
  expect("cf_fm_ranges_async", cf_fm_ranges_async(fv, NULL, NULL, NULL, NULL, NULL, 1, NULL), INV);
  expect("cf_fm_locate_async", cf_fm_locate_async(fv, NULL, NULL, 1, NULL), INV);
  /* chromofold_extra.h */
  expect("cf_rank2_async", cf_rank2_async(wv, NULL, NULL, 1, 8, NULL, NULL, NULL, 1, NULL), INV);
  expect("cf_embedding_gather_tpq_async", cf_embedding_gather_tpq_async(wv, NULL, 1, NULL, NULL, 1, NULL), INV);
  expect("cf_rrr_rank_async", cf_rrr_rank_async(NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, 1, NULL), INV);
  expect("cf_delta_fetch_async",
         cf_delta_fetch_async(NULL, 0, NULL, NULL, NULL, NULL, NULL, NULL, NULL, 1, NULL), INV);
  expect("cf_sparse_gather_fused_async", cf_sparse_gather_fused_async(rv, NULL, 1, NULL, NULL, 1, NULL), INV);
  expect("cf_sparse_decode_all_async", cf_sparse_decode_all_async(rv, NULL, 1, NULL), INV);
  expect("cf_sparse_gather_async", cf_sparse_gather_async(NULL, NULL, 1, NULL, NULL, 1, NULL), INV);
  expect("cf_rans_decode_async", cf_rans_decode_async(NULL, NULL, NULL, NULL, NULL, NULL, 64, 1, NULL, NULL), INV);
  expect("cf_fused_matmul_async",
         cf_fused_matmul_async(NULL, NULL, NULL, 8, 64, NULL, NULL, 1, 1, 1, 1.0f, 8, NULL), INV);
  expect("cf_dense_matmul_async",
         cf_dense_matmul_async(NULL, NULL, NULL, 8, 64, NULL, NULL, NULL, 1, 1, 1, 1.0f, 8, NULL), INV);
  /* chromofold_index.h */
  expect("cf_suffix_array", cf_suffix_array(NULL, 4, 3, NULL, NULL, 0, NULL), INV);
  expect("cf_suffix_array_workspace_bytes(0)", (int)cf_suffix_array_workspace_bytes(0, 1), 0);
  /* chromofold_qw.h */
  expect("cf_qw_validate", cf_qw_validate(NULL), INV);
  expect("cf_qw_matmul_async", cf_qw_matmul_async(NULL, NULL, NULL, 1, NULL), INV);
  expect("cf_qw_quantize_int4", cf_qw_quantize_int4(NULL, 1, 1, NULL, NULL), INV);
  expect("cf_qw_huffman_plan", (int)cf_qw_huffman_plan(NULL, 1, 1, NULL), 0);
  expect("cf_qw_huffman_encode", cf_qw_huffman_encode(NULL, 1, 1, NULL, NULL, 0, NULL), INV);
  /* kv_cuda.h */
  expect("cf_kv_validate_paged_attention_desc", cf_kv_validate_paged_attention_desc(NULL), INV);
  expect("cf_kv_paged_attention_async", cf_kv_paged_attention_async(NULL, NULL), INV);
  /* kv_codec_ext.h */
  expect("cf_kv_validate_batched_desc", cf_kv_validate_batched_desc(NULL), INV);
  expect("cf_kv_paged_attention_batched_async", cf_kv_paged_attention_batched_async(NULL, NULL), INV);
  expect("cf_kv_paged_attention_batched_noalloc_async", cf_kv_paged_attention_batched_noalloc_async(NULL, NULL), INV);
  /* kv_runtime.h */
  expect("cf_kv_validate_page", cf_kv_validate_page(NULL), INV);
  expect("cf_kv_validate_layout", cf_kv_validate_layout(NULL), INV);
  expect("cf_kv_page_resident_bytes", cf_kv_page_resident_bytes(NULL, NULL), INV);
  expect("cf_kv_cache_memory_stats", cf_kv_cache_memory_stats(NULL, NULL), INV);
  expect("cf_online_softmax_init", cf_online_softmax_init(NULL, NULL, 1), INV);
  expect("cf_online_softmax_accumulate", cf_online_softmax_accumulate(NULL, 0.0, NULL), INV);
  expect("cf_online_softmax_merge", cf_online_softmax_merge(NULL, NULL), INV);
  expect("cf_online_softmax_finalize", cf_online_softmax_finalize(NULL, NULL), INV);
  /* chromofold_kv_adapter.h: int 0 / -1 convention, NULL create for bad options */
  expect("cf_llama_kv_options_validate", cf_llama_kv_options_validate(NULL), -1);
  expect("cf_llama_kv_create", cf_llama_kv_create(NULL) == NULL, 1);
  expect("cf_llama_kv_append", cf_llama_kv_append(NULL, 0, 0, 0, NULL, NULL, 1, NULL), -1);
  expect("cf_llama_kv_attention", cf_llama_kv_attention(NULL, 0, NULL, NULL, 1, 1, 1, 0, 1.0f, 0, NULL), -1);
  expect("cf_llama_kv_flush", cf_llama_kv_flush(NULL, NULL), -1);
  expect("cf_llama_kv_get_stats", cf_llama_kv_get_stats(NULL, NULL), -1);
  expect("cf_llama_kv_last_error", cf_llama_kv_last_error(NULL) != NULL, 1);
  expect("cf_kv_encode_fixed_page", cf_kv_encode_fixed_page(4, NULL, NULL, 1, 1, 64, NULL, NULL, NULL, NULL, NULL), INV);
  expect("cf_kv_encode_groups_async",
         cf_kv_encode_groups_async(2, NULL, NULL, 1, NULL, NULL, NULL, 64, NULL, 2, NULL, NULL, NULL, 0, 0, NULL, NULL,
                                   NULL, NULL, 0, NULL), INV);
  expect("cf_kv_encode_groups_workspace_bytes", cf_kv_encode_groups_workspace_bytes(2, 20, 1, 2) == 0, 1);
  /* chromofold_measure.h */
  expect("cf_stream_read_async", cf_stream_read_async(NULL, 16, NULL, NULL), INV);
  {
    cf_rrrw_file_header rh;
    cf_fm_file_header fh;
    memset(&rh, 0, sizeof rh);
    memset(&fh, 0, sizeof fh);
    printf("sizeof cf_rrrw_file_header %zu\n", sizeof(cf_rrrw_file_header));
    printf("sizeof cf_fm_file_header %zu\n", sizeof(cf_fm_file_header));
    printf("sizeof cf_fm_file_arrays %zu\n", sizeof(cf_fm_file_arrays));
    expect("cf_rrrw_file_read_header", cf_rrrw_file_read_header(NULL, &rh), INV);
    expect("cf_rrrw_file_read", cf_rrrw_file_read("x", NULL, NULL, NULL), INV);
    expect("cf_rrrw_file_write", cf_rrrw_file_write("x", &rh, NULL, NULL), INV);
    expect("cf_fm_file_read_header", cf_fm_file_read_header(NULL, &fh), INV);
    expect("cf_fm_file_read", cf_fm_file_read("x", &fh, NULL, NULL), INV);
    expect("cf_fm_file_write", cf_fm_file_write(NULL, &fh, NULL, NULL), INV);
  }
  {
    printf("sizeof cf_device_tensor_view %zu\n", sizeof(cf_device_tensor_view));
    printf("sizeof cf_device_page_descriptor %zu\n", sizeof(cf_device_page_descriptor));
    printf("sizeof cf_device_seal_counters %zu\n", sizeof(cf_device_seal_counters));
    printf("sizeof cf_device_kv_counters %zu\n", sizeof(cf_device_kv_counters));
    printf("sizeof cf_ms_page_publication %zu\n", sizeof(cf_ms_page_publication));
    printf("sizeof cf_ms_batch_item %zu\n", sizeof(cf_ms_batch_item));
    printf("sizeof cf_ms_cuda_counters %zu\n", sizeof(cf_ms_cuda_counters));
    cf_device_tensor_view tv;
    memset(&tv, 0, sizeof tv);
    expect("cf_device_tensor_validate", cf_device_tensor_validate(&tv), -1);
    expect("cf_device_seal_create", cf_device_seal_create(NULL) == NULL, 1);
    expect("cf_device_seal_full_page_async", cf_device_seal_full_page_async(NULL, 0, NULL), -1);
    expect("cf_device_seal_attention_async",
           cf_device_seal_attention_async(NULL, 0, NULL, NULL, 3, 0, 0, 0, 0, 1.0f, 0, NULL), -1);
    expect("cf_device_seal_set_fault", cf_device_seal_set_fault(NULL, 0), -1);
    expect("cf_device_seal_get_pages", cf_device_seal_get_pages(NULL, 0, NULL, 0, NULL), -1);
    expect("cf_device_kv_create", cf_device_kv_create(NULL) == NULL, 1);
    expect("cf_device_kv_append_async", cf_device_kv_append_async(NULL, 0, 0, NULL, NULL, NULL), -1);
    expect("cf_device_kv_attention_async", cf_device_kv_attention_async(NULL, 0, NULL, NULL, 1, 0, 1.0f, 0, NULL), -1);
    expect("cf_ms_cuda_create", cf_ms_cuda_create(NULL) == NULL, 1);
    expect("cf_ms_cuda_execute_batch_async", cf_ms_cuda_execute_batch_async(NULL, NULL, 0, NULL), -1);
    expect("cf_ms_cuda_audit", cf_ms_cuda_audit(NULL), -1);
    expect("cf_ms_cuda_last_error", cf_ms_cuda_last_error(NULL) != NULL, 1);
  }
  {
    printf("sizeof cf_attention_runtime_config %zu\n", sizeof(cf_attention_runtime_config));
    printf("sizeof cf_attention_batch_item %zu\n", sizeof(cf_attention_batch_item));
    printf("sizeof cf_attention_counters %zu\n", sizeof(cf_attention_counters));
    expect("cf_attention_runtime_create", cf_attention_runtime_create(NULL) == NULL, 1);
    cf_attention_runtime_config cfg;
    memset(&cfg, 0, sizeof cfg);
    cfg.layer_count = 1;
    cfg.query_head_count = 8;
    cfg.kv_head_count = 2;
    cfg.head_dim = 64;
    cfg.gqa_group_size = 4;
    cfg.mode = CF_ATTENTION_REFERENCE;
    cf_attention_runtime *rt = cf_attention_runtime_create(&cfg);
    expect("cf_attention_runtime_create (valid)", rt != NULL, 1);
    cfg.gqa_group_size = 3;
    expect("cf_attention_runtime_create (heads != kv * gqa)", cf_attention_runtime_create(&cfg) == NULL, 1);
    cf_attention_batch_item item;
    memset(&item, 0, sizeof item);
    expect("cf_attention_execute_async (NULL)", cf_attention_execute_async(NULL, &item, 1, NULL), -1);
    expect("cf_attention_execute_async (no items)", cf_attention_execute_async(rt, NULL, 1, NULL), -1);
    expect("cf_attention_execute_async (reference mode)", cf_attention_execute_async(rt, &item, 1, NULL), -1);
    expect("cf_attention_compare_async", cf_attention_compare_async(rt, &item, 1, 1e-3f, 1e-4f, NULL), -1);
    expect("cf_attention_compare_async (bad tolerance)", cf_attention_compare_async(rt, &item, 1, 0.0f, 1.0f, NULL), -1);
    expect("cf_attention_invalidate_graphs", cf_attention_invalidate_graphs(rt), 0);
    cf_attention_counters c;
    expect("cf_attention_get_counters", cf_attention_get_counters(rt, &c), 0);
    expect("reference_launches", (int)c.reference_launches, 1);
    expect("graph_invalidations", (int)c.graph_invalidations, 1);
    expect("cf_attention_get_counters (NULL)", cf_attention_get_counters(NULL, &c), -1);
    expect("cf_attention_last_error", cf_attention_last_error(rt)[0] != 0, 1);
    expect("cf_attention_last_error (NULL)", cf_attention_last_error(NULL) != NULL, 1);
    cf_attention_runtime_destroy(rt, NULL);
    cf_attention_runtime_destroy(NULL, NULL);
    cfg.gqa_group_size = 4;
    cfg.mode = CF_ATTENTION_OPTIMIZED;
    rt = cf_attention_runtime_create(&cfg);
    /* an item with a NULL query is refused before any device work */
    expect("cf_attention_execute_async (NULL query)", cf_attention_execute_async(rt, &item, 1, NULL), -1);
    expect("cf_attention_last_error (NULL query)", strstr(cf_attention_last_error(rt), "NULL") != NULL, 1);
    cf_attention_runtime_destroy(rt, NULL);
    cfg.head_dim = 12;
    expect("cf_attention_runtime_create (head_dim 12)", cf_attention_runtime_create(&cfg) == NULL, 1);
  }
  printf("%s (%d failure%s)\n", failures ? "FAIL" : "PASS", failures, failures == 1 ? "" : "s");
  return failures ? 1 : 0;
}
