/* kv_cuda.h — the paged compressed-KV attention seam (name kept from the reference for drop-in linking).
 *
 * Drop-in for reference include/chromofold/kv_cuda.h: cf_kv_device_page (104 B) and cf_kv_paged_attention_desc
 * (96 B) are byte-identical, the limits are the same, and the two entry points keep their signatures and
 * validation rules. The implementation behind them is HIP for gfx950.
 *
 * Codec selection per page (legacy pages decode bit-for-bit as in the reference):
 *   fixed_code_length > 0                       fixed-width MSB-first codes of that many bits
 *   fixed_code_length == 0, k_max_code_length>0  canonical-Huffman LUT codes (lut[look] = sym | len << 8)
 *   fixed_code_length == 0, k_max_code_length==0 rANS page (additive to the reference): k_words points at one
 *       kv_codec_ext.h group blob of up to 64 tokens coded on its own (a chain start, or the INT8 raw fallback),
 *       k_lut / v_lut at its K and V tables (CF_KV_RANS_TABLE_BYTES each); the scales come from the blob header,
 *       the other page fields are not read. A blob that continues a chain or disagrees with the page's head_dim
 *       or token_count makes the outputs of that (query row, KV head) NaN.
 */
#ifndef CHROMOFOLD_KV_CUDA_H
#define CHROMOFOLD_KV_CUDA_H

#include <stdint.h>

#include "chromofold/chromofold.h"

#ifdef __cplusplus
extern "C" {
#endif

/* reference kv_cuda.h:12-13 */
#define CF_KV_CUDA_ABI_VERSION 0u
#define CF_KV_CUDA_MAX_PAGES_PER_LAUNCH 4096u

/* One immutable page of one KV head, device resident. K scales are per channel [head_dim], V scales per token
 * [token_count]. Bit offsets count from the first bit of the page's word stream. reference kv_cuda.h:21-41 */
typedef struct cf_kv_device_page {
    const uint32_t *k_words;
    const int32_t *k_block_offsets;
    const int32_t *k_lut;
    const float *k_scales;

    const uint32_t *v_words;
    const int32_t *v_block_offsets;
    const int32_t *v_lut;
    const float *v_scales;

    uint32_t token_begin;
    uint32_t token_count;
    uint32_t head_dim;
    uint32_t block_size;
    uint32_t k_max_code_length;
    uint32_t v_max_code_length;
    uint32_t zero_point;
    uint32_t kv_head;
    uint32_t fixed_code_length;
} cf_kv_device_page;

/* One layer, one sequence, query_count consecutive query tokens. queries/output are [query_count,
 * query_head_count, head_dim] fp32; query head h reads KV head h / gqa_group_size. active_k/active_v are an
 * optional dense fp32 tail [active_token_count, kv_head_count, head_dim]. reference kv_cuda.h:53-75 */
typedef struct cf_kv_paged_attention_desc {
    uint32_t struct_size;
    uint32_t abi_version;

    const cf_kv_device_page *pages;
    uint32_t page_count;
    uint32_t kv_head_count;
    uint32_t query_head_count;
    uint32_t gqa_group_size;

    const float *active_k;
    const float *active_v;
    uint32_t active_token_begin;
    uint32_t active_token_count;

    const float *queries;
    float *output;
    uint32_t query_token_begin;
    uint32_t query_count;
    uint32_t head_dim;
    uint32_t causal_window;
    float softmax_scale;
} cf_kv_paged_attention_desc;

/* Host-only structural validation; never dereferences a device pointer.
 * Replaces reference kv_cuda.h:78 (src/cuda/paged_kv_attention.cu:280-299). */
cf_status cf_kv_validate_paged_attention_desc(const cf_kv_paged_attention_desc *desc);

/* Paged attention, decoding each page inside the kernel. Allocates nothing, never synchronizes.
 * Replaces reference kv_cuda.h:86 (src/cuda/paged_kv_attention.cu:301-327).
 * Long contexts are split over many workgroups; their partial softmax states go to one of four 16 MiB regions of
 * a device array the library owns (per GPU), each region held by one stream at a time, and a second launch on the
 * same stream merges them. Calls on different streams or threads are therefore safe without serialisation by the
 * caller (the reference keeps no cross-call state either). Beyond four streams, a stream takes over a region only
 * after an event wait on the previous holder's stream, or runs unsplit. A stream under graph capture runs the
 * call unsplit. */
cf_status cf_kv_paged_attention_async(const cf_kv_paged_attention_desc *desc, void *stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* CHROMOFOLD_KV_CUDA_H */
