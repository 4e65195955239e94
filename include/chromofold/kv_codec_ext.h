/* kv_codec_ext.h — ADDITIVE extension of the paged-KV seam: rANS-coded KV pages and a batched multi-sequence
 * decode entry point. Nothing in kv_cuda.h changes; legacy fixed-width / Huffman pages keep decoding through
 * cf_kv_paged_attention_async bit-for-bit.
 *
 * Why an extension: the reference seam covers one sequence and at most CF_KV_CUDA_MAX_PAGES_PER_LAUNCH pages per
 * launch (reference include/chromofold/kv_cuda.h:13, src/cuda/paged_kv_attention.cu:289), and its only KV codecs
 * are fixed-width and block-Huffman (reference src/runtime/kv_gpu_fixture.cpp:18-43); the reference never wires
 * its block-rANS decoder (src/cuda/rans.cu) into attention. A Llama-3-8B decode step at 32k context and batch 32
 * is 32 sequences x 8 KV heads x 2048 pages, so it needs both a batched entry and an rANS page codec.
 *
 * ------------------------------------------------------------------------------------------------------------
 * Page codec CF_KV_CODEC_RANS_HYBRID (one KV head, 16 tokens, head_dim D with D % 16 == 0 and D <= 128)
 *
 * Quantisation: per page and head, K and V each get one absmax scale s = max|x| / 127 (1.0 if all zero) and
 * symbols sym = clamp(rint(x / s), -128, 127) + 128 (round half to even, IEEE fp32 division); x ~ (sym - 128) * s.
 *
 * Each symbol is split into a 2-bit high part h = sym >> 6 and a 6-bit low part l = sym & 63 ("hybrid integer"
 * coding, as in JPEG XL's HybridUint / CABAC bypass bins): the low parts of a Gaussian-like int8 distribution are
 * nearly uniform and are stored raw, the high parts carry the skew and are entropy coded. The four high parts of a
 * quad of values form one 8-bit joint symbol  j = h0 | h1 << 2 | h2 << 4 | h3 << 6  coded with rANS.
 *
 * Lane assignment (16 interleaved rANS states per stream, state/lane index t = 0..15), value order per lane:
 *   K stream: lane t owns token t and walks its dims d = 0..D-1; quad q = dims 4q..4q+3.
 *   V stream: lane t owns dims {t + 16 i : i < D/16}; quads in the order (tq = 0..3, i = 0..D/16-1),
 *             quad = tokens 4tq..4tq+3 at dim t + 16 i.
 * Every lane decodes D/4 quads. Pages with fewer than 16 tokens are padded with symbol 128 (value 0); the kernel
 * masks tokens >= the page's token count.
 *
 * rANS: M = 2^11 (11-bit probabilities), state in [2^16, 2^32), 16-bit renormalisation words. Decode step:
 *   slot = x & 2047; j, f, c = table[slot]; x = f * (x >> 11) + slot - c; if (x < 2^16) x = (x << 16) | word.
 * At step q all 16 lanes decode their quad q; the lanes that renormalise read consecutive words of ONE shared word
 * stream in ascending lane order (interleaved rANS; the encoder emits in the exact reverse order).
 *
 * Low parts, bit-sliced per lane in groups of 16 values (4 quads qd = 0..3, position i = 0..3 inside a quad):
 *   N0 = sum_i (l(0,i) & 15) << 8i | (l(1,i) & 15) << (8i + 4)      (quads 0,1)
 *   N1 = same for quads 2,3
 *   C  = sum_{qd,i} (l(qd,i) >> 4) << (8i + 2qd)
 * so that the symbol bytes of quad qd are  (nibbles) | (((C >> 2qd) << 4) & 0x30303030) | (highs << 6).
 * The words of lane t, group g, word w (0: N0, 1: N1, 2: C) sit at index (g*3 + w)*16 + t (coalesced reads).
 *
 * Page blob (16-byte aligned, all little-endian):
 *   [0]   cf_kv_rans_page_header (32 B)
 *   [32]  k_states[16] u32, v_states[16] u32
 *   [160] k_lows[3*(D/16)*16] u32, v_lows[3*(D/16)*16] u32
 *   then  k_words[k_word_count] u16, v_words[v_word_count] u16, zero padding to a 16-byte multiple.
 *
 * Table blob (CF_KV_RANS_TABLE_BYTES = 16 KiB): 2048 slot entries of two u32:
 *   lo = (f - 1) | c_slot << 11 | j << 22   with c_slot = slot - cum[j] (the in-symbol slot offset)
 *   hi = spread(j) = sum_i ((j >> 2i) & 3) << (8i + 6)
 *
 * Page codec CF_KV_CODEC_INT8: same header, then K then V symbol bytes, lane-major quads laid out like the low
 * words above (word (q*16 + t) holds the 4 symbol bytes of quad q of lane t). 4 KiB + 32 B per page at D = 128.
 * ------------------------------------------------------------------------------------------------------------ */
#ifndef CHROMOFOLD_KV_CODEC_EXT_H
#define CHROMOFOLD_KV_CODEC_EXT_H

#include <stddef.h>
#include <stdint.h>

#include "chromofold/chromofold.h"

#ifdef __cplusplus
extern "C" {
#endif

#define CF_KV_EXT_ABI_VERSION 1u
#define CF_KV_CODEC_INT8 1u
#define CF_KV_CODEC_RANS_HYBRID 2u
#define CF_KV_PAGE_TOKENS 16u
#define CF_KV_RANS_PROB_BITS 11u
#define CF_KV_RANS_LANES 16u
#define CF_KV_RANS_TABLE_BYTES 16384u

typedef struct cf_kv_rans_page_header {
    uint32_t codec;          /* CF_KV_CODEC_* */
    uint16_t k_word_count;   /* 16-bit rANS words in the K stream (0 for INT8) */
    uint16_t v_word_count;
    float k_scale;
    float v_scale;
    uint16_t token_count;    /* 1..16 */
    uint16_t head_dim;
    uint32_t k_table;        /* table index for the K stream (RANS_HYBRID) */
    uint32_t v_table;
    uint32_t reserved;
} cf_kv_rans_page_header;

/* Batched decode: `seq_count` sequences, each with `kv_head_count` heads of pages in token order.
 *   page_offsets [seq_count * kv_head_count * max_pages]  byte offset / 16 of each page blob inside `pool`
 *   seq_tokens   [seq_count]  visible context length per sequence (pages hold tokens 16p .. 16p+15)
 *   query_pos    [seq_count]  position of the decoded query token (causal limit; tokens > query_pos are masked)
 *   queries      [seq_count, query_head_count, head_dim] fp32, output the same shape
 * A shared prefix is expressed by several sequences pointing at the same page blobs (refcounted pages).
 * `workspace` is caller-owned device memory of cf_kv_batched_workspace_bytes() bytes (split-context partials);
 * the entry point allocates nothing and never synchronises. */
typedef struct cf_kv_batched_desc {
    uint32_t struct_size;
    uint32_t abi_version;
    uint32_t codec;
    uint32_t seq_count;
    uint32_t kv_head_count;
    uint32_t query_head_count;
    uint32_t head_dim;
    uint32_t max_pages;          /* per sequence and head (row stride of page_offsets) */
    const uint8_t *pool;         /* page blobs, 16-byte aligned */
    const uint32_t *page_offsets;
    const uint32_t *seq_tokens;
    const uint32_t *query_pos;
    const uint8_t *tables;       /* RANS_HYBRID: table blobs, CF_KV_RANS_TABLE_BYTES each */
    const float *queries;
    float *output;
    float softmax_scale;
    uint32_t splits;             /* context splits per (sequence, head); 0 = choose */
    void *workspace;
    uint64_t workspace_bytes;
} cf_kv_batched_desc;

/* Bytes of workspace the launch needs for this descriptor (0 when no split is used). Host only. */
uint64_t cf_kv_batched_workspace_bytes(const cf_kv_batched_desc *desc);

/* Host-only validation of a batched descriptor (no device dereference). */
cf_status cf_kv_validate_batched_desc(const cf_kv_batched_desc *desc);

/* Batched paged attention decode over INT8 or RANS_HYBRID pages. No counterpart in the reference (see above);
 * semantics of one (sequence, query head) equal cf_kv_paged_attention_async with one query row and no tail. */
cf_status cf_kv_paged_attention_batched_async(const cf_kv_batched_desc *desc, void *stream);

/* ---- host-side page encoder (CPU, used when sealing pages) ---------------------------------------------- */

/* Build a table blob (CF_KV_RANS_TABLE_BYTES) from a histogram of 256 joint high-part symbols. Every symbol gets
 * a nonzero frequency, so any page can be coded with any table. */
cf_status cf_kv_rans_build_table(const uint64_t *joint_histogram256, uint8_t *table_out);

/* Joint-symbol histogram of one page's K (or V) values [token_count, head_dim] (accumulates into hist256). */
cf_status cf_kv_rans_page_histogram(const float *values, uint32_t token_count, uint32_t head_dim,
                                    uint64_t *hist256);

/* Size bound for one encoded page blob at this head_dim (for pool allocation). */
uint64_t cf_kv_page_blob_max_bytes(uint32_t codec, uint32_t head_dim);

/* Quantise and encode one page (K and V [token_count, head_dim] fp32, token_count <= 16) into `blob`
 * (capacity `blob_capacity`); writes the blob size to *blob_bytes. Tables are host copies of table blobs. */
cf_status cf_kv_encode_page(uint32_t codec, const float *keys, const float *values, uint32_t token_count,
                            uint32_t head_dim, const uint8_t *k_table, const uint8_t *v_table,
                            uint32_t k_table_index, uint32_t v_table_index, uint8_t *blob,
                            uint64_t blob_capacity, uint64_t *blob_bytes);

/* Batch form of cf_kv_encode_page for npages page-major pages ([npages][16][head_dim] fp32 K and V), encoded
 * on `threads` host threads (0 = all) and packed 16-byte aligned into pool[pool_at ..]; offsets_out[p] = byte
 * offset / 16 of page p; *pool_end = first free byte. token_counts / heads (table pair per page) may be NULL. */
cf_status cf_kv_encode_pages(uint32_t codec, const float *keys, const float *values, uint64_t npages,
                             const uint32_t *token_counts, uint32_t head_dim, const uint8_t *tables,
                             const uint32_t *heads, uint8_t *pool, uint64_t pool_capacity, uint64_t pool_at,
                             uint32_t *offsets_out, uint64_t *pool_end, uint32_t threads);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* CHROMOFOLD_KV_CODEC_EXT_H */
