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
 * Storage unit: a "page group" = up to 4 consecutive 16-token pages of one (sequence, KV head) coded together, so
 * that one 64-lane wavefront decodes it with interleaved rANS states, 64 per word stream (wave-uniform cursor, lane
 * offset by mbcnt). Pages stay the logical unit: each page has its own token count and scales.
 * Lane L = 16 G + t belongs to page G of the group.
 *
 * Quantisation (per page and head; K and V separately): s = max|x| / 127 (1.0 if all zero),
 * sym = clamp(rint(x / s), -128, 127) + 128 (round half to even, IEEE fp32 division); x ~ (sym - 128) * s.
 * Absent pages and tokens are padded with symbol 128 (value 0); the kernel masks them.
 *
 * CF_KV_CODEC_RANS_HYBRID: each symbol splits into a 2-bit high part h = sym >> 6 and a 6-bit low part
 * l = sym & 63 ("hybrid integer" coding, as in JPEG XL's HybridUint / CABAC bypass bins): the low parts of a
 * Gaussian-like int8 distribution are nearly uniform and stay raw; the high parts carry the skew. The four high
 * parts of a quad of values form one 8-bit joint symbol  j = h0 | h1 << 2 | h2 << 4 | h3 << 6  coded with rANS.
 *
 * Value order per lane (D = head_dim, D % 16 == 0, D <= 128; every lane owns D values = D/4 quads):
 *   K stream: lane L owns token t of page G, dims d = 0..D-1; quad q = dims 4q..4q+3.
 *   V stream: lane L owns dims {t + 16 i : i < D/16} of page G; quads in the order (tq = 0..3, i = 0..D/16-1),
 *             quad = tokens 4tq..4tq+3 at dim t + 16 i.
 *
 * rANS: M = 2^11, state in [2^16, 2^32), 16-bit renormalisation words. Each stream (K, V) is coded as TWO
 * interleaved chains of 64 lane states: chain A holds the even quads (q = 0, 2, 4, ...) and chain B the odd quads,
 * each with its own word stream, so a lane advances four independent states (K A/B, V A/B) at once. Decode step of
 * a chain (all 64 lanes, its next quad q):
 *   slot = x & 2047; (f, c, j) = table[slot]; x = f * (x >> 11) + c; then the lanes with x < 2^16 read, in
 *   ascending lane order, the next words of the chain's stream: x = (x << 16) | word.  (c = slot - cum[j].)
 * The encoder runs the exact reverse per chain (its quads descending, lanes descending) starting every state at
 * 2^16, so a correct decode ends with all states at 2^16 and every cursor at its stream's word count.
 *
 * Low parts, bit-sliced per lane in groups of 16 values (4 quads qd = 0..3, position i = 0..3 inside a quad):
 *   N0 = sum_i (l(0,i) & 15) << 8i | (l(1,i) & 15) << (8i + 4)      (quads 0,1)
 *   N1 = same for quads 2,3
 *   C  = sum_{qd,i} (l(qd,i) >> 4) << (8i + 2qd)
 * The symbol bytes of quad qd: nibble (N0, N0 >> 4, N1, N1 >> 4) & 0x0F0F0F0F, bits 4-5 of every byte from
 * (C << 4, C << 2, C, C >> 2) & 0x30303030, bits 6-7 from the high parts.
 * The words of lane L, low group g, word w (0: N0, 1: N1, 2: C) sit at index (g*3 + w)*64 + L.
 *
 * Group blob (16-byte aligned, little-endian):
 *   [0]    cf_kv_group_header (64 B)
 *   RANS_HYBRID: [64] states u32: K chain A [64], K chain B [64], V chain A [64], V chain B [64];
 *                [1088] k_lows[3*(D/16)*64] u32, v_lows[same];
 *                then the word streams u16 of K A, K B, V A, V B (word_count[0..3] words each), zero padding to 16
 *                bytes.
 *   INT8:        [64] K symbol bytes, word (q*64 + L) = the 4 bytes of quad q of lane L; then V the same way.
 *
 * Table blob (CF_KV_RANS_TABLE_BYTES = 16 KiB): 2048 slot entries of two u32:
 *   lo = f | c << 11 | j << 22     (every symbol has f >= 1, so f <= 1793 fits 11 bits)
 *   hi = spread(j) = sum_i ((j >> 2i) & 3) << (8i + 6)
 * The batched launch uses table 2h for the K streams and 2h+1 for the V streams of KV head h.
 *
 * Raw fallback: a group whose rANS words (all four streams together) would exceed CF_KV_RANS_MAX_GROUP_WORDS
 * (data the tables do not fit, e.g. near-uniform high parts) is stored as an INT8 group instead (its header says
 * so); a RANS_HYBRID pool may therefore hold both kinds and the decoder dispatches per group.
 * ------------------------------------------------------------------------------------------------------------ */
#ifndef CHROMOFOLD_KV_CODEC_EXT_H
#define CHROMOFOLD_KV_CODEC_EXT_H

#include <stddef.h>
#include <stdint.h>

#include "chromofold/chromofold.h"

#ifdef __cplusplus
extern "C" {
#endif

#define CF_KV_EXT_ABI_VERSION 3u
#define CF_KV_GROUP_PAGES 4u
#define CF_KV_CODEC_INT8 1u
#define CF_KV_CODEC_RANS_HYBRID 2u
#define CF_KV_PAGE_TOKENS 16u
#define CF_KV_RANS_PROB_BITS 11u
#define CF_KV_RANS_LANES 64u
#define CF_KV_RANS_TABLE_BYTES 16384u
#define CF_KV_RANS_MAX_GROUP_WORDS 2048u

typedef struct cf_kv_group_header {
    uint32_t codec;            /* CF_KV_CODEC_* */
    uint16_t word_count[4];    /* 16-bit rANS words of the K A, K B, V A, V B streams (0 for INT8) */
    uint16_t token_count[4];   /* tokens of each page, 0 = page absent */
    uint16_t head_dim;
    uint16_t page_count;       /* 1..4 */
    uint32_t k_table;          /* table index of the K stream (informational) */
    uint32_t v_table;
    float k_scale[4];
    float v_scale[4];
} cf_kv_group_header;

/* Batched decode: `seq_count` sequences, each with `kv_head_count` heads of page groups in token order.
 *   group_offsets [seq_count * kv_head_count * max_groups]  byte offset / 16 of each group blob inside `pool`
 *   seq_tokens   [seq_count]  context length per sequence (group g holds tokens 64g .. 64g+63)
 *   query_pos    [seq_count]  position of the decoded query token (causal limit; tokens > query_pos are masked)
 *   queries      [seq_count, query_head_count, head_dim] fp32, output the same shape
 * A shared prefix is expressed by several sequences pointing at the same group blobs (refcounted pages).
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
    uint32_t max_groups;         /* per sequence and head (row stride of group_offsets) */
    const uint8_t *pool;         /* group blobs, 16-byte aligned */
    const uint32_t *group_offsets;
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

/* Cascade decode for a prefix shared by every sequence: the first `shared_groups` groups of each sequence are the
 * same blobs (sequence 0's group_offsets rows give them; the other sequences' entries for those groups are not
 * read). The prefix is streamed once per KV head for all sequences' queries (a dense pass on the matrix cores) and
 * merged with each sequence's own groups, which are decoded as by cf_kv_paged_attention_batched_async (desc->codec,
 * desc->splits apply to them). Requirements: head_dim 128; the prefix groups are INT8 blobs (a prefix group of
 * another codec turns the outputs of every sequence into NaN); 1 <= shared_groups <= max_groups. Query positions
 * and sequence lengths mask the prefix like any other tokens. `workspace` must hold
 * cf_kv_cascade_workspace_bytes() bytes; nothing is allocated, nothing synchronises. No counterpart in the
 * reference: its caller is a decode step of many sequences over one long common prefix (e.g. 256 sequences
 * sharing an 8192-token system prompt). */
uint64_t cf_kv_cascade_workspace_bytes(const cf_kv_batched_desc *desc, uint32_t shared_groups);
cf_status cf_kv_paged_attention_cascade_async(const cf_kv_batched_desc *desc, uint32_t shared_groups, void *stream);

/* ---- host-side page encoder (CPU, used when sealing pages) ---------------------------------------------- */

/* Build a table blob (CF_KV_RANS_TABLE_BYTES) from a histogram of 256 joint high-part symbols. Every symbol gets
 * a nonzero frequency, so any page can be coded with any table. */
cf_status cf_kv_rans_build_table(const uint64_t *joint_histogram256, uint8_t *table_out);

/* Joint-symbol histogram of one page's values [token_count, head_dim] in K lane order (accumulates). */
cf_status cf_kv_rans_page_histogram(const float *values, uint32_t token_count, uint32_t head_dim,
                                    uint64_t *hist256);

/* Size bound for one encoded group blob at this head_dim (for pool allocation). */
uint64_t cf_kv_group_blob_max_bytes(uint32_t codec, uint32_t head_dim);

/* Quantise and encode one page group: K and V [page_count * 16, head_dim] fp32 (page-major), token_counts[page]
 * (1..16; pages past page_count absent). Tables are host copies of table blobs (RANS_HYBRID). Writes the blob
 * into `blob` (capacity `blob_capacity`) and its size to *blob_bytes. */
cf_status cf_kv_encode_group(uint32_t codec, const float *keys, const float *values, uint32_t page_count,
                             const uint32_t *token_counts, uint32_t head_dim, const uint8_t *k_table,
                             const uint8_t *v_table, uint32_t k_table_index, uint32_t v_table_index, uint8_t *blob,
                             uint64_t blob_capacity, uint64_t *blob_bytes);

/* Batch form: ngroups groups, group i = page_counts[i] pages starting at page first_page[i] of the page-major
 * arrays keys/values ([*][16][head_dim]); table pair heads[i] (may be NULL: 0). Encoded on `threads` host
 * threads (0 = all), packed 16-byte aligned into pool[pool_at ..]; offsets_out[i] = byte offset / 16;
 * *pool_end = first free byte. token_counts is per page (NULL: all 16). */
cf_status cf_kv_encode_groups(uint32_t codec, const float *keys, const float *values, uint64_t ngroups,
                              const uint64_t *first_page, const uint32_t *page_counts, const uint32_t *token_counts,
                              uint32_t head_dim, const uint8_t *tables, const uint32_t *heads, uint8_t *pool,
                              uint64_t pool_capacity, uint64_t pool_at, uint32_t *offsets_out, uint64_t *pool_end,
                              uint32_t threads);

/* ---- device-side page encoder (sealing on the GPU) --------------------------------------------------------- */

/* Device twin of cf_kv_encode_groups: the same groups quantised and encoded on the GPU, producing the same blobs
 * at the same pool offsets, byte for byte (no counterpart in the reference, whose pages are always sealed on the
 * host: src/runtime/compressed_kv_cache.cu:89-109). Every array argument is DEVICE memory: keys/values (page-major
 * [*][16][head_dim] fp32, 16-byte aligned), first_page/page_counts/heads [ngroups], token_counts per page (NULL:
 * all 16), tables = table_count table blobs (RANS_HYBRID), pool (16-byte aligned), offsets_out [ngroups],
 * *pool_end, *status, workspace. Asynchronous on `stream`; allocates nothing and never synchronises.
 * Synchronous return: argument errors only. Device-side outcome in *status once the stream has run: CF_OK, or
 * CF_ERR_INVALID_ARGUMENT when a group has a bad page/token count or table pair (heads[i] must satisfy
 * 2 * heads[i] + 1 < table_count and both tables must be valid) or the blobs do not fit pool_capacity — in those
 * cases nothing is written to pool, offsets_out or *pool_end. */
uint64_t cf_kv_encode_groups_workspace_bytes(uint32_t codec, uint32_t head_dim, uint64_t ngroups,
                                             uint32_t table_count);
cf_status cf_kv_encode_groups_async(uint32_t codec, const float *keys, const float *values, uint64_t ngroups,
                                    const uint64_t *first_page, const uint32_t *page_counts,
                                    const uint32_t *token_counts, uint32_t head_dim, const uint8_t *tables,
                                    uint32_t table_count, const uint32_t *heads, uint8_t *pool,
                                    uint64_t pool_capacity, uint64_t pool_at, uint32_t *offsets_out,
                                    uint64_t *pool_end, uint32_t *status, void *workspace, uint64_t workspace_bytes,
                                    void *stream);

/* Host encoder of the reference's fixed-width page format (the format cf_kv_paged_attention_async decodes with
 * fixed_code_length = bits): K per-channel and V per-token scales max|x| / (2^(bits-1) - 1) (1.0 when all zero),
 * sym = clamp(lrint(x / s), -2^(bits-1), 2^(bits-1) - 1) + 2^(bits-1), codes packed MSB-first, one block offset
 * (bit position) every `block` symbols. bits is 4 or 8. Outputs: k_words/v_words [(T*D*bits + 31) / 32],
 * k_scales [D], v_scales [T], block_offsets [ceil(T*D / block)] (identical for K and V). Same results as reference
 * src/runtime/kv_gpu_fixture.cpp:12-95; returns CF_ERR_INVALID_ARGUMENT for bad shapes or non-finite input. */
cf_status cf_kv_encode_fixed_page(uint32_t bits, const float *keys, const float *values, uint32_t token_count,
                                  uint32_t head_dim, uint32_t block, uint32_t *k_words, uint32_t *v_words,
                                  float *k_scales, float *v_scales, int32_t *block_offsets);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* CHROMOFOLD_KV_CODEC_EXT_H */
