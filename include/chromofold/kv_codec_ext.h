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
 * q = clamp(rint(x / s), -128, 127) (round half to even, IEEE fp32 division); x ~ q * s. |q| <= 127 for every finite
 * page (only NaN inputs give -128). INT8 groups store sym = q + 128; absent pages and tokens are padded with
 * q = 0 and the kernel masks them.
 *
 * CF_KV_CODEC_RANS_HYBRID (format 4): each value is kept as a sign-magnitude byte b = (q < 0) << 7 | |q| and split
 * into a "big" bit (|q| >= 64), a raw sign bit and 6 raw low bits (|q| & 63): the low parts of a Gaussian-like int8
 * distribution are nearly uniform and the sign is a fair coin, so they stay raw; the big bits carry the skew. The
 * big bits of 8 values (two quads) form one 8-bit joint symbol coded with rANS.
 *
 * Value order per lane (D = head_dim, D % 32 == 0, D <= 128; every lane owns D values = D/4 quads):
 *   K stream: lane L owns token t of page G, dims d = 0..D-1; quad q = dims 4q..4q+3.
 *   V stream: lane L owns dims {t + 16 i : i < D/16} of page G; quads in the order (tq = 0..3, i = 0..D/16-1),
 *             quad = tokens 4tq..4tq+3 at dim t + 16 i.
 * Step p of a stream (p = 0 .. D/8 - 1) decodes quads 2p and 2p + 1: joint symbol
 *   j = sum_i big(quad 2p, value i) << i  |  big(quad 2p + 1, value i) << (4 + i).
 *
 * rANS: M = 2^11, state in [2^16, 2^32), 16-bit renormalisation words. One chain of 64 lane states per stream, so
 * a lane advances two independent states (K, V). Decode step (all 64 lanes, step p):
 *   slot = x & 2047; (f, c, j) = table[slot]; x = f * (x >> 11) + c; then the lanes with x < 2^16 read, in
 *   ascending lane order, the next words of the stream: x = (x << 16) | word.  (c = slot - cum[j].)
 * Chains span a group PAIR: the groups 2k and 2k + 1 of one (sequence, KV head) are coded as one chain (the lane
 * states follow the header of group 2k only; group 2k + 1's header says "continues" and its decode starts from the
 * states group 2k ends with). A group may also start a chain of its own (an odd group whose predecessor is stored
 * raw or belongs to another sequence's shared prefix, or an even group with no coded successor). The encoder runs
 * the exact reverse per chain (steps descending over the chain's groups, lanes descending) starting every state at
 * 2^16, so a correct decode ends each chain with all states at 2^16 and each group with every cursor at its
 * stream's word count.
 *
 * Raw bits, per lane and stream, in "sign groups" of 32 values = quads 8s .. 8s + 7 (k = q % 8), seven words each:
 *   N0 (quads k = 0, 1), N1 (k = 2, 3), C0 (k = 0..3), N2 (k = 4, 5), N3 (k = 6, 7), C1 (k = 4..7), S (k = 0..7),
 *   word w of sign group s of lane L at index (7 s + w) * 64 + L.
 * Quad k has a frame r_k = (0, 4, 2, 6, 1, 5, 3, 7)[k]: field bit f of value i (f = 0-3 nibble = |q| & 15,
 * 4-5 crumb = (|q| >> 4) & 3, 6 big, 7 sign) sits at word bit (8 i + r_k + f) mod 32 of the word holding that
 * field (nibbles in N, crumbs in C, signs in S). Rotating the assembled word right by r_k gives the quad's four
 * sign-magnitude bytes (nibbles of quads k, k+1 fill an N word, crumbs of 4 quads a C word, signs of 8 quads the S
 * word, without gaps).
 *
 * Group blob (16-byte aligned, little-endian):
 *   [0]    cf_kv_group_header (64 B)
 *   RANS_HYBRID: if header.chain == 1: [64] lane states u32: K [64], V [64];
 *                then the raw words u32: K (D/32 sign groups x 7 x 64), V (the same);
 *                then the word streams u16 of K and V (word_count[0..1] words each), zero padding to 16 bytes.
 *   INT8:        [64] K symbol bytes q + 128, word (q*64 + L) = the 4 bytes of quad q of lane L; then V the same
 *                way.
 *
 * Table blob (CF_KV_RANS_TABLE_BYTES = 16 KiB): 2048 slot entries of two u32:
 *   lo = f | c << 11 | j << 22     (every symbol has f >= 1, so f <= 1793 fits 11 bits)
 *   hi = spread(j): the big bits in the frames of a quad pair with r = 0 and 4:
 *        sum_i ((j >> i) & 1) << (8 i + 6)  |  ((j >> (4 + i)) & 1) << ((8 i + 10) mod 32)
 *        (the pair of quads 8s + 2m, 8s + 2m + 1 uses it rotated left by the first quad's frame r_{2m}).
 * The batched launch uses table 2h for the K streams and 2h+1 for the V streams of KV head h.
 *
 * Word bound: a decode step reads at most one word per lane, so a group's streams hold at most 16 * D words
 * together (CF_KV_RANS_MAX_GROUP_WORDS at D = 128).
 * Raw fallback: a group that holds a q of -128 (only NaN inputs give one) is stored as an INT8 group instead (its
 * header says so; the other group of its pair then starts a chain of its own); a RANS_HYBRID pool may therefore
 * hold both kinds and the decoder dispatches per group.
 * ------------------------------------------------------------------------------------------------------------ */
#ifndef CHROMOFOLD_KV_CODEC_EXT_H
#define CHROMOFOLD_KV_CODEC_EXT_H

#include <stddef.h>
#include <stdint.h>

#include "chromofold/chromofold.h"

#ifdef __cplusplus
extern "C" {
#endif

#define CF_KV_EXT_ABI_VERSION 4u
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
    uint16_t word_count[2];    /* 16-bit rANS words of the K and V streams of this group (0 for INT8) */
    uint16_t chain;            /* RANS_HYBRID: 1 = the group starts a chain (lane states follow), 0 = it continues
                                  the chain of the group before it (an odd group of its pair) */
    uint16_t reserved;
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
    const uint8_t *tables;       /* RANS_HYBRID: table blobs, CF_KV_RANS_TABLE_BYTES each, 16-byte aligned */
    const float *queries;
    float *output;
    float softmax_scale;
    uint32_t splits;             /* context splits per (sequence, head); 0 = choose */
    void *workspace;
    uint64_t workspace_bytes;
} cf_kv_batched_desc;

/* Bytes of workspace the launch needs for this descriptor (0 when no split is used). Host only. */
uint64_t cf_kv_batched_workspace_bytes(const cf_kv_batched_desc *desc);

/* Host-only validation of a batched descriptor (no device dereference). A pool or table pointer that is not
 * 16-byte aligned is CF_ERR_INVALID_ARGUMENT. */
cf_status cf_kv_validate_batched_desc(const cf_kv_batched_desc *desc);

/* Batched paged attention decode over INT8 or RANS_HYBRID pages. No counterpart in the reference (see above);
 * semantics of one (sequence, query head) equal cf_kv_paged_attention_async with one query row and no tail. */
cf_status cf_kv_paged_attention_batched_async(const cf_kv_batched_desc *desc, void *stream);

/* Allocation-free variant of cf_kv_paged_attention_batched_async: the same launches and results, but the split
 * partials go to a library-owned device array of CF_KV_BATCHED_NOALLOC_SCRATCH_BYTES per GPU instead of
 * desc->workspace (ignored). No counterpart in the reference; it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). It calls no allocator. A
 * descriptor whose cf_kv_batched_workspace_bytes() exceeds that size returns CF_ERR_UNSUPPORTED (use the workspace
 * entry point, or fewer splits). Every call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (concurrent streams or threads) race and must be serialised by the caller. */
#define CF_KV_BATCHED_NOALLOC_SCRATCH_BYTES (8u << 20)
cf_status cf_kv_paged_attention_batched_noalloc_async(const cf_kv_batched_desc *desc, void *stream);

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

/* Joint-symbol histogram of one page's values [token_count, head_dim] in K lane order (accumulates): the big bits
 * of dims 8p .. 8p + 7 of each token (tokens past token_count count as zeros). head_dim % 32 == 0. */
cf_status cf_kv_rans_page_histogram(const float *values, uint32_t token_count, uint32_t head_dim,
                                    uint64_t *hist256);

/* Size bound for one encoded group blob at this head_dim (for pool allocation). */
uint64_t cf_kv_group_blob_max_bytes(uint32_t codec, uint32_t head_dim);

/* Quantise and encode one page group that starts a chain of its own: K and V [page_count * 16, head_dim] fp32
 * (page-major), token_counts[page] (1..16; pages past page_count absent). Tables are host copies of table blobs
 * (RANS_HYBRID). Writes the blob into `blob` (capacity `blob_capacity`) and its size to *blob_bytes. */
cf_status cf_kv_encode_group(uint32_t codec, const float *keys, const float *values, uint32_t page_count,
                             const uint32_t *token_counts, uint32_t head_dim, const uint8_t *k_table,
                             const uint8_t *v_table, uint32_t k_table_index, uint32_t v_table_index, uint8_t *blob,
                             uint64_t blob_capacity, uint64_t *blob_bytes);

/* Batch form: ngroups groups, group i = page_counts[i] pages starting at page first_page[i] of the page-major
 * arrays keys/values ([*][16][head_dim]); table pair heads[i] (may be NULL: 0). continues[i] = 1 codes group i
 * as the second group of a chain pair with group i - 1 (they must be the two groups 2k, 2k + 1 of one sequence
 * and head, so heads[i] == heads[i - 1], and group i - 1 must not itself continue); NULL = every group starts its
 * own chain. Encoded on `threads` host threads (0 = all), packed 16-byte aligned into pool[pool_at ..] in group
 * order; offsets_out[i] = byte offset / 16; *pool_end = first free byte. token_counts is per page (NULL: all 16). */
cf_status cf_kv_encode_groups(uint32_t codec, const float *keys, const float *values, uint64_t ngroups,
                              const uint64_t *first_page, const uint32_t *page_counts, const uint32_t *token_counts,
                              uint32_t head_dim, const uint8_t *tables, const uint32_t *heads,
                              const uint8_t *continues, uint8_t *pool, uint64_t pool_capacity, uint64_t pool_at,
                              uint32_t *offsets_out, uint64_t *pool_end, uint32_t threads);

/* ---- device-side page encoder (sealing on the GPU) --------------------------------------------------------- */

/* Device twin of cf_kv_encode_groups: the same groups quantised and encoded on the GPU, producing the same blobs
 * at the same pool offsets, byte for byte (no counterpart in the reference, whose pages are always sealed on the
 * host: src/runtime/compressed_kv_cache.cu:89-109). Every array argument is DEVICE memory: keys/values (page-major
 * [*][16][head_dim] fp32, 16-byte aligned), first_page/page_counts/heads [ngroups], token_counts per page (NULL:
 * all 16), tables = table_count table blobs (RANS_HYBRID), continues [ngroups] (NULL: none; as in
 * cf_kv_encode_groups), pool (16-byte aligned), offsets_out [ngroups],
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
                                    uint32_t table_count, const uint32_t *heads, const uint8_t *continues,
                                    uint8_t *pool,
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
