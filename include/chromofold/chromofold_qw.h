/* chromofold_qw.h — ADDITIVE: entropy-coded int4 weight matrices for decode-in-matmul on MI355X.
 *
 * The reference's fused matmul (cf_fused_matmul_async, chromofold_extra.h) codes the whole row-major matrix as one
 * block-Huffman stream with a single table and one per-tensor scale; its block-rANS decoder (cf_rans_decode_async)
 * is a separate whole-tensor decode. This format keeps the decode-inside-the-GEMM contract for both entropy coders
 * and lays the matrix out for the gfx950 kernel:
 *   - symbols are int4 values q + zero (zero = 8: q = clamp(rint(w / s), -8, 7)), one scale s per (row, 64-column
 *     segment) = absmax(segment) / 7 (1 when the segment is all zero);
 *   - one code table per band of CF_QW_BAND_ROWS consecutive rows.
 * y[b, m] = sum_k x[b, k] * (sym[m, k] - zero) * scales[m, k / 64]; x is bf16 [batch, cols], y is f32 [batch, rows]
 * and is overwritten. No counterpart in the reference C ABI (the configuration it serves is the reference's
 * decode-in-matmul workload with per-row-block Huffman and rANS tables).
 *
 * CF_QW_CODEC_HUFFMAN
 *   - every (row, 64-column segment) is an independently addressable MSB-first canonical-Huffman code run starting at
 *     bit offsets[row * nseg + segment] of `words` (nseg = ceil(cols / 64));
 *   - tables: per band 16 code lengths (lengths <= 12, 0 = symbol absent; canonical codes are assigned in (length,
 *     symbol) order), 16 bytes per band, 16-byte aligned.
 * CF_QW_CODEC_RANS
 *   - symbols are coded in pairs: pair = sym[c] | sym[c + 1] << 4 (c even), one 256-symbol rANS alphabet per band;
 *     tables: per band the 256 pairs' cumulative starts cum_s (u16, cum_0 = 0, non-decreasing, cum_256 = 4096
 *     implied): pair s has frequency f_s = cum_{s+1} - cum_s out of 4096 (CF_QW_RANS_PROB_BITS = 12);
 *   - a stripe is 256 columns of one band (nstripes = ceil(cols / 256); columns past `cols` and rows past `rows`
 *     hold the pair (zero, zero)). A stripe is one stream of 16-bit words decoded by 64 interleaved lane states:
 *     lane l = 16 g + r (row r of the band) decodes at step t = 0..31 the pair at stripe column
 *     64 (t >> 3) + 16 g + 4 ((t >> 1) & 3) + 2 (t & 1). Decode step of a lane with state x: slot = x & 4095,
 *     s = the pair whose range [cum_s, cum_s + f_s) holds slot, x = f_s * (x >> 12) + slot - cum_s, and if
 *     x < 2^16 then x = (x << 16) | next word. Within a step, the lanes that need a word take the next words of the
 *     stream in lane order. The encoder starts every lane at 2^16, so a fully decoded stripe ends there;
 *     states[(band * nstripes + stripe) * 64 + lane] is the lane's initial state;
 *   - streams are grouped in chunks of CF_QW_CHUNK_STRIPES stripes (4096 columns). A band holds nchunks - 1 slots of
 *     chunk_words 16-bit words and a last slot of last_words; chunk c of band b starts at 16-bit word
 *     b * ((nchunks - 1) * chunk_words + last_words) + c * chunk_words of `words` (16-bit words in little-endian
 *     order inside the 32-bit words), and offsets[band * nstripes + stripe] is the stripe's first 16-bit word
 *     relative to its slot. Fixed slot sizes (the largest over the bands) let the kernel issue a chunk's loads
 *     before reading any offset.
 */
#ifndef CHROMOFOLD_QW_H
#define CHROMOFOLD_QW_H

#include <stddef.h>
#include <stdint.h>

#include "chromofold/chromofold.h"

#ifdef __cplusplus
extern "C" {
#endif

#define CF_QW_ABI_VERSION 3u
#define CF_QW_BAND_ROWS 16u
#define CF_QW_SEG_COLS 64u
#define CF_QW_MAX_CODE_LENGTH 12u
#define CF_QW_CODEC_HUFFMAN 1u
#define CF_QW_CODEC_RANS 2u
#define CF_QW_RANS_PROB_BITS 12u
#define CF_QW_STRIPE_COLS 256u
#define CF_QW_CHUNK_STRIPES 16u
#define CF_QW_MAX_CHUNK_WORDS 32768u /* 64 KiB slots: enough for 4096 x 16 symbols at <= 12 bits per pair */

typedef struct cf_qw_matrix {
  uint32_t struct_size; /* sizeof(cf_qw_matrix) */
  uint32_t abi_version; /* CF_QW_ABI_VERSION */
  uint32_t codec;       /* CF_QW_CODEC_HUFFMAN or CF_QW_CODEC_RANS */
  uint32_t rows;        /* M */
  uint32_t cols;        /* K */
  int32_t zero;         /* symbol of value 0 (8 for int4) */
  uint64_t word_count;  /* 32-bit words of `words` (bounds the decoder's reads) */
  const uint32_t *words;   /* device: code stream */
  const uint32_t *offsets; /* device: HUFFMAN [rows * nseg] bit offsets; RANS [bands * nstripes] slot offsets */
  const uint8_t *tables;   /* device: HUFFMAN [bands * 16] code lengths; RANS [bands * 256] u16 cumulative starts;
                              16-byte aligned */
  const float *scales;     /* device: [rows * nseg] */
  const uint32_t *states;  /* device: RANS [bands * nstripes * 64] initial lane states; HUFFMAN unused (NULL) */
  uint32_t chunk_words;    /* RANS: 16-bit words per slot of a full chunk (a multiple of 8, <= CF_QW_MAX_CHUNK_WORDS;
                              0 when the band has one chunk); HUFFMAN: 0 */
  uint32_t last_words;     /* RANS: 16-bit words of the slot of a band's last chunk (a multiple of 8, > 0,
                              <= CF_QW_MAX_CHUNK_WORDS); HUFFMAN: 0 */
} cf_qw_matrix;

/* Host-side checks of a descriptor (no device access). */
cf_status cf_qw_validate(const cf_qw_matrix *w);

/* y[b, :] for b < batch (device pointers, asynchronous on `stream`). */
cf_status cf_qw_matmul_async(const cf_qw_matrix *w, const uint16_t *x_bf16, float *y, uint32_t batch, void *stream);

/* ---- host encoder (plain C++ on the CPU) ---- */

/* Quantise a row-major f32 matrix: sym[rows * cols] int4 symbols (q + 8), scales[rows * ceil(cols / 64)]. */
cf_status cf_qw_quantize_int4(const float *w, uint32_t rows, uint32_t cols, uint8_t *sym, float *scales);

/* Per-band length-limited canonical-Huffman code lengths (code_lengths[ceil(rows / 16) * 16]); returns the number of
 * 32-bit words the payload needs (0 on bad arguments). */
uint64_t cf_qw_huffman_plan(const uint8_t *sym, uint32_t rows, uint32_t cols, uint8_t *code_lengths);

/* Encode with the planned lengths: words[word_capacity] (zero padded), seg_offsets[rows * ceil(cols / 64)]. */
cf_status cf_qw_huffman_encode(const uint8_t *sym, uint32_t rows, uint32_t cols, const uint8_t *code_lengths,
                               uint32_t *words, uint64_t word_capacity, uint32_t *seg_offsets);

/* rANS plan: per-band pair tables cum[ceil(rows / 16) * 256] (cumulative starts, frequencies summing to 4096; every
 * pair the band holds, padding pairs (zero, zero) included, gets f >= 1) and the slot sizes chunk_words / last_words
 * of the descriptor. `words` then needs bands * ((nchunks - 1) * chunk_words + last_words) / 2 32-bit words. */
cf_status cf_qw_rans_plan(const uint8_t *sym, uint32_t rows, uint32_t cols, uint8_t zero, uint16_t *cum,
                          uint32_t *chunk_words, uint32_t *last_words);

/* rANS encode with the planned tables and slot sizes: words[word_capacity] (slots zero padded),
 * offsets[bands * nstripes], states[bands * nstripes * 64]. */
cf_status cf_qw_rans_encode(const uint8_t *sym, uint32_t rows, uint32_t cols, uint8_t zero, const uint16_t *cum,
                            uint32_t chunk_words, uint32_t last_words, uint32_t *words, uint64_t word_capacity,
                            uint32_t *offsets, uint32_t *states);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* CHROMOFOLD_QW_H */
