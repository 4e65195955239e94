/* chromofold_qw.h — ADDITIVE: entropy-coded int4 weight matrices for decode-in-matmul on MI355X.
 *
 * The reference's fused matmul (cf_fused_matmul_async, chromofold_extra.h) codes the whole row-major matrix as one
 * block-Huffman stream with a single table and one per-tensor scale. This format keeps its decode-inside-the-GEMM
 * contract but is laid out for the gfx950 kernel:
 *   - symbols are int4 values q + zero (zero = 8: q = clamp(rint(w / s), -8, 7)), one scale s per (row, 64-column
 *     segment) = absmax(segment) / 7 (1 when the segment is all zero);
 *   - every (row, 64-column segment) is an independently addressable MSB-first canonical-Huffman code run starting at
 *     bit seg_offsets[row * ceil(cols / 64) + segment] of `words`;
 *   - one code table per band of CF_QW_BAND_ROWS consecutive rows, stored as 16 code lengths (lengths <= 12,
 *     0 = symbol absent; canonical codes are assigned in (length, symbol) order), 16 bytes per band.
 * y[b, m] = sum_k x[b, k] * (sym[m, k] - zero) * scales[m, k / 64]; x is bf16 [batch, cols], y is f32 [batch, rows]
 * and is overwritten. No counterpart in the reference C ABI (the configuration it serves is the reference's
 * decode-in-matmul workload with per-row-block tables); the kernel is shared with cf_fused_matmul_async.
 */
#ifndef CHROMOFOLD_QW_H
#define CHROMOFOLD_QW_H

#include <stddef.h>
#include <stdint.h>

#include "chromofold/chromofold.h"

#ifdef __cplusplus
extern "C" {
#endif

#define CF_QW_ABI_VERSION 2u
#define CF_QW_BAND_ROWS 16u
#define CF_QW_SEG_COLS 64u
#define CF_QW_MAX_CODE_LENGTH 12u
#define CF_QW_CODEC_HUFFMAN 1u

typedef struct cf_qw_matrix {
  uint32_t struct_size; /* sizeof(cf_qw_matrix) */
  uint32_t abi_version; /* CF_QW_ABI_VERSION */
  uint32_t codec;       /* CF_QW_CODEC_HUFFMAN */
  uint32_t rows;        /* M */
  uint32_t cols;        /* K */
  int32_t zero;         /* symbol of value 0 (8 for int4) */
  uint64_t word_count;  /* 32-bit words of `words` (bounds the decoder's read-ahead) */
  const uint32_t *words;        /* device: code stream */
  const uint32_t *seg_offsets;  /* device: [rows * ceil(cols / 64)] bit offsets */
  const uint8_t *code_lengths;  /* device: [ceil(rows / 16) * 16], 16-byte aligned */
  const float *scales;          /* device: [rows * ceil(cols / 64)] */
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

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* CHROMOFOLD_QW_H */
