/* chromofold.h — primary C ABI (v0) of the MI355X-native chromoFold decode-in-kernel engine.
 *
 * Drop-in for the reference header include/chromofold/chromofold.h: identical macros, enum values, struct layout
 * and function signatures, so callers and bindings written against the reference compile and link unchanged.
 *
 * Contract (reference chromofold.h:1-6):
 *   - every pointer argument is a DEVICE pointer (HBM-resident), owned by the caller;
 *   - no entry point allocates, synchronizes or copies between host and device;
 *   - `stream` is a hipStream_t passed as void* (NULL = the default stream);
 *   - argument validation happens on the host before any device call; a rejected call returns
 *     CF_ERR_INVALID_ARGUMENT (or CF_ERR_UNSUPPORTED for shapes beyond a kernel's limits) and touches nothing;
 *   - CF_ERR_CUDA keeps the reference's name and now means "the HIP runtime rejected the launch".
 */
#ifndef CHROMOFOLD_H
#define CHROMOFOLD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* reference chromofold.h:20-23 */
#define CHROMOFOLD_ABI_VERSION 0
#define CF_WAVELET_SB 8 /* 32-bit words per rank superblock of a packed bitplane */
#define CF_KV_MAX_HEAD_DIM 128
#define CF_KV_MAX_WINDOW 512

/* reference chromofold.h:25-30 */
typedef enum cf_status {
  CF_OK = 0,
  CF_ERR_INVALID_ARGUMENT = 1,
  CF_ERR_UNSUPPORTED = 2,
  CF_ERR_CUDA = 3 /* device runtime (HIP) error */
} cf_status;

/* Packed-wavelet (wavelet-matrix) index, all arrays in device memory (reference chromofold.h:38-46).
 *   bitplanes   [levels * nwords]        u32, bit i of level l = (bitplanes[l*nwords + i/32] >> (i%32)) & 1
 *   superblocks [levels * (nblocks + 1)] i32, cumulative popcount every CF_WAVELET_SB words
 *   zero_counts [levels]                 i32, number of 0-bits per level */
typedef struct cf_wavelet_view {
  const uint32_t *bitplanes;
  const int32_t *superblocks;
  const int32_t *zero_counts;
  uint64_t token_count;
  uint32_t levels;
  uint32_t nwords;
  uint32_t nblocks;
} cf_wavelet_view;

/* Batched access: out[t] = token at positions[t]. Replaces reference chromofold.h:51 (src/cuda/access.cu:21-47). */
cf_status cf_access_async(cf_wavelet_view index, const uint32_t *device_positions,
                          uint32_t *device_output, size_t count, void *stream);

/* Batched rank: out[t] = occurrences of symbols[t] in the first positions[t] tokens.
 * Replaces reference chromofold.h:56 (src/cuda/rank.cu:34-52). */
cf_status cf_rank_async(cf_wavelet_view index, const uint32_t *device_symbols,
                        const uint32_t *device_positions, uint32_t *device_output, size_t count, void *stream);

/* Fused access + embedding-row gather: out[t, :] = embeddings[access(positions[t]), :].
 * Replaces reference chromofold.h:62 (src/cuda/fused_embedding.cu:68-90). */
cf_status cf_embedding_gather_async(cf_wavelet_view index, const float *embeddings, uint32_t dim,
                                    const uint32_t *device_positions, float *out, size_t count, void *stream);

/* Non-paged causal-windowed attention over block-Huffman-coded K (per-channel scale) and V (per-token scale),
 * decoded inside the consumer kernel. Bounds: 0 < dim <= CF_KV_MAX_HEAD_DIM, 0 < window <= CF_KV_MAX_WINDOW,
 * 0 <= nq <= seq, block > 0. Replaces reference chromofold.h:81 (src/cuda/fused_kv_attention.cu:128-142). */
cf_status cf_kv_attn_fused_async(const uint32_t *kw, const int32_t *kb, const int32_t *kl, int kmax,
                                 const uint32_t *vw, const int32_t *vb, const int32_t *vl, int vmax,
                                 const float *kscale, const float *vscale, const float *Q, float *out,
                                 int seq, int dim, int nq, int window, int block, int zero, float sscale,
                                 void *stream);

/* Decode-then-dense twin of cf_kv_attn_fused_async: decodes K/V into caller scratch Kd/Vd [seq, dim] fp32, then
 * runs the same attention. Replaces reference chromofold.h:93 (src/cuda/fused_kv_attention.cu:145-161). */
cf_status cf_kv_attn_dense_async(const uint32_t *kw, const int32_t *kb, const int32_t *kl, int kmax,
                                 const uint32_t *vw, const int32_t *vb, const int32_t *vl, int vmax,
                                 const float *kscale, const float *vscale, const float *Q,
                                 float *Kd, float *Vd, float *out,
                                 int seq, int dim, int nq, int window, int block, int zero, float sscale,
                                 void *stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* CHROMOFOLD_H */
