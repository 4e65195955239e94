/* chromofold_extra.h — the reference's benchmark-level `extern "C"` entry points, declared in one header.
 *
 * The reference declares each of these locally in its benchmark drivers (the benchmark drivers) rather than in a public
 * header; they are exported here with the same names, argument order and meaning so those drivers, and bindings
 * written against them, link unchanged. Same contract as chromofold.h: device pointers owned by the caller, no
 * allocation, no synchronisation, host-side argument checks before any device call, `stream` is a hipStream_t
 * (NULL = default stream), CF_ERR_CUDA = the HIP runtime rejected the launch.
 */
#ifndef CHROMOFOLD_EXTRA_H
#define CHROMOFOLD_EXTRA_H

#include <stddef.h>
#include <stdint.h>

#include "chromofold/chromofold.h"
#include "chromofold/chromofold_search.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Packed-wavelet rank over a two-level directory: coarse[level * ncoarse + word / CB] (i32) plus
 * fine[level * (nwords + 1) + word] (u16, within-sample prefix, one sentinel per level), then one partial popcount.
 * Same answers as cf_rank_async. CB must be > 0. Replaces reference src/cuda/rank.cu:88-111 (declared at
 * benchmarks/rank_bench.cu:26). */
cf_status cf_rank2_async(cf_wavelet_view index, const int32_t *coarse, const uint16_t *fine, int ncoarse, int CB,
                         const uint32_t *device_symbols, const uint32_t *device_positions, uint32_t *device_output,
                         size_t count, void *stream);

/* Same output as cf_embedding_gather_async (the reference's thread-per-query variant; here both share the
 * wave-cooperative gather). Replaces reference src/cuda/fused_embedding.cu:41-66 (benchmarks/fused_embedding.cu:38). */
cf_status cf_embedding_gather_tpq_async(cf_wavelet_view index, const float *embeddings, uint32_t dim,
                                        const uint32_t *device_positions, float *out, size_t count, void *stream);

/* rank1 of a single RRR bitvector (T = 15-bit blocks, 64 blocks per sample): class nibbles LSB-first, offsets
 * LSB-first, sbrank/sboff one i32 per superblock. `width` and `binom` are fixed by the format and not read.
 * Replaces reference src/cuda/rrr.cu:75-85 (benchmarks/rrr_bench.cu:24). */
cf_status cf_rrr_rank_async(const uint32_t *classes, const uint32_t *offsets, const int32_t *sbrank,
                            const int32_t *sboff, const int *width, const int *binom, const uint32_t *positions,
                            uint32_t *out, size_t count, void *stream);

/* Delta-cluster fetch: out[t] = delta of leaf[t] at pos[t] if its sorted dpos[dstart[leaf] .. +dlen[leaf]) holds
 * pos[t] (the first such entry when positions repeat), else base[pos[t]] (or -1 when pos[t] >= nbase or
 * pos[t] < 0; the reference reads before the array for a negative position). Replaces reference
 * src/cuda/delta_apply.cu:33-43 (benchmarks/delta_bench.cu:25). */
cf_status cf_delta_fetch_async(const int32_t *base, int nbase, const int32_t *dpos, const int32_t *dval,
                               const int32_t *dstart, const int32_t *dlen, const int32_t *device_leaf,
                               const int32_t *device_pos, int32_t *out, size_t count, void *stream);

/* RRR-wavelet access fused with an embedding-row gather: out[t, :] = emb[access(pos[t]), :] (rows of `dim` f32).
 * Replaces reference src/cuda/sparse_gather.cu:55-66 (benchmarks/sparse_gather.cu:26). */
cf_status cf_sparse_gather_fused_async(cf_rrrw_view v, const float *emb, int dim, const uint32_t *pos, float *out,
                                       size_t K, void *stream);

/* Every token id of the RRR wavelet: ids[t] = access(t), t < n. Replaces reference src/cuda/sparse_gather.cu:68-79. */
cf_status cf_sparse_decode_all_async(cf_rrrw_view v, uint32_t *ids, size_t n, void *stream);

/* Gather through decoded ids: out[t, :] = emb[ids[pos[t]], :]. Replaces reference src/cuda/sparse_gather.cu:81-91
 * (benchmarks/sparse_gather.cu:29). */
cf_status cf_sparse_gather_async(const uint32_t *ids, const float *emb, int dim, const uint32_t *pos, float *out,
                                 size_t K, void *stream);

/* Whole-tensor block-rANS decode: n symbols in blocks of `block`, block b starting at byte byte_off[b] of `data` with
 * state state0[b]; 12-bit tables slot2sym[4096], freq[V], cum[V]; out i32[n]. block must be > 0.
 * Replaces reference src/cuda/rans.cu:40-50 (benchmarks/rans_bench.cu:24). */
cf_status cf_rans_decode_async(const uint8_t *data, const int32_t *byte_off, const uint32_t *state0,
                               const int32_t *slot2sym, const int32_t *freq, const int32_t *cum, int block, int n,
                               int32_t *out, void *stream);

/* Decode-in-matmul: y[b, m] = sum_k x[b, k] * ((q[m, k] - zero) * scale) for b < B, m < M, k < K, where q is the
 * row-major M x K int symbol matrix held as ONE block-Huffman stream (MSB-first codes, `block` symbols per
 * block_off entry, lut[2^maxlen] = symbol | code_length << 8). x [B, K] f32, y [B, M] f32 (overwritten). The dense
 * weight matrix never exists in memory. Replaces reference src/cuda/fused_matmul.cu:67-80
 * (benchmarks/fused_matmul.cu:26). */
cf_status cf_fused_matmul_async(const uint32_t *words, const int32_t *block_off, const int32_t *lut, int maxlen,
                                int block, const float *x, float *y, int B, int M, int K, float scale, int zero,
                                void *stream);

/* Materialising twin: decodes W [M, K] f32 into caller scratch `W`, then y = x W^T. Bit-identical to
 * cf_fused_matmul_async. Replaces reference src/cuda/fused_matmul.cu:83-96 (benchmarks/fused_matmul.cu:29). */
cf_status cf_dense_matmul_async(const uint32_t *words, const int32_t *block_off, const int32_t *lut, int maxlen,
                                int block, const float *x, float *W, float *y, int B, int M, int K, float scale,
                                int zero, void *stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* CHROMOFOLD_EXTRA_H */
