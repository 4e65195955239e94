// kv_seam_route.hpp — the decode-shape route of the reference seam (cf_kv_paged_attention_async, kv_legacy.hip),
// implemented in kv_batched.hip next to the batched decode whose per-group decode it reuses.
//
// A seam call with one query row and at most four query heads per KV head (a decode step) has four query vectors
// per KV head. The seam kernel's 64-vector tiles then carry 60 padding vectors, and its workgroups decode each
// page's two rANS chains one after another with nothing to overlap them. The route instead:
//   1. seam_list_kernel: one workgroup per chunk of 256 descriptors lists, for every KV head, the head's pages of
//      the chunk in descriptor order and records per (head, chunk) the page count, whether every such page is a
//      rANS page (the seam's tag) of the call's head_dim with 1..64 tokens and 16-byte aligned tables, and the K/V
//      table pointers of the first;
//   2. seam_group_kernel: each workgroup combines its head's chunk records (the route takes the head when every
//      page qualifies and all share one pair of K/V tables; the first split's workgroup publishes the decision); for
//      a head it takes, each wavefront decodes whole pages with the batched decode's group body (both chains
//      interleaved in one wavefront, QK^T on the GQA heads' MFMA broadcast, P.V on v_mfma_f32_16x16x32_f16) and
//      writes split partials in the seam's layout, slots [0, splits);
//   3. the seam kernel runs for the heads the route did not take (its slots follow), and the seam's merge kernel
//      combines all slots.
// Results follow the seam's rules: tokens in [window begin, query token] of every page; a page whose blob does not
// describe a self-contained group of its head_dim and token count, or whose chains do not end where the encoder
// started, makes its (query row, KV head) NaN; pages wholly outside the visible range are skipped unread.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "chromofold/kv_cuda.h"

namespace cfkv {

// Split slots the seam's merge kernel combines at most (the route's slots plus the seam kernel's).
constexpr uint32_t kSeamMergeMaxSlots = 128;
// Descriptors per list workgroup, KV heads the route serves at most, words of a (head, chunk) record
// (count, refused, K table lo/hi, V table lo/hi, 2 unused).
constexpr uint32_t kRouteChunk = 256;
constexpr uint32_t kRouteMaxHeads = 64;
constexpr uint32_t kRouteInfoWords = 8;
__host__ __device__ inline uint32_t seam_route_chunks(uint32_t page_count) {
  return (page_count + kRouteChunk - 1) / kRouteChunk;
}

// cf_kv_paged_attention_async with the route allowed or not. A caller that knows its pages carry another tag than
// the route takes (the llama adapter seals fixed-width pages) passes false and saves the route's two launches.
cf_status seam_paged_attention(const cf_kv_paged_attention_desc *desc, void *stream, bool allow_route);

// Host-side conditions of the route (the device side decides per KV head).
bool seam_route_applies(const cf_kv_paged_attention_desc &d);
// Context splits the route uses per KV head.
uint32_t seam_route_splits(const cf_kv_paged_attention_desc &d);
// Scratch (u32 words) the route needs: records [kv_heads][chunks][8], lists [kv_heads][page_count] of 16-byte page
// entries (chunk c's pages of a head from c * 256), taken [kv_heads]. The scratch is 16-byte aligned.
uint64_t seam_route_scratch_words(const cf_kv_paged_attention_desc &d);
// Launches steps 1 and 2 on `s`. `taken` (inside `scratch`) is what the seam kernel then reads.
cf_status seam_route_launch(const cf_kv_paged_attention_desc &d, uint32_t splits, float *partial, uint32_t *scratch,
                            hipStream_t s);
// The per-head "taken" flags inside the scratch.
inline const uint32_t *seam_route_taken(const cf_kv_paged_attention_desc &d, const uint32_t *scratch) {
  const uint64_t h = d.kv_head_count;
  return scratch + h * seam_route_chunks(d.page_count) * kRouteInfoWords + 4 * h * d.page_count;
}

}  // namespace cfkv
