// nibble_kv.hpp — host interface of the int4 nibble-page kernels (nibble_kv.hip) shared by the device seal engine,
// the device KV dataplane and the multi-sequence resolver.
//
// Page format (reference src/cuda/device_kv_seal_attention.cu:80-113): K (and V) values of a page flattened as
// [token][kv_head][dim], blocks of block_size values with scale = absmax / 7 (1 for an all-zero block), symbol =
// clamp(rint(x / scale), -8, 7) + 8, two symbols per byte with the even index in the low nibble.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <vector>

#include "chromofold/device_kv_seal_attention.h"

namespace cfnib {

// Device status words of one seal: non-finite counts from the scale pass, saturations from the pack pass.
struct SealStatus {
  unsigned long long nan_values, inf_values, saturated;
};

// Largest supported head_dim (8 dims per lane, at most 32 lanes per token-head row).
constexpr uint32_t kMaxHeadDim = 256;

inline bool head_dim_supported(uint32_t d) { return d >= 8 && d <= kMaxHeadDim && d % 8 == 0; }

// Block scales and non-finite counts of one page's K and V (`values` each); status must be zeroed beforehand.
hipError_t launch_block_scales(const float *k, const float *v, uint32_t values, uint32_t block_size, float *k_scales,
                               float *v_scales, SealStatus *status, hipStream_t stream);
// Quantise + pack both streams with the scales above (values % 8 == 0; payloads 4-byte aligned).
hipError_t launch_pack(const float *k, const float *v, uint32_t values, uint32_t block_size, const float *k_scales,
                       const float *v_scales, uint8_t *k_payload, uint8_t *v_payload, SealStatus *status,
                       hipStream_t stream);
// Strided f16/bf16/f32 view -> fp32 [*, head_count, head_dim] rows starting at token `dst_token`.
hipError_t launch_convert(const cf_device_tensor_view &src, float *dst, uint32_t dst_token, hipStream_t stream);
// Clears `count` SealStatus records with a kernel (safe under graph capture).
hipError_t launch_clear_status(SealStatus *status, uint32_t count, hipStream_t stream);

// Request flags (AttnRequest::flags, AttnItem::flags); 0 = the sealed-page format and causal visibility above.
// A flagged request runs on the VALU kernel, except one with all three (kContractFlags) at head_dim 128, whose
// pages the MFMA kernel reads where it can (kMfmaContract).
constexpr uint32_t kSignedNibbles = 1u;  // payload nibbles are two's-complement int4 (n - 16 for n >= 8)
constexpr uint32_t kOpenWindow = 2u;     // position p visible unless window > 0 and p + window < query position
                                         // (no causal bound; default: p <= q and, with a window, p + window > q)
constexpr uint32_t kRowBlocks = 4u;      // scale blocks counted per (token, KV head) row of ceil(page head_dim /
                                         // block_size) blocks (default: blocks over the page's flat value index);
                                         // pages with a NULL payload / scale pointer or block_size 0 are skipped

// One attention request as the kernel reads it (built on the host, uploaded as a table).
struct AttnItem {
  const void *q;
  uint64_t q_token_stride, q_head_stride, q_elem_stride;
  uint32_t q_type, q_tokens;
  void *out;
  uint64_t o_token_stride, o_head_stride, o_elem_stride;
  uint32_t o_type, nsplit;
  const cf_device_page_descriptor *pages;
  uint32_t page_count;
  uint32_t units_per_split;  // pages (VALU kernel) or 64-token tiles (MFMA kernel) per context split
  uint32_t page_splits;      // splits over the sealed pages; split page_splits is the active page (when present)
  uint32_t mfma_nb;          // 0: the VALU kernel reads the pages; 1/2/4: the MFMA kernel, scale blocks per row;
                             // kMfmaContract: the MFMA kernel reads the pages mfma_page_ok accepts (nibble_page.hpp)
  uint32_t vsplits;          // splits of the VALU kernel over the pages, after the MFMA kernel's page_splits (none
                             // for 1/2/4; for kMfmaContract they take only the pages the MFMA kernel refuses)
  uint32_t vunits;           // pages per VALU split (at most 64)
  uint32_t mfma_cap;         // kMfmaContract: tokens a page may hold on the MFMA path (16 per planned chunk)
  const float *active_k;
  const float *active_v;
  uint32_t active_begin, active_count;
  uint32_t q_begin, window;
  float scale_log2;  // softmax_scale * log2(e)
  uint32_t flags;
  uint64_t ws_offset;  // float offset of the item's split partials
};

struct AttnShape {
  uint32_t kv_heads, q_heads, gqa, head_dim;
  uint32_t page_size;  // tokens per page (pages may hold fewer)
};

// mfma_nb of a batched-items request (all three flags above) on the MFMA path: block size per page, read on the
// device; the kernel runs with one scale per 32-dim quarter of a row.
constexpr uint32_t kContractFlags = kSignedNibbles | kOpenWindow | kRowBlocks;
constexpr uint32_t kMfmaContract = 3u;

// Scale blocks per 128-dim row for the MFMA path (0 = not eligible): block_size 32 / 64 / any multiple of 128.
inline uint32_t mfma_sets(uint32_t head_dim, uint32_t block_size) {
  if (head_dim != 128 || block_size == 0) return 0;
  if (block_size == 32) return 4;
  if (block_size == 64) return 2;
  return block_size % 128 == 0 ? 1 : 0;
}

// Launch of the MFMA kernel over the items whose mfma_nb == nb (nibble_mfma.hip).
hipError_t launch_nib_mfma(uint32_t nb, const AttnItem *items, uint32_t nitems, uint32_t max_page_splits,
                           uint32_t max_qtok, const AttnShape &sh, float *ws, hipStream_t stream);

// Host description of one request before splitting.
struct AttnRequest {
  cf_device_tensor_view query;
  void *output;
  uint32_t output_type;
  uint64_t o_token_stride, o_head_stride, o_elem_stride;
  const cf_device_page_descriptor *pages;  // device table
  uint32_t page_count;
  const float *active_k, *active_v;
  uint32_t active_begin, active_count;
  uint32_t query_begin, window;
  float softmax_scale;
  uint32_t block_size;  // the block size of every page of the request, 0 when mixed or unknown
  uint32_t flags;       // kSignedNibbles | kOpenWindow | kRowBlocks
};

// Runs a batch of requests: the split-context attention launches over every item (the VALU kernel, the MFMA kernel
// per mfma_nb mode), then one merge launch.
// Owns a device workspace (item table + split partials) grown on demand; calls must be ordered on one stream.
class AttnRunner {
 public:
  AttnRunner() = default;
  AttnRunner(const AttnRunner &) = delete;
  AttnRunner &operator=(const AttnRunner &) = delete;
  ~AttnRunner();
  // Returns hipSuccess or the first runtime error; `error` receives a message on failure.
  hipError_t run(const std::vector<AttnRequest> &requests, const AttnShape &shape, hipStream_t stream,
                 std::string &error);
  uint64_t workspace_bytes() const { return bytes_; }
  uint32_t last_launches() const { return launches_; }

 private:
  void *ws_ = nullptr;
  uint64_t bytes_ = 0;
  uint32_t launches_ = 0;
};

size_t scalar_bytes(uint32_t type);

}  // namespace cfnib
