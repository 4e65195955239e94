// nibble_page.hpp — which caller-held nibble pages the MFMA kernel (nibble_mfma.hip) reads for a batched-items
// request (production_attention.h semantics). The MFMA kernel takes every page this accepts and the VALU kernel
// (nibble_kv.hip) every page it refuses, both testing the same descriptor fields on the device, so a request's
// pages are split between the two kernels without the host reading the page table.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace cfnib {

// A page the MFMA kernel can read: both payloads 16-byte aligned (its rows are staged by 16-byte copies) and both
// scale arrays present; head_dim 128 (its row is the kernel's 64-byte row); a block size that is a non-zero
// multiple of 32, so that each 32-dim quarter of a row (one accumulator chain of that kernel) lies in one scale
// block; at most `cap` tokens (the 16-token chunks per page the launch plans for).
__device__ __forceinline__ bool mfma_page_ok(const void *kp, const void *vp, const float *ks, const float *vs,
                                             uint32_t block_size, uint32_t head_dim, uint32_t token_count,
                                             uint32_t cap) {
  const uintptr_t pa = reinterpret_cast<uintptr_t>(kp) | reinterpret_cast<uintptr_t>(vp);
  return kp && vp && ks && vs && (pa & 15u) == 0u && head_dim == 128u && block_size != 0u &&
         (block_size & 31u) == 0u && token_count <= cap;
}

}  // namespace cfnib
