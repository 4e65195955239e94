// gather_core.hpp — wave-cooperative row gather shared by the decode-and-gather kernels (packed-wavelet embedding
// gather, RRR sparse gather, id gather).
//
// Layout choice for wave64: a wave first resolves the row ids of 64 consecutive queries (one per lane, the
// dependent index walk runs 64-wide), then copies those 64 rows with every lane on the copy. Rows of dim4 16-byte
// vectors are packed `64 / p` to a pass, where p = the next power of two >= dim4 capped at 64, so a lane's
// (query, vector) pair comes from shifts and masks and short rows still keep the lanes busy. Row ids travel
// between lanes with ds_bpermute (__shfl with a per-lane source).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace cfg {

// Host side: the vector path needs 16-byte aligned tables/outputs and a row length that is a multiple of 4 floats.
inline bool vec4_ok(const void *src, const void *dst, uint64_t dim) {
  return dim % 4 == 0 && (reinterpret_cast<uintptr_t>(src) & 15u) == 0 && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0;
}

// Copy rows src[id(j) * dim .. +dim) to dst[(q0 + j) * dim ..] for j in [0, nq), nq <= 64; `id` is this lane's row
// id for query q0 + lane (lanes >= nq carry junk and are never read). Every lane of the wave must call this.
template <bool VEC>
__device__ __forceinline__ void copy_rows(uint32_t id, int nq, const float *__restrict__ src, uint64_t dim,
                                          float *__restrict__ dst, uint64_t q0) {
  const int lane = static_cast<int>(threadIdx.x & 63u);
  const uint64_t units = VEC ? dim / 4 : dim;  // 16-byte vectors (or floats) per row
  int shift = 0;                               // p = 1 << shift = min(64, next pow2 >= units)
  while (shift < 6 && (uint64_t(1) << shift) < units) ++shift;
  const int per_pass = 64 >> shift;
  const int sub = lane >> shift;
  const uint64_t e0 = static_cast<uint64_t>(lane & ((1 << shift) - 1));
  for (int j0 = 0; j0 < nq; j0 += per_pass) {
    const int j = j0 + sub;
    const uint32_t row = static_cast<uint32_t>(__shfl(static_cast<int>(id), j < 64 ? j : 63));
    if (j >= nq) continue;
    const uint64_t s = static_cast<uint64_t>(row) * dim, d = (q0 + static_cast<uint64_t>(j)) * dim;
    if constexpr (VEC) {
      const float4 *__restrict__ s4 = reinterpret_cast<const float4 *>(src + s);
      float4 *__restrict__ d4 = reinterpret_cast<float4 *>(dst + d);
      for (uint64_t e = e0; e < units; e += (uint64_t(1) << shift)) d4[e] = s4[e];
    } else {
      for (uint64_t e = e0; e < units; e += (uint64_t(1) << shift)) dst[d + e] = src[s + e];
    }
  }
}

}  // namespace cfg
