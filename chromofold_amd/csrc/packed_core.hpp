// packed_core.hpp — per-lane primitives of the packed (uncompressed-bitplane) wavelet matrix: rank1 with a
// superblock directory every CF_WAVELET_SB words, access and rank. Semantics of reference
// include/chromofold/detail/access_device.cuh:12-47 and src/cuda/rank.cu:14-52; the FM-index mark plane uses the
// same rank1.
#pragma once

#include "chromofold/chromofold.h"
#include "cf_device.hpp"

namespace cfp {

// set bits of a bitplane over [0, pos): superblock sample + whole-word popcounts + partial word
__device__ __forceinline__ int rank1(const uint32_t *__restrict__ w, const int32_t *__restrict__ sb, int pos) {
  const int word = pos >> 5, bit = pos & 31, blk = word / CF_WAVELET_SB;
  int r = sb[blk];
#pragma unroll
  for (int k = 0; k < CF_WAVELET_SB; ++k)
    if (blk * CF_WAVELET_SB + k < word) r += __popc(w[blk * CF_WAVELET_SB + k]);
  if (bit) r += __popc(w[word] & ((1u << bit) - 1u));
  return r;
}

template <int LEVELS>
__device__ __forceinline__ uint32_t access_one(const cf_wavelet_view &v, int i) {
  const int L = LEVELS > 0 ? LEVELS : static_cast<int>(v.levels);
  uint32_t val = 0;
  for (int lvl = 0; lvl < L; ++lvl) {
    const uint32_t *w = v.bitplanes + static_cast<size_t>(lvl) * v.nwords;
    const int r = rank1(w, v.superblocks + static_cast<size_t>(lvl) * (v.nblocks + 1), i);
    const int b = static_cast<int>((w[i >> 5] >> (i & 31)) & 1u);
    val = (val << 1) | static_cast<uint32_t>(b);
    i = b ? v.zero_counts[lvl] + r : i - r;
  }
  return val;
}

template <int LEVELS>
__device__ __forceinline__ uint32_t rank_one(const cf_wavelet_view &v, int c, int i) {
  const int L = LEVELS > 0 ? LEVELS : static_cast<int>(v.levels);
  int p = 0, q = i;
  for (int lvl = 0; lvl < L; ++lvl) {
    if (p >= q) break;
    const uint32_t *w = v.bitplanes + static_cast<size_t>(lvl) * v.nwords;
    const int32_t *sb = v.superblocks + static_cast<size_t>(lvl) * (v.nblocks + 1);
    const int rp = rank1(w, sb, p), rq = rank1(w, sb, q);
    if ((c >> (L - 1 - lvl)) & 1) {
      p = v.zero_counts[lvl] + rp;
      q = v.zero_counts[lvl] + rq;
    } else {
      p -= rp;
      q -= rq;
    }
  }
  return static_cast<uint32_t>(q - p);
}

}  // namespace cfp
