// kv_group_decode.hpp — device primitives of the format-4 group decode (kv_codec_ext.h), shared by the batched
// decode (kv_batched.hip) and the reference seam's rANS page path (kv_legacy.hip).
#pragma once

#include <cstdint>

#include "chromofold/kv_codec_ext.h"

namespace cfkv {

constexpr uint32_t kSlots = 1u << CF_KV_RANS_PROB_BITS;
constexpr int kHdr = 64;                 // group header bytes
constexpr int kStateBytes = 2 * 64 * 4;  // K and V lane states of a chain start

// u32 raw words of one stream of a RANS group: 7 per sign group (32 values of a lane) per lane
__host__ __device__ constexpr int raw_words_of(int D) { return 7 * (D / 32) * 64; }

// (a & mask) | (b & ~mask) in one v_bfi_b32
__device__ __forceinline__ uint32_t bfi(uint32_t mask, uint32_t a, uint32_t b) {
  uint32_t r;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "s"(mask), "v"(a), "v"(b));
  return r;
}

// rANS decode of one 64-lane stream, split in three so that the two chains of a lane overlap their LDS round
// trips: the slot entry lookups of both chains are issued first, then the state updates with their
// renormalisation-word fetches, then the word merges. x = lane state; wbase = wave-uniform address of the current
// word (cursor) of the stream staged in LDS. The slot entry is {f | c << 16, spread big bits}.
__device__ __forceinline__ uint2 rans_lookup(const uint2 *__restrict__ tab, uint32_t x) {
  return tab[x & (kSlots - 1)];
}

template <typename WordPtr>
__device__ __forceinline__ uint32_t rans_advance(uint32_t ex, uint32_t &x, WordPtr &wbase, uint32_t &sel) {
  // x = f * (x >> 11) + c with f, c the two 16-bit halves of ex, read in place by SDWA operand selects
  const uint32_t xs = x >> CF_KV_RANS_PROB_BITS;
  uint32_t fx;
  asm("v_mul_u32_u24_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:DWORD"
      : "=v"(fx) : "v"(ex), "v"(xs));
  asm("v_add_u32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:WORD_1 src1_sel:DWORD"
      : "=v"(x) : "v"(ex), "v"(fx));
  const bool need = x < 65536u;
  const uint64_t m = __builtin_amdgcn_ballot_w64(need);
  const uint32_t idx = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                                 __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u));
  const uint32_t w = wbase[idx];  // lanes that do not renormalise read a harmless in-bounds word
  wbase += __builtin_popcountll(m);
  sel = need ? 0x05040100u : 0x07060504u;  // (x << 16) | w  or  x
  return w;
}

// ---- format-4 value assembly (kv_codec_ext.h): quad k of a sign group sits in frame r = kFrame[k]
constexpr uint32_t kFrame[8] = {0, 4, 2, 6, 1, 5, 3, 7};
constexpr uint32_t kNWord[4] = {0, 1, 3, 4};  // raw word with the nibbles of quads 2m, 2m + 1 (N0 N1 C0 N2 N3 C1 S)
constexpr uint32_t rotl_c(uint32_t v, uint32_t r) { return r ? (v << r) | (v >> (32 - r)) : v; }

template <uint32_t R>
__device__ __forceinline__ uint32_t rotr(uint32_t v) {
  if constexpr (R == 0) return v;
  else return __builtin_amdgcn_alignbit(v, v, R);
}

// The magnitude bytes |q| (bit 7 clear) of the quad in frame R: nibbles from n, crumbs from c, big bits from the
// pair's spread word (already in the pair's frames), then rotated back to byte alignment.
template <uint32_t R>
__device__ __forceinline__ uint32_t quad_mag(uint32_t n, uint32_t c, uint32_t spread) {
  return rotr<R>(bfi(rotl_c(0x0F0F0F0Fu, R), n, bfi(rotl_c(0x30303030u, R), c, spread)));
}

// The sign bytes (0x80 or 0x00) of the quad in frame R.
template <uint32_t R>
__device__ __forceinline__ uint32_t quad_signs(uint32_t s) { return rotr<R>(s) & 0x80808080u; }

}  // namespace cfkv
