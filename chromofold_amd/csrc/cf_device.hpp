// cf_device.hpp — device-side building blocks shared by the gfx950 kernels of libchromofold.
//
// Everything here is written for the CDNA4 wave64 execution model: lane masks are 64-bit, cross-lane sums use
// ballot/mbcnt, and tables that every lane indexes at random are either compile-time constants (read through the
// scalar or vector cache) or staged into LDS by the kernel that needs them.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "chromofold/chromofold.h"

namespace cfd {

// ------------------------------------------------------------------------------------------------ launch helpers
inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

// Status of the launch just issued: a launch-configuration error is reported synchronously as CF_ERR_CUDA
// (the name is kept for ABI compatibility; it means "the HIP runtime rejected the call").
inline cf_status launch_status() { return hipPeekAtLastError() == hipSuccess ? CF_OK : CF_ERR_CUDA; }

inline unsigned grid_for(size_t work, unsigned per_block) {
  return static_cast<unsigned>((work + per_block - 1) / per_block);
}

// ------------------------------------------------------------------------------------------------ RRR constants
// T = 15-bit blocks, S = 64 blocks per rank superblock, K = 32 superblocks per int32 anchor. These are baked into
// the .cfrw/.cffm formats (reference include/chromofold/detail/rrr_wavelet_device.cuh:16-18).
constexpr int kRrrT = 15;
constexpr int kRrrS = 64;
constexpr int kRrrK = 32;

struct RrrTables {
  // width[k] = ceil(log2 C(15,k)), 0 when C(15,k) <= 1 — the enumerative-offset width of a class-k block.
  int width[16];
  // base[k] = sum_{j<k} C(15,j): start of class k inside the unrank table.
  int base[17];
  // unrank[base[k] + r] = the 15-bit word with k ones whose combinatorial-number-system rank is r
  // (rank = sum over set bit positions c, taken in increasing order with i = 1..k, of C(c, i)).
  uint16_t unrank[1 << kRrrT];
};

constexpr int64_t binom_ce(int n, int k) {
  if (k < 0 || k > n) return 0;
  int64_t r = 1;
  for (int i = 1; i <= k; ++i) r = r * (n - k + i) / i;
  return r;
}

constexpr RrrTables make_rrr_tables() {
  RrrTables t{};
  int64_t C[16][16] = {};
  for (int n = 0; n < 16; ++n) {
    C[n][0] = 1;
    for (int k = 1; k <= n; ++k) C[n][k] = C[n - 1][k - 1] + C[n - 1][k];
  }
  int at = 0;
  for (int k = 0; k <= 15; ++k) {
    const int64_t c = C[kRrrT][k];
    int w = 0;
    while ((int64_t(1) << w) < c) ++w;
    t.width[k] = c > 1 ? w : 0;
    t.base[k] = at;
    at += static_cast<int>(c);
  }
  t.base[16] = at;
  // Enumerate every 15-bit word once and drop it at its class/rank slot: the rank of a word with set positions
  // c_1 < c_2 < ... < c_k is sum_i C(c_i, i) (the encoder's formula, reference tools/build_index.cpp:90-148).
  for (int word = 0; word < (1 << kRrrT); ++word) {
    int k = 0;
    int64_t r = 0;
    for (int c = 0; c < kRrrT; ++c)
      if ((word >> c) & 1) {
        ++k;
        r += C[c][k];
      }
    t.unrank[t.base[k] + r] = static_cast<uint16_t>(word);
  }
  return t;
}

// Widths packed 4 bits per class (class 0 in the low nibble); lets a lane look a width up without memory.
constexpr uint64_t make_width_nibbles() {
  const RrrTables t = make_rrr_tables();
  uint64_t v = 0;
  for (int k = 0; k < 16; ++k) v |= static_cast<uint64_t>(t.width[k]) << (4 * k);
  return v;
}

constexpr uint64_t kWidthNibbles = make_width_nibbles();

// Sum of the 8 nibbles of x (8 block classes in one class word).
__device__ __forceinline__ int nibble_sum(uint32_t x) {
  // popcount of each bit plane weighted by its bit value
  return __popc(x & 0x11111111u) + 2 * __popc(x & 0x22222222u) + 4 * __popc(x & 0x44444444u) +
         8 * __popc(x & 0x88888888u);
}

// Sum over the 8 nibbles k of x of width[k]. width is symmetric (width[k] == width[15-k]) so it is a function of
// m = min(k, 15-k) in 0..7: width = 4[m>=1] + 3[m>=2] + 2[m>=3] + 2[m>=4] + [m>=5] + [m>=6]. Each indicator is
// counted across all 8 nibbles at once: (m + 8 - t) has its nibble bit 3 set exactly when m >= t.
__device__ __forceinline__ int nibble_width_sum(uint32_t x) {
  const uint32_t hi = (x >> 3) & 0x11111111u;     // 1 in every nibble whose class is >= 8
  const uint32_t m = (x ^ (hi * 15u)) & 0x77777777u;  // min(k, 15-k) per nibble
  const uint32_t H = 0x88888888u;
  int s = 4 * __popc((m + 0x77777777u) & H);  // m >= 1
  s += 3 * __popc((m + 0x66666666u) & H);     // m >= 2
  s += 2 * __popc((m + 0x55555555u) & H);     // m >= 3
  s += 2 * __popc((m + 0x44444444u) & H);     // m >= 4
  s += __popc((m + 0x33333333u) & H);         // m >= 5
  s += __popc((m + 0x22222222u) & H);         // m >= 6
  return s;
}

__device__ __forceinline__ int width_of(int k) { return static_cast<int>((kWidthNibbles >> (4 * k)) & 15u); }

// Max / sum over the 16 lanes of a row (every lane of the row gets the result) with DPP moves inside the row:
// quad_perm [1,0,3,2], [2,3,0,1], then row_half_mirror and row_mirror (a ds_bpermute per step would put an LDS
// round trip on a softmax's dependency chain).
template <int CTRL>
__device__ __forceinline__ float dpp_row(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row16_max(float x) {
  x = fmaxf(x, dpp_row<0xb1>(x));
  x = fmaxf(x, dpp_row<0x4e>(x));
  x = fmaxf(x, dpp_row<0x141>(x));
  return fmaxf(x, dpp_row<0x140>(x));
}
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_row<0xb1>(x);
  x += dpp_row<0x4e>(x);
  x += dpp_row<0x141>(x);
  return x + dpp_row<0x140>(x);
}

// Max / sum over the lanes {l, l ^ 16, l ^ 32, l ^ 48} (the same position in the four rows; every lane gets the
// result) with gfx950's v_permlane16_swap / v_permlane32_swap, VALU exchanges that keep an LDS round trip
// (ds_bpermute) off a softmax's dependency chain. Bit-identical to the xor-16 / xor-32 shuffle reductions: each
// step combines the same pair of values in every lane. The max is a plain v_max_f32 (fmaxf would first canonicalise
// both operands).
__device__ __forceinline__ float vmax_f32(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float rows4_max(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = vmax_f32(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return vmax_f32(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float rows4_sum(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Global-address-space view of a generic pointer (one read from a struct or from LDS): its loads become global_load
// (vmcnt only) instead of flat_load, which also counts in lgkmcnt, so that every wait for an LDS access would wait
// for those loads too.
#ifndef CF_GLOBAL
#define CF_GLOBAL __attribute__((address_space(1)))
#endif
template <typename T>
__device__ __forceinline__ const CF_GLOBAL T *global_ptr(const T *p) {
  return (const CF_GLOBAL T *)p;  // an address-space conversion (C-style cast)
}

// a * b as f16 hi + lo (hi + lo = the product to about 21 bits), the MFMA operands of fp32-grade inputs.
// hi comes from one explicit conversion (round toward zero) whose result is both stored and subtracted. Written as
// (half)(a * b), the compiler may form the subtracted hi as v_fma_mix (one rounding of the exact product) and the
// stored hi as v_cvt_pk_f16_f32 of the fp32 product (two roundings); they differ by an f16 ulp when the double
// rounding crosses a tie, and hi + lo then misses the product by that ulp (measured: 2e-4 relative on a few
// attention rows). Pragmas do not stop it: hipcc contracts with -ffp-contract=fast.
__device__ __forceinline__ void split_mul_f16(float a, float b, _Float16 &hi, _Float16 &lo) {
  const float x = a * b;
  const _Float16 h = static_cast<_Float16>(__builtin_amdgcn_cvt_pkrtz(x, 0.0f)[0]);
  hi = h;
  lo = static_cast<_Float16>(x - static_cast<float>(h));
}

// Two products a0 * b and a1 * b split the same way, with one packed round-toward-zero conversion for both hi parts
// and each lo part from a fused multiply-add of the exact product minus its hi (hi + lo then misses a * b by at most
// the rounding of lo): 5 VALU for the pair instead of 8.
__device__ __forceinline__ void split2_mul_f16(float a0, float a1, float b, _Float16 &hi0, _Float16 &lo0,
                                               _Float16 &hi1, _Float16 &lo1) {
  const auto h = __builtin_amdgcn_cvt_pkrtz(a0 * b, a1 * b);
  hi0 = static_cast<_Float16>(h[0]);
  hi1 = static_cast<_Float16>(h[1]);
  lo0 = static_cast<_Float16>(__builtin_fmaf(a0, b, -static_cast<float>(h[0])));
  lo1 = static_cast<_Float16>(__builtin_fmaf(a1, b, -static_cast<float>(h[1])));
}

}  // namespace cfd
