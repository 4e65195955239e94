// qw_rans.hip — decode-in-matmul over the pair-rANS int4 format (CF_QW_CODEC_RANS, include/chromofold/chromofold_qw.h)
// on gfx950: y[b, m] = sum_k x[b, k] * (sym[m, k] - zero) * scale[m, k / 64], the weight matrix held only in its
// coded form.
//
// One 1024-thread workgroup (16 waves) owns one band of 16 rows and walks K in chunks of 16 stripes (4096 columns);
// wave w decodes stripe w of the chunk, its 64 lanes being the stripe's 64 interleaved rANS states:
//   stage    the chunk's slot (fixed size, so its address needs no offset read) is loaded with straight-line 16-byte
//            loads together with the lane states, the stripe offsets, the scales and the first x fragments;
//   table    while those loads are in flight the band's 256 pair frequencies become a 4096-entry LDS table:
//            slot -> {f | (slot - cum) << 16, the pair's two weights as bf16 (sym - zero, exact)};
//   decode   32 steps per lane: table lookup, x = f * (x >> 12) + slot - cum, and a 16-bit renormalisation word
//            for the lanes whose state fell below 2^16, taken from the staged stream at a wave-uniform cursor plus
//            the lane's rank among the lanes that need one (ballot / mbcnt);
//   MFMA     every two steps give a lane 4 consecutive weights of its row: the B operand of one
//            v_mfma_f32_16x16x16_bf16 (lane 16 g + r: row r, k = 4 g..4 g + 3). The stripe's column order puts the
//            same lane's x values in the A operand, so decoded weights never leave the registers; each 64-column
//            segment's 4 MFMAs accumulate apart and the segment's scale multiplies them once;
//   reduce   the 16 waves' partial tiles are summed through LDS in a fixed order and y is written once.
// Batches above 64 rows run as several launches of up to 4 tiles each.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "cf_device.hpp"
#include "chromofold/chromofold_qw.h"
#include "qw_internal.hpp"

namespace {

typedef short bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kSlots = 1 << CF_QW_RANS_PROB_BITS;           // 4096 table entries
constexpr int kSlotW16 = CF_QW_MAX_CHUNK_WORDS;              // largest chunk slot, 16-bit words
constexpr int kStage = kSlotW16 / 8 / kThreads;             // 16-byte loads per thread for the largest slot
constexpr int kMaxTiles = 4;

static_assert(CF_QW_CHUNK_STRIPES == kWaves, "one stripe per wave per chunk");
static_assert(CF_QW_STRIPE_COLS == 256 && CF_QW_BAND_ROWS == 16, "the lane / column map of chromofold_qw.h");

struct RansArgs {
  const uint4 *words;  // as 16-byte units
  const uint32_t *offsets;
  const uint16_t *freqs;
  const float *scales;
  const uint32_t *states;
  const uint16_t *x;
  float *y;
  int B, M, K, zero, bt0, chunk_words, last_words, nstripes, nchunks;
};

__device__ __forceinline__ uint32_t bf16_bits(int v) {  // |v| <= 15: exact
  return __float_as_uint(static_cast<float>(v)) >> 16;
}

// Barrier for LDS traffic only (waits for this wave's LDS operations, not for its global loads in flight).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt left at their maxima
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// The band's table. Wave 0 turns the 256 frequencies (lane L holds pairs 4L..4L+3 in `fw`) into cumulative starts;
// then 4 threads per pair fill the pair's slot range (every 4th slot each).
__device__ void build_table(uint2 fw, int zero, uint2 *__restrict__ tab, uint32_t *__restrict__ s_cum) {
  const int t = threadIdx.x, lane = t & 63;
  if (t < 64) {
    const uint32_t f0 = fw.x & 0xFFFFu, f1 = fw.x >> 16, f2 = fw.y & 0xFFFFu, f3 = fw.y >> 16;
    const uint32_t own = f0 + f1 + f2 + f3;
    uint32_t incl = own;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const uint32_t v = __shfl_up(incl, d);
      if (lane >= d) incl += v;
    }
    const uint32_t c0 = incl - own;
    s_cum[4 * lane] = c0;
    s_cum[4 * lane + 1] = c0 + f0;
    s_cum[4 * lane + 2] = c0 + f0 + f1;
    s_cum[4 * lane + 3] = c0 + f0 + f1 + f2;
    if (lane == 63) s_cum[256] = incl;
  }
  lds_barrier();
  const int s = t >> 2;
  const uint32_t lo = s_cum[s], hi = min(s_cum[s + 1], static_cast<uint32_t>(kSlots));
  const uint32_t f = hi - lo;
  const uint32_t w = bf16_bits((s & 15) - zero) | (bf16_bits((s >> 4) - zero) << 16);
  for (uint32_t k = lo + (t & 3); k < hi; k += 4) tab[k] = make_uint2(f | ((k - lo) << 16), w);
}

// 8 bf16 of x row b from column c (one 16-byte unit): the A operands of two MFMAs of lane group g.
// FAST: K a multiple of 64 and x 16-byte aligned, so a segment lies wholly inside or outside [0, K).
template <bool FAST>
__device__ __forceinline__ uint4 x_frag8(const uint16_t *__restrict__ x, int b, int B, int c, int K) {
  if constexpr (FAST) {
    const uint4 v = *reinterpret_cast<const uint4 *>(x + static_cast<int64_t>(min(b, B - 1)) * K + min(c, K - 8));
    return c < K ? v : make_uint4(0, 0, 0, 0);
  } else {
    uint32_t v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (b < B && c + e < K) ? x[static_cast<int64_t>(b) * K + c + e] : 0u;
    return make_uint4(v[0] | (v[1] << 16), v[2] | (v[3] << 16), v[4] | (v[5] << 16), v[6] | (v[7] << 16));
  }
}

__device__ __forceinline__ bf16x4_t as_bf16x4(uint32_t a, uint32_t b) {
  bf16x4_t r;
  r[0] = static_cast<short>(a & 0xFFFFu);
  r[1] = static_cast<short>(a >> 16);
  r[2] = static_cast<short>(b & 0xFFFFu);
  r[3] = static_cast<short>(b >> 16);
  return r;
}

// One decode step of a lane: returns the pair's two weights (bf16 x2); x and the wave's cursor advance.
__device__ __forceinline__ uint32_t rans_step(const uint2 *__restrict__ tab, uint32_t &x,
                                              const uint16_t *__restrict__ &cur) {
  const uint2 e = tab[x & (kSlots - 1)];
  x = (e.x & 0xFFFFu) * (x >> CF_QW_RANS_PROB_BITS) + (e.x >> 16);
  const bool need = x < 65536u;
  const uint64_t m = __builtin_amdgcn_ballot_w64(need);
  const uint32_t idx = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                                 __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u));
  const uint32_t w = cur[idx];  // lanes that need no word read a harmless word inside the staged slot
  cur += __builtin_popcountll(m);
  x = need ? (x << 16) | w : x;
  return e.y;
}

template <int NT, bool FAST>
__global__ void __launch_bounds__(kThreads) qw_rans_kernel(RansArgs a) {
  __shared__ __attribute__((aligned(16))) uint2 s_tab[kSlots];
  // the chunk slot; reused by the reduction. A stripe's cursor starts at most at the slot's end (clamped) and a step
  // moves it by at most 64, with reads up to 63 words past it: 32 steps stay within kSlotW16 + 64 * 33 words
  // whatever the stream holds.
  __shared__ __attribute__((aligned(16))) uint16_t s_slot[kSlotW16 + 64 * 33];
  __shared__ uint32_t s_cum[257];
  static_assert(sizeof(s_slot) >= kWaves * NT * 256 * 4, "reduction fits the slot buffer");

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int band = blockIdx.x, m0 = band * 16;
  const int M = a.M, K = a.K, B = a.B;
  const int nseg = (K + 63) / 64;
  const int g = lane >> 4, r = lane & 15;
  const int row = min(m0 + r, M - 1);  // rows past M decode padding and are never written

  f32x4_t acc[NT];
#pragma unroll
  for (int i = 0; i < NT; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // the band's frequencies (wave 0): issued first, first used by the table build
  uint2 fw = make_uint2(0, 0);
  if (wave == 0) fw = reinterpret_cast<const uint2 *>(a.freqs + static_cast<size_t>(band) * 256)[lane];
  const size_t band_words = static_cast<size_t>(a.nchunks - 1) * a.chunk_words + a.last_words;
  for (int ch = 0; ch < a.nchunks; ++ch) {
    const int slot_words = ch + 1 == a.nchunks ? a.last_words : a.chunk_words;
    const int n16 = slot_words / 8;  // 16-byte units of the slot
    const int stripe = ch * kWaves + wave;
    const bool active = stripe < a.nstripes;  // wave-uniform
    const int st = min(stripe, a.nstripes - 1);
    // ---- straight-line loads: the slot, the lane's state, the stripe offset, scales, first x fragments
    const uint4 *slot = a.words + (band * band_words + static_cast<size_t>(ch) * a.chunk_words) / 8;
    static_assert(kStage == 4, "four 16-byte staging loads per thread");
    const uint4 st0 = slot[min(t, n16 - 1)], st1 = slot[min(t + kThreads, n16 - 1)];
    const uint4 st2 = slot[min(t + 2 * kThreads, n16 - 1)], st3 = slot[min(t + 3 * kThreads, n16 - 1)];
    uint32_t x = a.states[(static_cast<size_t>(band) * a.nstripes + st) * 64 + lane];
    const uint32_t soff = min(a.offsets[static_cast<size_t>(band) * a.nstripes + st],
                              static_cast<uint32_t>(slot_words));
    float sc[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) sc[q] = a.scales[static_cast<size_t>(row) * nseg + min(4 * st + q, nseg - 1)];
    // x fragments by half segment (8 columns of each lane group; half h = 2 q + (j >> 1)) in a ring of XH: one tile
    // holds all 8 halves of the stripe, more tiles prefetch XH - 1 halves ahead of the decode (register budget)
    constexpr int XH = NT == 1 ? 8 : NT == 2 ? 4 : 2;
    uint4 xf[XH][NT];
    const int col0 = st * 256 + 16 * g;
    auto load_x = [&](int h) {
#pragma unroll
      for (int i = 0; i < NT; ++i)
        xf[h % XH][i] = x_frag8<FAST>(a.x, (a.bt0 + i) * 16 + r, B, col0 + 64 * (h >> 1) + 8 * (h & 1), K);
    };
#pragma unroll
    for (int h = 0; h < XH - 1; ++h) load_x(h);
    // ---- the band's table (first chunk only) while the loads are in flight
    if (ch == 0) build_table(fw, a.zero, s_tab, s_cum);
    uint4 *s_slot4 = reinterpret_cast<uint4 *>(s_slot);
    if (t < n16) s_slot4[t] = st0;
    if (t + kThreads < n16) s_slot4[t + kThreads] = st1;
    if (t + 2 * kThreads < n16) s_slot4[t + 2 * kThreads] = st2;
    if (t + 3 * kThreads < n16) s_slot4[t + 3 * kThreads] = st3;
    __syncthreads();
    // ---- decode + MFMA
    if (active) {
      const uint16_t *cur = s_slot + soff;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        f32x4_t part[NT];
#pragma unroll
        for (int i = 0; i < NT; ++i) part[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int h = 2 * q + (j >> 1);
          if ((j & 1) == 0 && h + XH - 1 < 8) load_x(h + XH - 1);
          const uint32_t w0 = rans_step(s_tab, x, cur);
          const uint32_t w1 = rans_step(s_tab, x, cur);
          const bf16x4_t bfrag = as_bf16x4(w0, w1);
#pragma unroll
          for (int i = 0; i < NT; ++i) {
            const uint4 &u = xf[h % XH][i];
            const bf16x4_t afrag = (j & 1) ? as_bf16x4(u.z, u.w) : as_bf16x4(u.x, u.y);
            part[i] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(afrag, bfrag, part[i], 0, 0, 0);
          }
        }
#pragma unroll
        for (int i = 0; i < NT; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[i][e] += sc[q] * part[i][e];  // the lane's output column is row r
      }
    }
    __syncthreads();  // slot buffer free for the next chunk (or the reduction)
  }

  // ---- fixed-order cross-wave reduction, one write of y per (b, m)
  float *red = reinterpret_cast<float *>(s_slot);
#pragma unroll
  for (int i = 0; i < NT; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) red[(wave * NT + i) * 256 + lane * 4 + e] = acc[i][e];
  __syncthreads();
  if (t < NT * 256) {
    const int i = t >> 8, idx = t & 255;
    const int fl = idx >> 2, fr = idx & 3;
    const int b = (a.bt0 + i) * 16 + 4 * (fl >> 4) + fr, m = m0 + (fl & 15);
    float s = 0.f;
    for (int w = 0; w < kWaves; ++w) s += red[(w * NT + i) * 256 + idx];
    if (b < B && m < M) a.y[static_cast<int64_t>(b) * M + m] = s;
  }
}

template <int NT>
void launch_rans(const RansArgs &a, unsigned grid, hipStream_t s) {
  if ((a.K & 63) == 0 && (reinterpret_cast<uintptr_t>(a.x) & 15) == 0)
    qw_rans_kernel<NT, true><<<grid, kThreads, 0, s>>>(a);
  else
    qw_rans_kernel<NT, false><<<grid, kThreads, 0, s>>>(a);
}

}  // namespace

namespace cfqw {

cf_status rans_validate(const cf_qw_matrix *w) {
  if (!w->states) return CF_ERR_INVALID_ARGUMENT;
  const uint64_t bands = (w->rows + 15) / 16, nstripes = (static_cast<uint64_t>(w->cols) + 255) / 256;
  const uint64_t nchunks = (nstripes + CF_QW_CHUNK_STRIPES - 1) / CF_QW_CHUNK_STRIPES;
  if (w->chunk_words % 8 != 0 || w->chunk_words > CF_QW_MAX_CHUNK_WORDS || (nchunks > 1 && w->chunk_words == 0))
    return CF_ERR_INVALID_ARGUMENT;
  if (w->last_words == 0 || w->last_words % 8 != 0 || w->last_words > CF_QW_MAX_CHUNK_WORDS)
    return CF_ERR_INVALID_ARGUMENT;
  if ((reinterpret_cast<uintptr_t>(w->words) & 15) != 0) return CF_ERR_INVALID_ARGUMENT;
  if (w->word_count < bands * ((nchunks - 1) * w->chunk_words + w->last_words) / 2) return CF_ERR_INVALID_ARGUMENT;
  return CF_OK;
}

cf_status rans_matmul(const cf_qw_matrix *w, const uint16_t *x, float *y, uint32_t batch, hipStream_t s) {
  RansArgs a{};
  a.words = reinterpret_cast<const uint4 *>(w->words);
  a.offsets = w->offsets;
  a.freqs = reinterpret_cast<const uint16_t *>(w->tables);
  a.scales = w->scales;
  a.states = w->states;
  a.x = x;
  a.y = y;
  a.B = static_cast<int>(batch);
  a.M = static_cast<int>(w->rows);
  a.K = static_cast<int>(w->cols);
  a.zero = w->zero;
  a.chunk_words = static_cast<int>(w->chunk_words);
  a.last_words = static_cast<int>(w->last_words);
  a.nstripes = static_cast<int>((static_cast<uint64_t>(w->cols) + 255) / 256);
  a.nchunks = (a.nstripes + CF_QW_CHUNK_STRIPES - 1) / CF_QW_CHUNK_STRIPES;
  const unsigned grid = cfd::grid_for(a.M, 16);
  const int tiles = (a.B + 15) / 16;
  for (int bt0 = 0; bt0 < tiles; bt0 += kMaxTiles) {
    a.bt0 = bt0;
    switch (min(kMaxTiles, tiles - bt0)) {
      case 1: launch_rans<1>(a, grid, s); break;
      case 2: launch_rans<2>(a, grid, s); break;
      case 3: launch_rans<3>(a, grid, s); break;
      default: launch_rans<4>(a, grid, s); break;
    }
    const cf_status ls = cfd::launch_status();
    if (ls != CF_OK) return ls;
  }
  return CF_OK;
}

}  // namespace cfqw
