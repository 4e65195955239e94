// qw_rans.hip — decode-in-matmul over the pair-rANS int4 format (CF_QW_CODEC_RANS, include/chromofold/chromofold_qw.h)
// on gfx950: y[b, m] = sum_k x[b, k] * (sym[m, k] - zero) * scale[m, k / 64], the weight matrix held only in its
// coded form.
//
// One 1024-thread workgroup (16 waves) owns one band of 16 rows and walks K in chunks of 16 stripes (4096 columns);
// wave w decodes stripe w of the chunk, its 64 lanes being the stripe's 64 interleaved rANS states (the code also
// runs 8 waves of two stripes each, decoded together as two chains per lane: measured slower, 9.9 against 9.1 us at
// B = 1):
//   stage    the chunk's slot (fixed size, so its address needs no offset read) is loaded with straight-line 16-byte
//            loads together with the lane states, the stripe offsets, the scales and the first x fragments;
//   table    while those loads are in flight the band's 256 cumulative starts become a 4096-entry LDS table:
//            slot -> {f | (slot - cum) << 16, the pair's two weights as bf16 (sym - zero, exact)};
//   decode   32 steps per lane: table lookup, x = f * (x >> 12) + slot - cum, and a 16-bit renormalisation word
//            for the lanes whose state fell below 2^16, taken from the staged stream at a wave-uniform cursor plus
//            the lane's rank among the lanes that need one (ballot / mbcnt);
//   MFMA     every two steps give a lane 4 consecutive weights of its row: the B operand of one
//            v_mfma_f32_16x16x16_bf16 (lane 16 g + r: row r, k = 4 g..4 g + 3). The stripe's column order puts the
//            same lane's x values in the A operand, so decoded weights never leave the registers; each 64-column
//            segment's 4 MFMAs accumulate apart and the segment's scale multiplies them once;
//   reduce   the waves' partial tiles are summed through LDS in a fixed order and y is written once.
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
constexpr int kPer = CF_QW_CHUNK_STRIPES / kWaves;           // stripes per wave per chunk, decoded together
constexpr int kSlots = 1 << CF_QW_RANS_PROB_BITS;           // 4096 table entries
constexpr int kSlotW16 = CF_QW_MAX_CHUNK_WORDS;              // largest chunk slot, 16-bit words
constexpr int kMaxTiles = 4;

static_assert(kPer * kWaves == CF_QW_CHUNK_STRIPES, "the chunk's stripes split evenly over the waves");
static_assert(kSlotW16 <= 4 * kThreads * 8, "four 16-byte staging loads per thread cover the largest slot");
static_assert(CF_QW_STRIPE_COLS == 256 && CF_QW_BAND_ROWS == 16, "the lane / column map of chromofold_qw.h");

struct RansArgs {
  const uint4 *words;  // as 16-byte units
  const uint32_t *offsets;
  const uint16_t *cums;
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

// The band's table from its cumulative starts (lane L of wave 0 holds cum_4L .. cum_4L+3 in `cw`): entry slot =
// {f | (slot - cum) << 16, the pair's two weights as bf16}. (16-byte entries with f and slot - cum in words of their
// own save two VALU per step but made the decode 1.7x slower: the random lookups' LDS bank conflicts grow with the
// entry size.) Thread t fills
// slots 8t .. 8t + 7, finding each slot's pair by binary search. The largest s with cum_s <= slot has
// cum_s+1 > slot, so the search never lands on an absent pair (f = 0) even when cum repeats.
__device__ void build_table(uint2 cw, int zero, uint2 *__restrict__ tab, uint32_t *__restrict__ s_cum) {
  const int t = threadIdx.x;
  if (t < 64) {
    reinterpret_cast<uint4 *>(s_cum)[t] = make_uint4(cw.x & 0xFFFFu, cw.x >> 16, cw.y & 0xFFFFu, cw.y >> 16);
    if (t == 0) s_cum[256] = kSlots;
  }
  lds_barrier();
  constexpr int kN = kSlots / kThreads;  // slots per thread
#pragma unroll
  for (int half = 0; half < kN / 4; ++half) {
    const uint32_t slot0 = static_cast<uint32_t>(kN * t + 4 * half);
    uint32_t s[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int bit = 7; bit >= 0; --bit)
#pragma unroll
      for (int k = 0; k < 4; ++k) {  // four independent searches: their LDS reads overlap
        const uint32_t c = s[k] + (1u << bit);
        if (s_cum[c] <= slot0 + k) s[k] = c;
      }
    uint32_t ex[4], ey[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t lo = s_cum[s[k]], hi = s_cum[s[k] + 1];
      ex[k] = ((hi - lo) & 0xFFFFu) | ((slot0 + k - lo) << 16);
      ey[k] = bf16_bits(static_cast<int>(s[k] & 15) - zero) | (bf16_bits(static_cast<int>(s[k] >> 4) - zero) << 16);
    }
    uint4 *tab4 = reinterpret_cast<uint4 *>(tab + slot0);
    tab4[0] = make_uint4(ex[0], ey[0], ex[1], ey[1]);
    tab4[1] = make_uint4(ex[2], ey[2], ex[3], ey[3]);
  }
}

// 8 bf16 of x row b from column c (one 16-byte unit), zero for a row past the batch or a column past K: the A
// operands of two MFMAs of lane group g (the general path; FAST loads 16 bytes straight from x).
__device__ __forceinline__ uint4 x_frag8(const uint16_t *__restrict__ x, int b, int B, int c, int K) {
  uint32_t v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = (b < B && c + e < K) ? x[static_cast<int64_t>(b) * K + c + e] : 0u;
  return make_uint4(v[0] | (v[1] << 16), v[2] | (v[3] << 16), v[4] | (v[5] << 16), v[6] | (v[7] << 16));
}

__device__ __forceinline__ bf16x4_t as_bf16x4(uint32_t a, uint32_t b) {  // {a.lo, a.hi, b.lo, b.hi}
  return __builtin_bit_cast(bf16x4_t, make_uint2(a, b));
}

// One decode step of a lane: returns the pair's two weights (bf16 x2); x and the wave's cursor advance.
__device__ __forceinline__ uint32_t rans_step(const uint2 *__restrict__ tab, uint32_t &x,
                                              const uint16_t *__restrict__ &cur) {
  const uint2 e = tab[x & (kSlots - 1)];
  // x = f * (x >> 12) + (slot - cum), f and slot - cum the two 16-bit halves of e.x (SDWA operand selects in inline
  // assembly measured 1.6x slower here than the plain code)
  x = __umul24(e.x & 0xFFFFu, x >> CF_QW_RANS_PROB_BITS) + (e.x >> 16);
  const bool need = x < 65536u;
  const uint64_t m = __builtin_amdgcn_ballot_w64(need);
  const uint32_t idx = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                                 __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u));
  const uint32_t w = cur[idx];  // lanes that need no word read a harmless word inside the staged slot
  cur += __builtin_popcountll(m);
  x = need ? (x << 16) | w : x;
  return e.y;
}

template <int NT, bool FAST, int SL, int XR>
__global__ void __launch_bounds__(kThreads) qw_rans_kernel(RansArgs a) {
  static_assert(kThreads == 1024 && (SL == 2 || SL == 4), "staging loads per thread");
  static_assert(XR == 0 || (NT == 1 && FAST), "x rows staged in LDS: one batch tile, whole stripes");
  __shared__ __attribute__((aligned(16))) uint2 s_tab[kSlots];
  // the chunk slot; reused by the reduction. A stripe's cursor starts at most at the slot's end (clamped) and a step
  // moves it by at most 64, with reads up to 63 words past it: 32 steps stay within kSlotW16 + 64 * 33 words
  // whatever the stream holds.
  __shared__ __attribute__((aligned(16))) uint16_t s_slot[kSlotW16 + 64 * 33];
  __shared__ __attribute__((aligned(16))) uint32_t s_cum[260];
  // XR > 0 (a batch of at most XR rows): the chunk's x columns of rows 0..XR-1, staged once per workgroup (8 bytes
  // per thread and row) instead of every lane loading its 16-byte fragments from global memory, where the 16 row
  // lanes of a lane group would all fetch the same row (B = 1: 9.2 -> 8.8 us per call)
  constexpr int kXCols = CF_QW_CHUNK_STRIPES * CF_QW_STRIPE_COLS;
  __shared__ __attribute__((aligned(16))) uint16_t s_x[XR > 0 ? XR * kXCols : 8];
  static_assert(sizeof(s_slot) >= kWaves * NT * 256 * 4, "reduction fits the slot buffer");

  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);  // in a scalar register: stripe choices are wave-uniform
  const int band = blockIdx.x, m0 = band * 16;
  const int M = a.M, K = a.K, B = a.B;
  const int nseg = (K + 63) / 64;
  const int g = lane >> 4, r = lane & 15;
  const int row = min(m0 + r, M - 1);  // rows past M decode padding and are never written

  f32x4_t acc[NT];
#pragma unroll
  for (int i = 0; i < NT; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const size_t band_words = static_cast<size_t>(a.nchunks - 1) * a.chunk_words + a.last_words;
  for (int ch = 0; ch < a.nchunks; ++ch) {
    const int slot_words = ch + 1 == a.nchunks ? a.last_words : a.chunk_words;
    const int n16 = slot_words / 8;  // 16-byte units of the slot
    // the wave's stripes: wave and wave + kWaves of the chunk (wave-uniform)
    int st[kPer];
    bool active[kPer];
#pragma unroll
    for (int c = 0; c < kPer; ++c) {
      const int stripe = ch * CF_QW_CHUNK_STRIPES + wave + kWaves * c;
      active[c] = stripe < a.nstripes;
      st[c] = min(stripe, a.nstripes - 1);
    }
    // ---- straight-line loads (no branch, no select on a loaded value: either would make the compiler wait for
    // the loads issued before): the band's cumulative starts (first used by the table build; every wave loads
    // them, wave 0 uses them), the slot, the lanes' states, the stripe offsets, scales, first x fragments
    const uint2 cw = reinterpret_cast<const uint2 *>(a.cums + static_cast<size_t>(band) * 256)[lane];
    asm volatile("" ::: "memory");  // issued first: not sunk into the table build, behind the other loads
    const uint4 *slot = a.words + (band * band_words + static_cast<size_t>(ch) * a.chunk_words) / 8;
    // SL unconditional 16-byte loads per thread (clamped addresses: a branch around a load makes the compiler wait
    // for the loads before it) into named registers (a private array here is promoted to LDS and stored there at
    // once); the host picks SL = 2 when the slot fits 2048 16-byte units. (Letting only the first four wavefronts
    // load the whole slot, so that it is in flight earlier, measured slower: their longer prologues delay the
    // table barrier.)
    const uint32_t last = static_cast<uint32_t>(n16 - 1), tt = static_cast<uint32_t>(t);
    const uint4 st0 = slot[min(tt, last)], st1 = slot[min(tt + kThreads, last)];
    uint4 st2 = make_uint4(0, 0, 0, 0), st3 = st2;
    if constexpr (SL == 4) {
      st2 = slot[min(tt + 2 * kThreads, last)];
      st3 = slot[min(tt + 3 * kThreads, last)];
    }
    uint32_t x[kPer], soff[kPer];
    float sc[kPer][4];
#pragma unroll
    for (int c = 0; c < kPer; ++c) {
      x[c] = a.states[(static_cast<size_t>(band) * a.nstripes + st[c]) * 64 + lane];
      soff[c] = min(a.offsets[static_cast<size_t>(band) * a.nstripes + st[c]], static_cast<uint32_t>(slot_words));
    }
    // x fragments by half segment (8 columns of each lane group; half h = 2 q + (j >> 1)) in a ring of XH: one tile
    // holds all 8 halves of both stripes, more tiles prefetch XH - 1 halves ahead of the decode (register budget)
    constexpr int XH = NT == 1 ? 8 : NT == 2 ? 4 : 2;
    uint4 xf[kPer][XH][NT];
    // FAST: 32-bit per-lane offsets from wave-uniform bases (the prologue's address arithmetic is a large part of
    // its issue time, which the wavefronts of a SIMD spend one after another before the first barrier)
    const uint16_t *xb = a.x + static_cast<size_t>(a.bt0) * 16 * K;  // wave-uniform
    uint32_t xoff[NT];
    if constexpr (FAST) {
#pragma unroll
      for (int c = 0; c < kPer; ++c) {  // 4 scales of the lane's row in one 16-byte load (nseg: a multiple of 4)
        const float4 s4 = *reinterpret_cast<const float4 *>(
            a.scales + 4 * st[c] + static_cast<uint32_t>(row) * static_cast<uint32_t>(nseg));
        sc[c][0] = s4.x;
        sc[c][1] = s4.y;
        sc[c][2] = s4.z;
        sc[c][3] = s4.w;
      }
#pragma unroll
      for (int i = 0; i < NT; ++i) {  // rows past the batch read the batch's last row (outputs never written)
        const uint32_t rr = static_cast<uint32_t>(min((a.bt0 + i) * 16 + r, B - 1) - a.bt0 * 16);
        xoff[i] = rr * static_cast<uint32_t>(K) + static_cast<uint32_t>(16 * g);
      }
    } else {
#pragma unroll
      for (int c = 0; c < kPer; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          sc[c][q] = a.scales[static_cast<size_t>(row) * nseg + min(4 * st[c] + q, nseg - 1)];
    }
    auto load_x = [&](int h) {
#pragma unroll
      for (int c = 0; c < kPer; ++c)
#pragma unroll
        for (int i = 0; i < NT; ++i) {
          const int col = st[c] * 256 + 64 * (h >> 1) + 8 * (h & 1);
          if constexpr (XR > 0)
            xf[c][h % XH][i] = *reinterpret_cast<const uint4 *>(
                s_x + min(r, XR - 1) * kXCols + (col - ch * kXCols) + 16 * g);
          else if constexpr (FAST)
            xf[c][h % XH][i] = *reinterpret_cast<const uint4 *>(xb + xoff[i] + col);
          else
            xf[c][h % XH][i] = x_frag8(a.x, (a.bt0 + i) * 16 + r, B, col + 16 * g, K);
        }
    };
    uint2 xs[XR > 0 ? XR : 1];
    if constexpr (XR > 0) {  // x rows 0..XR-1 (rows past the batch repeat its last row), 4 columns per thread
      const int c4 = min(ch * kXCols + 4 * t, K - 4);
#pragma unroll
      for (int rr = 0; rr < XR; ++rr)
        xs[rr] = *reinterpret_cast<const uint2 *>(xb + static_cast<uint32_t>(min(rr, B - 1)) * static_cast<uint32_t>(K) + c4);
    } else {
#pragma unroll
      for (int h = 0; h < XH - 1; ++h) load_x(h);
    }
    // ---- the band's table while the loads are in flight (rebuilt for every chunk: a build under a branch would
    // let the compiler sink the table load into it, behind the others)
    build_table(cw, a.zero, s_tab, s_cum);
    uint4 *s_slot4 = reinterpret_cast<uint4 *>(s_slot);
    const uint32_t n = static_cast<uint32_t>(n16);
    if (tt < n) s_slot4[tt] = st0;
    if (tt + kThreads < n) s_slot4[tt + kThreads] = st1;
    if constexpr (SL == 4) {
      if (tt + 2 * kThreads < n) s_slot4[tt + 2 * kThreads] = st2;
      if (tt + 3 * kThreads < n) s_slot4[tt + 3 * kThreads] = st3;
    }
    if constexpr (XR > 0) {
#pragma unroll
      for (int rr = 0; rr < XR; ++rr) *reinterpret_cast<uint2 *>(s_x + rr * kXCols + 4 * t) = xs[rr];
    }
    __syncthreads();
    if constexpr (XR > 0) {
#pragma unroll
      for (int h = 0; h < XH - 1; ++h) load_x(h);
    }
    // ---- decode + MFMA: the wave's two stripes step together (two independent chains); a stripe past the
    // matrix (last chunk) decodes the matrix's last stripe again and its partials are dropped
    const uint16_t *cur[kPer];
#pragma unroll
    for (int c = 0; c < kPer; ++c) cur[c] = s_slot + __builtin_amdgcn_readfirstlane(soff[c]);  // scalar cursor
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      f32x4_t part[kPer][NT];
#pragma unroll
      for (int c = 0; c < kPer; ++c)
#pragma unroll
        for (int i = 0; i < NT; ++i) part[c][i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int h = 2 * q + (j >> 1);
        if ((j & 1) == 0 && h + XH - 1 < 8) load_x(h + XH - 1);
        uint32_t w0[kPer], w1[kPer];
#pragma unroll
        for (int c = 0; c < kPer; ++c) w0[c] = rans_step(s_tab, x[c], cur[c]);
#pragma unroll
        for (int c = 0; c < kPer; ++c) w1[c] = rans_step(s_tab, x[c], cur[c]);
#pragma unroll
        for (int c = 0; c < kPer; ++c) {
          const bf16x4_t bfrag = as_bf16x4(w0[c], w1[c]);
#pragma unroll
          for (int i = 0; i < NT; ++i) {
            const uint4 &u = xf[c][h % XH][i];
            const bf16x4_t afrag = (j & 1) ? as_bf16x4(u.z, u.w) : as_bf16x4(u.x, u.y);
            part[c][i] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(afrag, bfrag, part[c][i], 0, 0, 0);
          }
        }
      }
#pragma unroll
      for (int c = 0; c < kPer; ++c) {
        if (!active[c]) continue;  // wave-uniform
#pragma unroll
        for (int i = 0; i < NT; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[i][e] += sc[c][q] * part[c][i][e];  // the lane's output column is row r
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
  // four threads per output, each summing a quarter of the waves, then two lane swaps (fixed order throughout)
  static_assert(kWaves % 4 == 0, "four partial sums per output");
  for (int o4 = t; o4 < NT * 256 * 4; o4 += kThreads) {
    const int o = o4 >> 2, part = o4 & 3;
    const int i = o >> 8, idx = o & 255;
    float s = 0.f;
#pragma unroll
    for (int w = part * (kWaves / 4); w < (part + 1) * (kWaves / 4); ++w) s += red[(w * NT + i) * 256 + idx];
    // the quad's four quarter sums by DPP moves (quad_perm [1,0,3,2], then [2,3,0,1]), no LDS round trip
    s += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(s), 0xb1, 0xf, 0xf, false));
    s += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(s), 0x4e, 0xf, 0xf, false));
    const int fl = idx >> 2, fr = idx & 3;
    const int b = (a.bt0 + i) * 16 + 4 * (fl >> 4) + fr, m = m0 + (fl & 15);
    if (part == 0 && b < B && m < M) a.y[static_cast<int64_t>(b) * M + m] = s;
  }
}

template <int NT, bool FAST, int XR>
void launch_rans_sl(const RansArgs &a, unsigned grid, hipStream_t s) {
  if (max(a.chunk_words, a.last_words) <= 2 * kThreads * 8)
    qw_rans_kernel<NT, FAST, 2, XR><<<grid, kThreads, 0, s>>>(a);
  else
    qw_rans_kernel<NT, FAST, 4, XR><<<grid, kThreads, 0, s>>>(a);
}

template <int NT>
void launch_rans(const RansArgs &a, unsigned grid, hipStream_t s) {
  // FAST: whole stripes (K a multiple of 256), a 16-byte aligned x, and every per-lane offset within 32 bits
  // (64 rows of x, and the scales)
  const bool fast = (a.K & 255) == 0 && (reinterpret_cast<uintptr_t>(a.x) & 15) == 0 && a.K <= (1 << 24) &&
                    static_cast<uint64_t>(a.M) * (a.K / 64) < (1ull << 30);
  // a batch of one row stages its x row in LDS (staging four rows for batches of up to four measured slower: 9.6
  // against 9.4 us at B = 4)
  if (fast && NT == 1 && a.B == 1)
    launch_rans_sl<NT, true, NT == 1 ? 1 : 0>(a, grid, s);
  else if (fast)
    launch_rans_sl<NT, true, 0>(a, grid, s);
  else
    launch_rans_sl<NT, false, 0>(a, grid, s);
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
  a.cums = reinterpret_cast<const uint16_t *>(w->tables);
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
