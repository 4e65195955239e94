// quads_core.hpp — a 4-ary wavelet matrix of a sequence, derived on the device from an RRR wavelet matrix (the
// binary levels stay as they are), and the rank primitives over it.
//
// Symbols of `bits` bits are read as L4 = ceil(bits / 2) base-4 digits, most significant first (the top digit of an
// odd `bits` is 0 or 1). Level l holds the sequence's digit l in the order of a wavelet matrix: level 0 in sequence
// order, level l + 1 the positions of level l stably sorted by their digit l (digit 0 first, then 1, 2, 3). With
// Z_l[d] = number of positions of level l whose digit is below d, the walk of a position maps a to
// Z_l[d] + rank_d(l, a). A query walks L4 levels instead of the binary matrix's `bits`: 8 records instead of 15 at
// bits 15, and it is the record reads (one L2 request each) that bound these walks.
//
// Level l's digits are stored as records of 16 u32 = 64 bytes:
//   words 0..2   how many of digits 0, 1, 2 lie in positions [0, 208 r) of the level (digit 3: the rest)
//   words 3..15  positions [208 r, 208 r + 208) of the level, 16 digits per word, digit j at bits 2j..2j+1
// After the L4 levels: Z [L4][4] (u32), then base[c] = (X ? X[c] : 0) - e(c) for c < nsym, e(c) = the end of the
// walk of symbol c from position 0, so that rank(c, i) = a_L(i) - e(c) and the FM-index's LF(i) = a_L(i) + base[c]
// (the walk of c's start chain never depends on i; the same property the binary line layout uses).
#pragma once

#include <hipcub/hipcub.hpp>

#include "chromofold/chromofold_search.h"
#include "cf_device.hpp"
#include "rrr_core.hpp"

namespace cfq {

constexpr uint32_t kDigits = 208;  // digits per record
constexpr uint32_t kRecWords = 16;
constexpr unsigned kBuildThreads = 256;

__host__ __device__ inline uint32_t levels_for(int bits) { return static_cast<uint32_t>(bits + 1) / 2u; }
// Records per level when positions up to and including `n` must resolve.
__host__ __device__ inline uint32_t nrec_for(uint64_t n) { return static_cast<uint32_t>(n / kDigits) + 1u; }

__device__ __forceinline__ void load_record(const uint32_t *__restrict__ rec, uint32_t (&w)[16]) {
  const uint4 *q = reinterpret_cast<const uint4 *>(rec);
  const uint4 a = q[0], b = q[1], c = q[2], d = q[3];
  w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
  w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
  w[8] = c.x; w[9] = c.y; w[10] = c.z; w[11] = c.w;
  w[12] = d.x; w[13] = d.y; w[14] = d.z; w[15] = d.w;
}

// The digit at payload position `off` (< 208) of a record.
__device__ __forceinline__ uint32_t record_digit(const uint32_t (&w)[16], uint32_t off) {
  return (w[3 + min(off >> 4, 12u)] >> ((off & 15u) * 2u)) & 3u;
}

// Digits d of the level in positions [0, 208 r + off): the record's count before it plus the matches among the
// payload's first `off` digits (a digit equal to d turns into 00 under x ^ (d repeated), which ~(y | y >> 1) marks in
// the low bit of its field).
__device__ __forceinline__ uint32_t record_rank(const uint32_t (&w)[16], uint32_t rec_start, uint32_t off, uint32_t d) {
  const uint32_t full = off >> 4, sh = (off & 15u) * 2u;
  const uint32_t pat = d * 0x55555555u;
  uint32_t r = 0;
#pragma unroll
  for (uint32_t i = 0; i < 13; ++i) {
    const uint32_t y = w[3 + i] ^ pat;
    const uint32_t m = ~(y | (y >> 1)) & 0x55555555u;
    const uint32_t lim = i < full ? 0xFFFFFFFFu : (i == full ? ((1u << sh) - 1u) : 0u);
    r += __popc(m & lim);
  }
  const uint32_t before = d == 0 ? w[0] : d == 1 ? w[1] : d == 2 ? w[2] : rec_start - w[0] - w[1] - w[2];
  return before + r;
}

// One step of a walk at level l: position a -> Z_l[d] + rank_d(l, a); the record index is clamped to the level, so
// a position past the end yields an unspecified value instead of a read outside the layout. With kDigit the digit
// is the one stored at a (an access walk) and is returned in *dg; otherwise d is the caller's.
template <bool kDigit>
__device__ __forceinline__ uint32_t step(const uint32_t *__restrict__ quads, uint32_t nrec, const uint32_t *__restrict__ Z,
                                         uint32_t l, uint32_t a, uint32_t d, uint32_t *dg) {
  const uint32_t rec = min(a / kDigits, nrec - 1u);
  uint32_t w[16];
  load_record(quads + (static_cast<size_t>(l) * nrec + rec) * kRecWords, w);
  const uint32_t off = min(a - rec * kDigits, kDigits);
  if constexpr (kDigit) {
    d = record_digit(w, min(off, kDigits - 1u));
    *dg = d;
  }
  return Z[4 * l + d] + record_rank(w, rec * kDigits, off, d);
}

// ---- build kernels
// Every position's symbol from the RRR wavelet matrix (the binary matrix's access walk).
template <int LEVELS>
__global__ __launch_bounds__(256) void tokens_kernel(cf_rrrw_view w, uint32_t *__restrict__ seq, uint32_t n) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i < n) seq[i] = cfr::access_one<LEVELS>(w, static_cast<int>(i));
}

// Per record r of the level whose digit is (seq >> shift) & 3: the count of each digit, into cnt[d][r]
// (cnt rows of nrec + 1 entries; entry nrec stays 0 so that an exclusive scan leaves the totals there).
static __global__ __launch_bounds__(kBuildThreads) void count_kernel(const uint32_t *__restrict__ seq, uint32_t n,
                                                              uint32_t nrec, uint32_t shift, uint32_t *__restrict__ cnt) {
  __shared__ uint32_t s_c[kBuildThreads / 64][4];
  const uint32_t r = blockIdx.x, t = threadIdx.x, wave = t >> 6, lane = t & 63u;
  const uint32_t i = r * kDigits + t;
  const bool valid = t < kDigits && i < n;
  const uint32_t d = valid ? (seq[i] >> shift) & 3u : 4u;
#pragma unroll
  for (uint32_t v = 0; v < 4; ++v) {
    const uint64_t b = __builtin_amdgcn_ballot_w64(d == v);
    if (lane == 0) s_c[wave][v] = static_cast<uint32_t>(__builtin_popcountll(b));
  }
  __syncthreads();
  if (t < 4) {
    uint32_t s = 0;
#pragma unroll
    for (uint32_t k = 0; k < kBuildThreads / 64; ++k) s += s_c[k][t];
    cnt[t * (nrec + 1) + r] = s;
    if (r == 0) cnt[t * (nrec + 1) + nrec] = 0;
  }
}

// The level's records from the exclusive prefix counts pre[d][r] (totals at pre[d][nrec]), and the stable partition
// of the sequence by the digit into `next`: position i of record r goes to Z[d] + pre[d][r] + (its rank among the
// record's d digits). Workgroup 0 writes Z.
static __global__ __launch_bounds__(kBuildThreads) void write_kernel(const uint32_t *__restrict__ seq, uint32_t *__restrict__ next,
                                                              uint32_t n, uint32_t nrec, uint32_t shift,
                                                              const uint32_t *__restrict__ pre,
                                                              uint32_t *__restrict__ level, uint32_t *__restrict__ Z) {
  __shared__ uint32_t s_c[kBuildThreads / 64][4];
  const uint32_t r = blockIdx.x, t = threadIdx.x, wave = t >> 6, lane = t & 63u;
  const uint32_t i = r * kDigits + t;
  const bool valid = t < kDigits && i < n;
  const uint32_t s = valid ? seq[i] : 0u;
  const uint32_t d = valid ? (s >> shift) & 3u : 4u;
  uint64_t mine = 0;
#pragma unroll
  for (uint32_t v = 0; v < 4; ++v) {
    const uint64_t b = __builtin_amdgcn_ballot_w64(d == v);
    if (d == v) mine = b;
    if (lane == 0) s_c[wave][v] = static_cast<uint32_t>(__builtin_popcountll(b));
  }
  __syncthreads();
  const uint32_t t0 = pre[0 * (nrec + 1) + nrec], t1 = pre[1 * (nrec + 1) + nrec], t2 = pre[2 * (nrec + 1) + nrec];
  if (valid) {
    uint32_t before = 0;  // this digit's matches in the record's earlier wavefronts
    for (uint32_t k = 0; k < wave; ++k) before += s_c[k][d];
    const uint32_t zd = d == 0 ? 0u : d == 1 ? t0 : d == 2 ? t0 + t1 : t0 + t1 + t2;
    const uint32_t in_rec = before + __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mine >> 32),
                                                              __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mine), 0u));
    next[zd + pre[d * (nrec + 1) + r] + in_rec] = s;
  }
  // payload: word j = digits 16 j .. 16 j + 15 (positions past n hold 0)
  uint32_t x = (valid ? d : 0u) << (2u * (t & 15u));
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) x |= static_cast<uint32_t>(__shfl_xor(static_cast<int>(x), o));
  uint32_t *rec = level + static_cast<size_t>(r) * kRecWords;
  if (t < kDigits && (t & 15u) == 0) rec[3 + (t >> 4)] = x;
  if (t < 3) rec[t] = pre[t * (nrec + 1) + r];
  if (r == 0 && t == 0) {
    Z[0] = 0;
    Z[1] = t0;
    Z[2] = t0 + t1;
    Z[3] = t0 + t1 + t2;
  }
}

// base[c] = (X ? X[c] : 0) - e(c) for c < nsym, one thread per symbol.
static __global__ __launch_bounds__(256) void base_kernel(const uint32_t *__restrict__ quads, uint32_t nrec,
                                                   const uint32_t *__restrict__ Z, uint32_t L4, int32_t nsym,
                                                   const int32_t *__restrict__ X, int32_t *__restrict__ base) {
  const int c = static_cast<int>(blockIdx.x * 256u + threadIdx.x);
  if (c >= nsym) return;
  uint32_t p = 0;
  for (uint32_t l = 0; l < L4; ++l)
    p = step<false>(quads, nrec, Z, l, p, (static_cast<uint32_t>(c) >> (2u * (L4 - 1u - l))) & 3u, nullptr);
  base[c] = (X ? X[c] : 0) - static_cast<int32_t>(p);
}

// ---- host side
struct Layout {
  uint32_t L4, nrec;
  uint64_t rec_words, z_words, base_words;  // offsets (u32 words) of Z and base: rec_words, rec_words + z_words
  uint64_t bytes() const { return (rec_words + z_words + base_words) * 4u; }
};
inline Layout layout(int bits, uint64_t n, int32_t nsym) {
  Layout L{};
  L.L4 = levels_for(bits);
  L.nrec = nrec_for(n);
  L.rec_words = static_cast<uint64_t>(L.L4) * L.nrec * kRecWords;
  L.z_words = 4ull * L.L4;
  L.base_words = static_cast<uint64_t>(nsym);
  return L;
}

// Workspace: two sequence buffers of n u32, counts and prefix counts [4][nrec + 1], the scan's temporary storage.
inline uint64_t scan_tmp_bytes(uint32_t nrec) {
  size_t b = 0;
  static_cast<void>(hipcub::DeviceScan::ExclusiveSum(nullptr, b, static_cast<uint32_t *>(nullptr),
                                                     static_cast<uint32_t *>(nullptr), static_cast<int>(nrec + 1)));
  return (b + 255) & ~size_t(255);
}
inline uint64_t workspace_bytes(uint64_t n, uint32_t nrec) {
  const uint64_t seq = ((n * 4 + 255) & ~uint64_t(255));
  const uint64_t cnt = ((4ull * (nrec + 1) * 4 + 255) & ~uint64_t(255));
  return 2 * seq + 2 * cnt + scan_tmp_bytes(nrec);
}

// Builds the layout of the sequence held by RRR wavelet matrix w (n symbols) into `quads` (L.bytes() bytes).
inline cf_status build(const cf_rrrw_view &w, uint64_t n, int32_t nsym, const int32_t *X, uint32_t *quads, void *ws,
                       hipStream_t s) {
  const Layout L = layout(w.bits, n, nsym);
  const uint32_t nrec = L.nrec;
  uint8_t *p = static_cast<uint8_t *>(ws);
  const uint64_t seq_b = ((n * 4 + 255) & ~uint64_t(255)), cnt_b = ((4ull * (nrec + 1) * 4 + 255) & ~uint64_t(255));
  uint32_t *seq = reinterpret_cast<uint32_t *>(p);
  uint32_t *nxt = reinterpret_cast<uint32_t *>(p + seq_b);
  uint32_t *cnt = reinterpret_cast<uint32_t *>(p + 2 * seq_b);
  uint32_t *pre = reinterpret_cast<uint32_t *>(p + 2 * seq_b + cnt_b);
  void *tmp = p + 2 * seq_b + 2 * cnt_b;
  size_t tmp_b = scan_tmp_bytes(nrec);
  const uint32_t nn = static_cast<uint32_t>(n);
  const unsigned g = cfd::grid_for(static_cast<size_t>(n), 256);
  if (n > 0) {
    switch (w.bits) {
      case 15: tokens_kernel<15><<<g, 256, 0, s>>>(w, seq, nn); break;
      case 16: tokens_kernel<16><<<g, 256, 0, s>>>(w, seq, nn); break;
      default: tokens_kernel<0><<<g, 256, 0, s>>>(w, seq, nn); break;
    }
  }
  uint32_t *Z = quads + L.rec_words;
  for (uint32_t l = 0; l < L.L4; ++l) {
    const uint32_t shift = 2u * (L.L4 - 1u - l);
    count_kernel<<<nrec, kBuildThreads, 0, s>>>(seq, nn, nrec, shift, cnt);
    for (uint32_t d = 0; d < 4; ++d)
      if (hipcub::DeviceScan::ExclusiveSum(tmp, tmp_b, cnt + d * (nrec + 1), pre + d * (nrec + 1),
                                           static_cast<int>(nrec + 1), s) != hipSuccess)
        return CF_ERR_CUDA;
    write_kernel<<<nrec, kBuildThreads, 0, s>>>(seq, nxt, nn, nrec, shift, pre,
                                                quads + static_cast<size_t>(l) * nrec * kRecWords, Z + 4 * l);
    uint32_t *t = seq;
    seq = nxt;
    nxt = t;
  }
  base_kernel<<<cfd::grid_for(static_cast<size_t>(nsym), 256), 256, 0, s>>>(
      quads, nrec, Z, L.L4, nsym, X, reinterpret_cast<int32_t *>(Z + L.z_words));
  return cfd::launch_status();
}

}  // namespace cfq
