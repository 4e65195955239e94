// lines_core.hpp — the line layout of a wavelet matrix's levels, derived on the device from the RRR levels, and
// the rank primitives over it (shared by the wavelet access/rank kernels and the FM-index kernels).
//
// Level l's bitvector is stored as records of 16 u32 = 64 bytes (half a 128-byte L2 line):
//   word 0      ones of the level in bits [0, 480 r)
//   words 1..15 bits [480 r, 480 r + 480) of the level, LSB-first (32 RRR blocks of 15 bits)
// A rank1 (and the bit at a position) reads one record: four 16-byte loads from one line, then up to 15 masked
// popcounts. On the RRR level the same rank1 reads three or four separate lines (the superblock's samples, its
// class words, the offset bits) and an unrank table entry.
//
// After the levels comes a per-symbol table base[c] = X[c] - e(c), where e(c) is the position at which the rank
// walk of symbol c started at 0 ends on the last level (X = the FM-index's C table, or 0 for a plain wavelet).
// A rank walk maps its start-of-c chain p and its position chain a by the same rule (a' = zeros + rank1(a) on a
// 1 bit, a - rank1(a) on a 0 bit) and p never depends on the position, so
//   rank(c, i) = a_L(i) - e(c)          and the FM-index's LF(i) = C[c] + rank(c, i) = a_L(i) + base[c].
// A rank or an LF step then walks one chain, one record per level.
#pragma once

#include "chromofold/chromofold_search.h"
#include "cf_device.hpp"
#include "rrr_core.hpp"

namespace cfl {

constexpr uint32_t kLineBits = 480;  // payload bits of a record
constexpr uint32_t kRecWords = 16;

// Records per level when positions up to and including `n` must resolve: n / 480 + 1.
__host__ __device__ inline uint32_t nrec_for(uint64_t n) { return static_cast<uint32_t>(n / kLineBits) + 1u; }

// One record into registers (four 16-byte loads; the layout is 16-byte aligned).
__device__ __forceinline__ void load_record(const uint32_t *__restrict__ rec, uint32_t (&w)[16]) {
  const uint4 *q = reinterpret_cast<const uint4 *>(rec);
  const uint4 a = q[0], b = q[1], c = q[2], d = q[3];
  w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
  w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
  w[8] = c.x; w[9] = c.y; w[10] = c.z; w[11] = c.w;
  w[12] = d.x; w[13] = d.y; w[14] = d.z; w[15] = d.w;
}

// Ones of the level before bit `off` of the record (word 0 + the payload's bits [0, off)); with kBit also the bit
// at `off`. An `off` past the payload counts all of it (and reads bit 0).
template <bool kBit>
__device__ __forceinline__ int record_rank(const uint32_t (&w)[16], uint32_t off, int *bit) {
  const uint32_t full = off >> 5, sh = off & 31u;
  int r = static_cast<int>(w[0]);
  uint32_t tw = 0;
#pragma unroll
  for (uint32_t i = 0; i < 15; ++i) {
    const uint32_t x = w[1 + i];
    if (kBit && i == full) tw = x;
    r += __popc(i < full ? x : (i == full ? x & ((1u << sh) - 1u) : 0u));
  }
  if constexpr (kBit) *bit = static_cast<int>((tw >> sh) & 1u);
  return r;
}

// rank1 of level `lvl` at position `a` (and the bit there with kBit). The record index is clamped to the level,
// so a position past the end yields an unspecified count instead of a read outside the layout.
template <bool kBit>
__device__ __forceinline__ int rank1(const uint32_t *__restrict__ lines, uint32_t nrec, int lvl, uint32_t a,
                                     int *bit) {
  const uint32_t rec = min(a / kLineBits, nrec - 1u);
  uint32_t w[16];
  load_record(lines + (static_cast<size_t>(lvl) * nrec + rec) * kRecWords, w);
  return record_rank<kBit>(w, a - rec * kLineBits, bit);
}

// Records of the layout from the RRR levels: one wavefront per pair of records (2 sb, 2 sb + 1) of a level = RRR
// superblock sb (64 blocks x 15 bits = 960 bits). Lane i decodes block 64 sb + i (class nibble; offset at the
// superblock's offset sample + the wave's exclusive prefix sum of the widths; table unrank) and ORs its 15 bits
// into the payload in LDS. Word 0 of record 2 sb is the superblock's rank sample; of record 2 sb + 1 that plus the
// ones of blocks 0..31. Blocks at or past `nblocks` are zero. Pairs past the last superblock hold the level's total
// ones: n - zeros[l] when n >= 0, else the rank sample of superblock nsb (the format keeps nsb + 1 samples).
constexpr unsigned kBuildThreads = 256;
static __global__ __launch_bounds__(kBuildThreads) void build_records_kernel(cf_rrrw_view w,
                                                                             uint32_t *__restrict__ lines,
                                                                             uint32_t nrec, uint32_t npairs,
                                                                             uint32_t nblocks, int64_t n) {
  __shared__ uint32_t s_pay[kBuildThreads / 64][2][16];
  const uint32_t wv = threadIdx.x >> 6, lane = threadIdx.x & 63u;
  const uint32_t gw = blockIdx.x * (kBuildThreads / 64) + wv;
  const uint32_t lvl = gw / npairs, sb = gw - lvl * npairs;
  const bool live = lvl < static_cast<uint32_t>(w.bits);
  if (lane < 32u) s_pay[wv][lane >> 4][lane & 15u] = 0u;
  __syncthreads();
  const uint32_t blk = sb * 64u + lane;
  const bool in_sb = live && sb < static_cast<uint32_t>(w.nsb);
  const bool inside = in_sb && blk < nblocks;
  uint32_t k = 0;
  if (inside) k = (w.classes[static_cast<size_t>(lvl) * w.cwords + (blk >> 3)] >> (4u * (blk & 7u))) & 15u;
  const int wd = cfd::width_of(static_cast<int>(k));
  int pre = wd;  // inclusive prefix sum of the widths over the wave
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(pre, d);
    if (lane >= static_cast<uint32_t>(d)) pre += o;
  }
  int ones = static_cast<int>(k);  // ones of blocks 0..31 of the superblock
#pragma unroll
  for (int d = 1; d < 32; d <<= 1) ones += __shfl_xor(ones, d);
  ones = __shfl(ones, 0);
  uint32_t rank0 = 0;
  if (live) {
    const uint32_t sbs = in_sb ? sb : static_cast<uint32_t>(w.nsb);
    const size_t srow = static_cast<size_t>(lvl) * (w.nsb + 1) + sbs;
    const size_t arow = static_cast<size_t>(lvl) * w.na + (sbs >> 5);
    if (in_sb || n < 0) rank0 = static_cast<uint32_t>(w.rank_a[arow] + w.rank_d[srow]);
    else rank0 = static_cast<uint32_t>(n - w.zeros[lvl]);
    if (inside) {
      const uint32_t off = wd > 0 ? cfr::read_bits(w.offsets, static_cast<int64_t>(w.offbase[lvl]) + w.off_a[arow] +
                                                                  w.off_d[srow] + (pre - wd), wd)
                                  : 0u;
      k = cfr::kTab.unrank[cfr::kTab.base[k] + off];  // the block's 15 bits
    }
  }
  if (inside) {
    const uint32_t bit = 15u * (lane & 31u);
    uint32_t *pay = s_pay[wv][lane >> 5] + 1;
    atomicOr(pay + (bit >> 5), k << (bit & 31u));
    if ((bit & 31u) > 17u) atomicOr(pay + (bit >> 5) + 1, k >> (32u - (bit & 31u)));
  }
  __syncthreads();
  const uint32_t r = lane >> 4, j = lane & 15u, rec = 2u * sb + r;
  if (live && lane < 32u && rec < nrec) {
    const uint32_t word = j == 0 ? rank0 + (r ? static_cast<uint32_t>(ones) : 0u) : s_pay[wv][r][j];
    lines[(static_cast<size_t>(lvl) * nrec + rec) * kRecWords + j] = word;
  }
}

// base[c] = (X ? X[c] : 0) - e(c) for c < nsym, one thread per symbol (the start-of-c chain on the RRR levels).
template <int LEVELS>
__global__ __launch_bounds__(256) void walk_base_kernel(cf_rrrw_view w, int32_t nsym, const int32_t *__restrict__ X,
                                                        int32_t *__restrict__ base) {
  const int c = blockIdx.x * 256 + static_cast<int>(threadIdx.x);
  if (c >= nsym) return;
  const int L = LEVELS > 0 ? LEVELS : w.bits;
  int p = 0;
  for (int lvl = 0; lvl < L; ++lvl) {
    const int rp = cfr::rank1_lvl<false>(w, lvl, p, nullptr);
    p = (c >> (L - 1 - lvl)) & 1 ? w.zeros[lvl] + rp : p - rp;
  }
  base[c] = (X ? X[c] : 0) - p;
}

// Launches the two build kernels; `base` follows the records.
inline cf_status build(const cf_rrrw_view &w, uint32_t *lines, uint32_t nrec, uint32_t nblocks, int64_t n,
                       int32_t nsym, const int32_t *X, hipStream_t s) {
  const uint32_t npairs = (nrec + 1) / 2;
  const uint64_t waves = static_cast<uint64_t>(w.bits) * npairs;
  const uint64_t blocks = (waves + kBuildThreads / 64 - 1) / (kBuildThreads / 64);
  if (blocks == 0 || blocks > 0x7fffffffu) return CF_ERR_INVALID_ARGUMENT;
  build_records_kernel<<<static_cast<unsigned>(blocks), kBuildThreads, 0, s>>>(w, lines, nrec, npairs, nblocks, n);
  int32_t *base = reinterpret_cast<int32_t *>(lines + static_cast<size_t>(w.bits) * nrec * kRecWords);
  const unsigned g = cfd::grid_for(static_cast<size_t>(nsym), 256);
  switch (w.bits) {
    case 15: walk_base_kernel<15><<<g, 256, 0, s>>>(w, nsym, X, base); break;
    case 16: walk_base_kernel<16><<<g, 256, 0, s>>>(w, nsym, X, base); break;
    default: walk_base_kernel<0><<<g, 256, 0, s>>>(w, nsym, X, base); break;
  }
  return cfd::launch_status();
}

}  // namespace cfl
