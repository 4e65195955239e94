// rrr_core.hpp — per-lane RRR wavelet-matrix primitives (rank1 of one level, access, rank), shared by the
// wavelet kernels and the FM-index kernels.
//
// Semantics follow reference include/chromofold/detail/rrr_wavelet_device.cuh:40-149 exactly (same samples, same
// class stream, same LSB-first offset stream, same enumerative code); the arithmetic is reorganised for gfx950
// (SWAR class-word scan, table unrank) as described in rrr_wavelet.hip.
#pragma once

#include "chromofold/chromofold_search.h"
#include "cf_device.hpp"

namespace cfr {

// One copy per code object; 64 KiB unrank table + widths + class bases, all fixed by the RRR format.
static __device__ const cfd::RrrTables kTab = cfd::make_rrr_tables();

// LSB-first read of `w` bits at bit position `at` (may straddle two words; the offset stream carries two words of
// padding per level so the second read is always in bounds). reference rrr_wavelet_device.cuh:30-38.
__device__ __forceinline__ uint32_t read_bits(const uint32_t *__restrict__ s, int64_t at, int w) {
  const int64_t wi = at >> 5;
  const int b = static_cast<int>(at & 31);
  const uint32_t lo = s[wi];
  const uint32_t hi = (b + w > 32) ? s[wi + 1] : 0u;
  const uint64_t both = (static_cast<uint64_t>(hi) << 32) | lo;
  return static_cast<uint32_t>(both >> b) & ((1u << w) - 1u);
}

// Where rank1 reads the per-superblock samples and the unrank table: straight from the view (global memory, L2)
// or from copies staged in LDS by a persistent kernel (LdsTables, see rrr_wavelet.hip).
struct GlobalTables {
  const cf_rrrw_view &v;
  __device__ int rank(size_t arow_a, size_t srow_sb) const { return v.rank_a[arow_a] + v.rank_d[srow_sb]; }
  __device__ int off(size_t arow_a, size_t srow_sb) const { return v.off_a[arow_a] + v.off_d[srow_sb]; }
  __device__ int base(int k) const { return kTab.base[k]; }
  __device__ uint32_t unrank(int i) const { return kTab.unrank[i]; }
};
// Tables staged in LDS by a persistent kernel: the anchors, the unrank table and its class starts always; the
// per-superblock deltas too when kDeltas (small indexes), else those stay in global memory.
template <bool kDeltas>
struct StagedTables {
  const int32_t *rank_a, *off_a;   // LDS [bits * na]
  const uint16_t *rank_d, *off_d;  // LDS or global [bits * (nsb + 1)]
  const uint16_t *unrank_tab;      // LDS, the 64 KiB unrank table
  const int32_t *base_tab;         // LDS, the unrank table's class starts (17 entries)
  __device__ int rank(size_t arow_a, size_t srow_sb) const { return rank_a[arow_a] + rank_d[srow_sb]; }
  __device__ int off(size_t arow_a, size_t srow_sb) const { return off_a[arow_a] + off_d[srow_sb]; }
  __device__ int base(int k) const { return base_tab[k]; }
  __device__ uint32_t unrank(int i) const { return unrank_tab[i]; }
};

// LDS layout of the staged tables (16-byte aligned parts); `bytes` = the workgroup's dynamic LDS.
struct StageLayout {
  size_t unrank, base, rank_a, off_a, rank_d, off_d, bytes;
};

__host__ __device__ inline size_t align16(size_t x) { return (x + 15) & ~static_cast<size_t>(15); }

__host__ __device__ inline StageLayout stage_layout(const cf_rrrw_view &v, bool deltas) {
  StageLayout l{};
  const size_t nd = static_cast<size_t>(v.bits) * (v.nsb + 1), na = static_cast<size_t>(v.bits) * v.na;
  l.unrank = 0;
  l.base = align16(sizeof(cfd::RrrTables::unrank));
  l.rank_a = l.base + align16(sizeof(cfd::RrrTables::base));
  l.off_a = l.rank_a + align16(na * 4);
  l.rank_d = l.off_a + align16(na * 4);
  l.off_d = l.rank_d + (deltas ? align16(nd * 2) : 0);
  l.bytes = l.off_d + (deltas ? align16(nd * 2) : 0);
  return l;
}

// Cooperative copy by all `nthreads` threads of the workgroup, ending with a barrier.
template <bool kDeltas>
__device__ StagedTables<kDeltas> stage_tables(const cf_rrrw_view &v, uint8_t *smem, unsigned nthreads) {
  const StageLayout l = stage_layout(v, kDeltas);
  const unsigned t = threadIdx.x;
  {
    const uint4 *src = reinterpret_cast<const uint4 *>(kTab.unrank);
    uint4 *dst = reinterpret_cast<uint4 *>(smem + l.unrank);
    for (size_t i = t; i < sizeof(cfd::RrrTables::unrank) / 16; i += nthreads) dst[i] = src[i];
  }
  int32_t *bs = reinterpret_cast<int32_t *>(smem + l.base);
  if (t < 17) bs[t] = kTab.base[t];
  const size_t na = static_cast<size_t>(v.bits) * v.na;
  int32_t *ra = reinterpret_cast<int32_t *>(smem + l.rank_a), *oa = reinterpret_cast<int32_t *>(smem + l.off_a);
  for (size_t i = t; i < na; i += nthreads) {
    ra[i] = v.rank_a[i];
    oa[i] = v.off_a[i];
  }
  StagedTables<kDeltas> tb{ra, oa, v.rank_d, v.off_d, reinterpret_cast<const uint16_t *>(smem + l.unrank), bs};
  if constexpr (kDeltas) {
    const size_t nd = static_cast<size_t>(v.bits) * (v.nsb + 1);
    uint16_t *rd = reinterpret_cast<uint16_t *>(smem + l.rank_d), *od = reinterpret_cast<uint16_t *>(smem + l.off_d);
    for (size_t i = t; i < nd; i += nthreads) {
      rd[i] = v.rank_d[i];
      od[i] = v.off_d[i];
    }
    tb.rank_d = rd;
    tb.off_d = od;
  }
  __syncthreads();
  return tb;
}

// Launch of a persistent staged kernel with `bytes` of dynamic LDS (above the default 64 KiB limit).
template <class K, class... Args>
inline cf_status launch_staged(unsigned threads, K kernel, unsigned grid, size_t bytes, hipStream_t s,
                               const Args &...args) {
  if (hipFuncSetAttribute(reinterpret_cast<const void *>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          static_cast<int>(bytes)) != hipSuccess)
    return CF_ERR_CUDA;
  kernel<<<grid, threads, bytes, s>>>(args...);
  return cfd::launch_status();
}

// Which staged variant a persistent launch of `threads`-thread workgroups over `count` items can use: 2 = every
// table in LDS, 1 = all but the per-superblock deltas, 0 = none (the index is too large, or the batch too small to
// give each lane of one workgroup per CU an item). `cus` receives the CU count.
inline int staged_mode(const cf_rrrw_view &v, size_t count, unsigned threads, unsigned &cus) {
  static int n_cu = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return 0;
    return n;
  }();
  constexpr size_t kLimit = 160 * 1024;
  cus = n_cu > 0 ? static_cast<unsigned>(n_cu) : 0u;
  if (cus == 0 || v.bits <= 0 || v.nsb < 0 || v.na < 0 || count < static_cast<size_t>(cus) * threads) return 0;
  if (stage_layout(v, true).bytes <= kLimit) return 2;
  if (stage_layout(v, false).bytes <= kLimit) return 1;
  return 0;
}

// The 8 class words of superblock sbi: two 16-byte loads (4-byte aligned) when all 8 lie inside the level's
// `cwords`, otherwise word by word (only the level's last superblock can be short).
__device__ __forceinline__ void class_words(const uint32_t *__restrict__ cls, int sbi, int cwords, int full,
                                            uint32_t (&x)[8]) {
  const uint32_t *__restrict__ cw = cls + (static_cast<size_t>(sbi) << 3);
  if ((sbi << 3) + 8 <= cwords) {
    uint4 a, b;
    __builtin_memcpy(&a, cw, 16);
    __builtin_memcpy(&b, cw + 4, 16);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
  } else {
#pragma unroll
    for (int w = 0; w < 8; ++w) x[w] = w <= full ? cw[w] : 0u;
  }
}

// rank1 of level `lvl` over [0, pos); with kBit also the plane bit at pos (the access primitive, one block decode
// serving both). reference rrr_wavelet_device.cuh:56-113.
template <bool kBit, class Tables, bool kVecClasses = false>
__device__ __forceinline__ int rank1_lvl_t(const cf_rrrw_view &v, const Tables &tb, int lvl, int pos, int *bit) {
  const uint32_t *__restrict__ cls = v.classes + static_cast<size_t>(lvl) * v.cwords;
  const size_t srow = static_cast<size_t>(lvl) * (v.nsb + 1);
  const size_t arow = static_cast<size_t>(lvl) * v.na;
  const int blk = pos / cfd::kRrrT;
  const int b = pos - blk * cfd::kRrrT;
  const int sbi = blk >> 6;  // / kRrrS
  const int a = sbi >> 5;    // / kRrrK
  int r = tb.rank(arow + a, srow + sbi);
  const int obit = tb.off(arow + a, srow + sbi);

  // class words of superblock sbi: blocks [sbi*64 + 8w, +8) live in word sbi*8 + w
  const int nblk = blk - (sbi << 6);  // blocks to sum before the target block, 0..63
  const int full = nblk >> 3, rem = nblk & 7;
  uint32_t xs[8];
  if constexpr (kVecClasses) {
    class_words(cls, sbi, v.cwords, full, xs);
  } else {
    const uint32_t *__restrict__ cw = cls + (static_cast<size_t>(sbi) << 3);
#pragma unroll
    for (int w = 0; w < 8; ++w) xs[w] = w <= full ? cw[w] : 0u;
  }
  int csum = 0, wsum = 0;
  uint32_t target_word = 0;
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    if (w <= full) {
      uint32_t x = xs[w];
      if (w == full) {
        target_word = x;
        x &= rem ? ((1u << (4 * rem)) - 1u) : 0u;
      }
      csum += cfd::nibble_sum(x);
      wsum += cfd::nibble_width_sum(x);
    }
  }
  r += csum;
  if (kBit || b > 0) {
    const int k = static_cast<int>((target_word >> (4 * rem)) & 15u);
    const int w = cfd::width_of(k);
    const uint32_t off = w ? read_bits(v.offsets, static_cast<int64_t>(v.offbase[lvl]) + obit + wsum, w) : 0u;
    const uint32_t word = tb.unrank(tb.base(k) + static_cast<int>(off));
    r += __popc(word & ((1u << b) - 1u));
    if (kBit) *bit = static_cast<int>((word >> b) & 1u);
  }
  return r;
}

template <bool kBit>
__device__ __forceinline__ int rank1_lvl(const cf_rrrw_view &v, int lvl, int pos, int *bit) {
  return rank1_lvl_t<kBit>(v, GlobalTables{v}, lvl, pos, bit);
}

// token at position i: one block decode per level (reference rrr_wavelet_device.cuh:117-134)
template <int LEVELS, class Tables, bool kVec>
__device__ __forceinline__ uint32_t access_one_t(const cf_rrrw_view &v, const Tables &tb, int i) {
  const int L = LEVELS > 0 ? LEVELS : v.bits;
  uint32_t val = 0;
  for (int lvl = 0; lvl < L; ++lvl) {
    int bit = 0;
    const int r = rank1_lvl_t<true, Tables, kVec>(v, tb, lvl, i, &bit);
    val = (val << 1) | static_cast<uint32_t>(bit);
    i = bit ? v.zeros[lvl] + r : i - r;
  }
  return val;
}

// occurrences of c in [0, i): two rank1 per level narrowing [p, q) (reference rrr_wavelet_device.cuh:137-149).
// Once the interval is empty every later level keeps it empty, so the walk stops early with the same answer.
template <int LEVELS, class Tables, bool kVec>
__device__ __forceinline__ uint32_t rank_one_t(const cf_rrrw_view &v, const Tables &tb, int c, int i) {
  const int L = LEVELS > 0 ? LEVELS : v.bits;
  int p = 0, q = i;
  for (int lvl = 0; lvl < L; ++lvl) {
    if (p >= q) break;
    const int rp = rank1_lvl_t<false, Tables, kVec>(v, tb, lvl, p, nullptr);
    const int rq = rank1_lvl_t<false, Tables, kVec>(v, tb, lvl, q, nullptr);
    if ((c >> (L - 1 - lvl)) & 1) {
      p = v.zeros[lvl] + rp;
      q = v.zeros[lvl] + rq;
    } else {
      p -= rp;
      q -= rq;
    }
  }
  return static_cast<uint32_t>(q - p);
}

template <int LEVELS>
__device__ __forceinline__ uint32_t access_one(const cf_rrrw_view &v, int i) {
  return access_one_t<LEVELS, GlobalTables, false>(v, GlobalTables{v}, i);
}

template <int LEVELS>
__device__ __forceinline__ uint32_t rank_one(const cf_rrrw_view &v, int c, int i) {
  return rank_one_t<LEVELS, GlobalTables, false>(v, GlobalTables{v}, c, i);
}

// rank(c, lo) and rank(c, hi) together: both walks share the start-of-c chain p (its rank1 is computed once),
// so a backward-search step costs 3 rank1 per level instead of 4. Identical results to two rank_one calls.
template <int LEVELS, class Tables = GlobalTables, bool kVec = false>
__device__ __forceinline__ void rank_pair(const cf_rrrw_view &v, int c, int lo, int hi, int &rlo, int &rhi,
                                          const Tables &tb) {
  const int L = LEVELS > 0 ? LEVELS : v.bits;
  int p = 0, a = lo, b = hi;
  for (int lvl = 0; lvl < L; ++lvl) {
    const int rp = rank1_lvl_t<false, Tables, kVec>(v, tb, lvl, p, nullptr);
    const int ra = rank1_lvl_t<false, Tables, kVec>(v, tb, lvl, a, nullptr);
    const int rb = rank1_lvl_t<false, Tables, kVec>(v, tb, lvl, b, nullptr);
    if ((c >> (L - 1 - lvl)) & 1) {
      p = v.zeros[lvl] + rp;
      a = v.zeros[lvl] + ra;
      b = v.zeros[lvl] + rb;
    } else {
      p -= rp;
      a -= ra;
      b -= rb;
    }
  }
  rlo = a - p;
  rhi = b - p;
}

// One LF-mapping step: c = BWT[i] and rank(c, i) in a single walk. The access walk of i follows exactly the bits
// of c, so it IS the rank walk of position i for symbol c; only the start-of-c chain p needs its own rank1.
// Returns rank(c, i) (so LF(i) = C[c] + rank) and writes c. Two rank1 per level instead of three.
template <int LEVELS, class Tables = GlobalTables, bool kVec = false>
__device__ __forceinline__ int access_rank(const cf_rrrw_view &v, int i, int &c_out, const Tables &tb) {
  const int L = LEVELS > 0 ? LEVELS : v.bits;
  int p = 0, c = 0;
  for (int lvl = 0; lvl < L; ++lvl) {
    int bit = 0;
    const int ri = rank1_lvl_t<true, Tables, kVec>(v, tb, lvl, i, &bit);
    const int rp = rank1_lvl_t<false, Tables, kVec>(v, tb, lvl, p, nullptr);
    c = (c << 1) | bit;
    if (bit) {
      i = v.zeros[lvl] + ri;
      p = v.zeros[lvl] + rp;
    } else {
      i -= ri;
      p -= rp;
    }
  }
  c_out = c;
  return i - p;
}

}  // namespace cfr

namespace cfr {

// rank1 over [0, pos) of a single RRR bitvector with one-level samples: sbrank[sbi] set bits and sboff[sbi] offset
// bit position at the start of superblock sbi (64 blocks). Semantics of reference src/cuda/rrr.cu:38-57; the class
// scan and the unrank use the same SWAR word scan and table as the wavelet levels.
__device__ __forceinline__ int rank1_plain(const uint32_t *__restrict__ cls, const uint32_t *__restrict__ offsets,
                                           const int32_t *__restrict__ sbrank, const int32_t *__restrict__ sboff,
                                           int pos) {
  const int blk = pos / cfd::kRrrT;
  const int b = pos - blk * cfd::kRrrT;
  const int sbi = blk >> 6;
  int r = sbrank[sbi];
  const int obit = sboff[sbi];
  const uint32_t *__restrict__ cw = cls + (static_cast<size_t>(sbi) << 3);
  const int nblk = blk - (sbi << 6);
  const int full = nblk >> 3, rem = nblk & 7;
  int csum = 0, wsum = 0;
  uint32_t target_word = 0;
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    if (w <= full && (w < full || rem || b)) {  // the target block's word is read only when it is needed
      uint32_t x = cw[w];
      if (w == full) {
        target_word = x;
        x &= rem ? ((1u << (4 * rem)) - 1u) : 0u;
      }
      csum += cfd::nibble_sum(x);
      wsum += cfd::nibble_width_sum(x);
    }
  }
  r += csum;
  if (b > 0) {
    const int k = static_cast<int>((target_word >> (4 * rem)) & 15u);
    const int w = cfd::width_of(k);
    const uint32_t off = w ? read_bits(offsets, static_cast<int64_t>(obit) + wsum, w) : 0u;
    const uint32_t word = kTab.unrank[kTab.base[k] + off];
    r += __popc(word & ((1u << b) - 1u));
  }
  return r;
}

}  // namespace cfr
