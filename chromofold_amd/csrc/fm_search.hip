// fm_search.hip — FM-index backward search (count / SA ranges) and locate over the RRR-compressed BWT, gfx950.
//
// Replaces reference src/cuda/fm_search.cu:10-89 and include/chromofold/detail/fm_search_device.cuh:31-62 behind
// the unchanged cf_fm_* C ABI. One lane per pattern (count/ranges) or per occurrence (locate), like the
// reference, with two algebraic savings that keep the results bit-identical:
//   * backward search computes rank(c, lo) and rank(c, hi) in one walk sharing the start-of-c chain
//     (3 rank1 per wavelet level instead of 4);
//   * the LF step of locate takes c = BWT[p] and rank(c, p) from one walk (2 rank1 per level instead of 3).
// Out-of-alphabet pattern symbols empty the range; locate returns (SA[sample] + steps) mod n in 64-bit.
#include "chromofold/chromofold_index.h"
#include "chromofold/chromofold_search.h"
#include "cf_device.hpp"
#include "packed_core.hpp"
#include "rrr_core.hpp"

namespace {

constexpr unsigned kThreads = 256;

// reference fm_search_device.cuh:31-48
template <int LEVELS, class Tables = cfr::GlobalTables, bool kVec = false>
__device__ __forceinline__ void backward(const cf_fm_view &v, const int32_t *__restrict__ pat, int st, int len,
                                         int &lo, int &hi, const Tables &tb) {
  lo = 0;
  hi = v.n;
  for (int k = len - 1; k >= 0; --k) {
    const int c = pat[st + k];
    if (c < 0 || c >= v.sigma) {
      lo = hi = 0;
      continue;
    }
    if (lo < hi) {
      int rl, rh;
      cfr::rank_pair<LEVELS, Tables, kVec>(v.w, c, lo, hi, rl, rh, tb);
      lo = v.C[c] + rl;
      hi = v.C[c] + rh;
    }
  }
}

template <int LEVELS>
__global__ __launch_bounds__(kThreads) void fm_count_kernel(cf_fm_view v, const int32_t *__restrict__ pat,
                                                            const int32_t *__restrict__ pstart,
                                                            const int32_t *__restrict__ plen,
                                                            uint32_t *__restrict__ out, size_t npat) {
  const size_t t = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
  if (t >= npat) return;
  int lo, hi;
  backward<LEVELS>(v, pat, pstart[t], plen[t], lo, hi, cfr::GlobalTables{v.w});
  out[t] = static_cast<uint32_t>(hi - lo);
}

template <int LEVELS>
__global__ __launch_bounds__(kThreads) void fm_ranges_kernel(cf_fm_view v, const int32_t *__restrict__ pat,
                                                             const int32_t *__restrict__ pstart,
                                                             const int32_t *__restrict__ plen,
                                                             int32_t *__restrict__ lo_out,
                                                             int32_t *__restrict__ hi_out, size_t npat) {
  const size_t t = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
  if (t >= npat) return;
  int lo, hi;
  backward<LEVELS>(v, pat, pstart[t], plen[t], lo, hi, cfr::GlobalTables{v.w});
  lo_out[t] = lo;
  hi_out[t] = hi;
}

// reference fm_search_device.cuh:52-62
template <int LEVELS, class Tables = cfr::GlobalTables, bool kVec = false>
__device__ __forceinline__ int32_t locate_one(const cf_fm_view &v, int p, const Tables &tb) {
  int steps = 0;
  while (!((v.mwords[p >> 5] >> (p & 31)) & 1u)) {
    int c;
    const int r = cfr::access_rank<LEVELS, Tables, kVec>(v.w, p, c, tb);
    p = v.C[c] + r;
    ++steps;
  }
  const int idx = cfp::rank1(v.mwords, v.msb, p);
  return static_cast<int32_t>((static_cast<int64_t>(v.sval[idx]) + steps) % v.n);
}

template <int LEVELS>
__global__ __launch_bounds__(kThreads) void fm_locate_kernel(cf_fm_view v, const int32_t *__restrict__ rows,
                                                             int32_t *__restrict__ out, size_t nocc) {
  const size_t t = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
  if (t >= nocc) return;
  out[t] = locate_one<LEVELS>(v, rows[t], cfr::GlobalTables{v.w});
}

// ---- persistent variants: one 1024-thread workgroup per CU stages the wavelet's anchors, the unrank table and
// its class starts (and, for small indexes, the per-superblock deltas) in LDS, then works through its items.
constexpr unsigned kStagedThreads = 1024;

// Work distribution of the staged kernels: workgroup b owns items [b * per, (b + 1) * per) and its lanes take the
// next item from an LDS counter as soon as they finish one (pattern lengths and LF-walk lengths vary widely, so a
// static assignment would leave most lanes of a wave waiting for its longest item). Each item is computed exactly
// as by the kernels above.
struct ItemQueue {
  size_t begin, end;
  uint32_t *next;  // LDS
  __device__ size_t take() const { return begin + atomicAdd(next, 1u); }
};

__device__ ItemQueue item_queue(size_t count, uint32_t *s_next) {
  const size_t per = (count + gridDim.x - 1) / gridDim.x;
  ItemQueue q{min(count, blockIdx.x * per), min(count, (blockIdx.x + 1) * per), s_next};
  if (threadIdx.x == 0) *s_next = 0;
  __syncthreads();
  return q;
}

// Backward search of the queue's patterns: each loop iteration consumes one symbol of the lane's current pattern,
// or stores its result and takes the next pattern once all its symbols are consumed.
template <int LEVELS, bool kDeltas>
__device__ __forceinline__ void count_or_ranges(const cf_fm_view &v, const int32_t *__restrict__ pat,
                                                const int32_t *__restrict__ pstart, const int32_t *__restrict__ plen,
                                                size_t npat, const cfr::StagedTables<kDeltas> &tb, uint32_t *s_next,
                                                uint32_t *__restrict__ cnt_out, int32_t *__restrict__ lo_out,
                                                int32_t *__restrict__ hi_out) {
  const ItemQueue q = item_queue(npat, s_next);
  size_t t = q.take();
  bool active = t < q.end;
  int st = 0, k = 0, lo = 0, hi = 0;
  if (active) {
    st = pstart[t];
    k = plen[t];
    hi = v.n;
  }
  while (__any(active)) {
    if (active) {
      if (k > 0) {  // reference fm_search_device.cuh:31-48, one symbol (right to left)
        --k;
        const int c = pat[st + k];
        if (c < 0 || c >= v.sigma) {
          lo = hi = 0;
        } else if (lo < hi) {
          int rl, rh;
          cfr::rank_pair<LEVELS, cfr::StagedTables<kDeltas>, true>(v.w, c, lo, hi, rl, rh, tb);
          lo = v.C[c] + rl;
          hi = v.C[c] + rh;
        }
      } else {
        if (cnt_out) cnt_out[t] = static_cast<uint32_t>(hi - lo);
        if (lo_out) {
          lo_out[t] = lo;
          hi_out[t] = hi;
        }
        t = q.take();
        active = t < q.end;
        if (active) {
          st = pstart[t];
          k = plen[t];
          lo = 0;
          hi = v.n;
        }
      }
    }
  }
}

template <int LEVELS, bool kDeltas>
__global__ __launch_bounds__(kStagedThreads) void fm_count_staged_kernel(cf_fm_view v, const int32_t *__restrict__ pat,
                                                                         const int32_t *__restrict__ pstart,
                                                                         const int32_t *__restrict__ plen,
                                                                         uint32_t *__restrict__ out, size_t npat) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ uint32_t s_next;
  const auto tb = cfr::stage_tables<kDeltas>(v.w, smem, kStagedThreads);
  count_or_ranges<LEVELS, kDeltas>(v, pat, pstart, plen, npat, tb, &s_next, out, nullptr, nullptr);
}

template <int LEVELS, bool kDeltas>
__global__ __launch_bounds__(kStagedThreads) void fm_ranges_staged_kernel(
    cf_fm_view v, const int32_t *__restrict__ pat, const int32_t *__restrict__ pstart,
    const int32_t *__restrict__ plen, int32_t *__restrict__ lo_out, int32_t *__restrict__ hi_out, size_t npat) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ uint32_t s_next;
  const auto tb = cfr::stage_tables<kDeltas>(v.w, smem, kStagedThreads);
  count_or_ranges<LEVELS, kDeltas>(v, pat, pstart, plen, npat, tb, &s_next, nullptr, lo_out, hi_out);
}

template <int LEVELS, bool kDeltas>
__global__ __launch_bounds__(kStagedThreads) void fm_locate_staged_kernel(cf_fm_view v,
                                                                          const int32_t *__restrict__ rows,
                                                                          int32_t *__restrict__ out, size_t nocc) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ uint32_t s_next;
  const auto tb = cfr::stage_tables<kDeltas>(v.w, smem, kStagedThreads);
  const ItemQueue q = item_queue(nocc, &s_next);
  size_t t = q.take();
  bool active = t < q.end;
  int p = active ? rows[t] : 0, steps = 0;
  while (__any(active)) {
    if (active) {  // reference fm_search_device.cuh:52-62, one LF step per iteration
      if ((v.mwords[p >> 5] >> (p & 31)) & 1u) {
        const int idx = cfp::rank1(v.mwords, v.msb, p);
        out[t] = static_cast<int32_t>((static_cast<int64_t>(v.sval[idx]) + steps) % v.n);
        t = q.take();
        active = t < q.end;
        if (active) {
          p = rows[t];
          steps = 0;
        }
      } else {
        int c;
        const int r = cfr::access_rank<LEVELS, cfr::StagedTables<kDeltas>, true>(v.w, p, c, tb);
        p = v.C[c] + r;
        ++steps;
      }
    }
  }
}

// Launches the staged variant when one applies (levels 15 and 16 get fixed-depth instances); false otherwise.
#define CF_FM_STAGED(KERNEL, COUNT, ...)                                                                         \
  do {                                                                                                        \
    unsigned g = 0;                                                                                           \
    const int mode = cfr::staged_mode(v.w, (COUNT), kStagedThreads, g);                                      \
    if (mode != 0) {                                                                                          \
      const size_t lb = cfr::stage_layout(v.w, mode == 2).bytes;                                              \
      if (mode == 2) {                                                                                        \
        if (v.w.bits == 15) return cfr::launch_staged(kStagedThreads, KERNEL<15, true>, g, lb, s, __VA_ARGS__); \
        if (v.w.bits == 16) return cfr::launch_staged(kStagedThreads, KERNEL<16, true>, g, lb, s, __VA_ARGS__); \
        return cfr::launch_staged(kStagedThreads, KERNEL<0, true>, g, lb, s, __VA_ARGS__);                    \
      }                                                                                                       \
      if (v.w.bits == 15) return cfr::launch_staged(kStagedThreads, KERNEL<15, false>, g, lb, s, __VA_ARGS__); \
      if (v.w.bits == 16) return cfr::launch_staged(kStagedThreads, KERNEL<16, false>, g, lb, s, __VA_ARGS__); \
      return cfr::launch_staged(kStagedThreads, KERNEL<0, false>, g, lb, s, __VA_ARGS__);                     \
    }                                                                                                         \
  } while (0)

// ---- the line layout (chromofold_index.h, cf_fm_lines_*), derived on the device from the RRR levels:
//   * level l's bitvector as records of 16 u32: word 0 = ones in bits [0, 480 r) of the level, words 1..15 = bits
//     [480 r, 480 r + 480) LSB-first (32 RRR blocks). A rank1 reads one 64-byte line; on the RRR level it reads
//     three or four (samples, class words, offset bits) plus the unrank table;
//   * a per-symbol table lfb[c] = C[c] - e(c), e(c) = where the rank walk of c from position 0 ends on the last
//     level. The walk of rank(c, i) maps its start-of-c chain p and its position chain a by the same rule and p
//     never depends on i, so rank(c, i) = a_L - e(c) and LF(i) = C[c] + rank(c, i) = a_L + lfb[c].
// Backward search then takes 2 rank1 per level (lo and hi) and the LF step of locate 1 (the access walk of i is the
// rank walk of i for c = BWT[i]); every result equals the RRR kernels' above.

constexpr uint32_t kLineBits = 480;  // payload bits of a 64-byte record (word 0 is the rank before it)
__host__ __device__ inline uint32_t lines_nrec(int n) { return static_cast<uint32_t>(n) / kLineBits + 1u; }

// Records of the line layout: one wavefront per pair of records (2 sb, 2 sb + 1) of a level = RRR superblock sb
// (64 blocks x 15 bits = 960 bits). Lane i decodes block 64 sb + i (class nibble, offset at the superblock's offset
// sample + the wave's exclusive prefix sum of the widths, table unrank) and ORs its 15 bits into the record payload
// in LDS. Word 0 of record 2 sb is the superblock's rank sample; of record 2 sb + 1 that + the ones of blocks 0..31.
// Pairs past the last superblock (the record at bit n when n is a multiple of 960) hold the level's total ones.
constexpr unsigned kLinesBuildThreads = 256;
__global__ __launch_bounds__(kLinesBuildThreads) void fm_lines_build_kernel(cf_fm_view v, uint32_t *__restrict__ lines,
                                                                            uint32_t nrec, uint32_t npairs) {
  __shared__ uint32_t s_pay[kLinesBuildThreads / 64][2][16];
  const cf_rrrw_view &w = v.w;
  const uint32_t wv = threadIdx.x >> 6, lane = threadIdx.x & 63u;
  const uint32_t gw = blockIdx.x * (kLinesBuildThreads / 64) + wv;
  const uint32_t lvl = gw / npairs, sb = gw - lvl * npairs;
  const bool live = lvl < static_cast<uint32_t>(w.bits);
  if (lane < 32u) s_pay[wv][lane >> 4][lane & 15u] = 0u;
  __syncthreads();
  const uint32_t nblocks = (static_cast<uint32_t>(v.n) + cfd::kRrrT - 1) / cfd::kRrrT;
  const uint32_t blk = sb * 64u + lane;
  const bool inside = live && sb < static_cast<uint32_t>(w.nsb) && blk < nblocks;
  uint32_t k = 0;
  if (inside) k = (w.classes[static_cast<size_t>(lvl) * w.cwords + (blk >> 3)] >> (4u * (blk & 7u))) & 15u;
  const int wd = cfd::width_of(static_cast<int>(k));
  int pre = wd;  // inclusive prefix sum of the widths over the wave
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(pre, d);
    if (lane >= static_cast<uint32_t>(d)) pre += o;
  }
  int ones = static_cast<int>(k);  // ones of blocks 0..31 of the superblock (lanes 0..31)
#pragma unroll
  for (int d = 1; d < 32; d <<= 1) ones += __shfl_xor(ones, d);
  ones = __shfl(ones, 0);
  uint32_t rank0 = 0;
  if (live) {
    if (sb < static_cast<uint32_t>(w.nsb)) {
      const size_t srow = static_cast<size_t>(lvl) * (w.nsb + 1) + sb, arow = static_cast<size_t>(lvl) * w.na + (sb >> 5);
      rank0 = static_cast<uint32_t>(w.rank_a[arow] + w.rank_d[srow]);
      if (inside && wd > 0) {
        const int64_t at = static_cast<int64_t>(w.offbase[lvl]) + w.off_a[arow] + w.off_d[srow] + (pre - wd);
        k = cfr::kTab.unrank[cfr::kTab.base[k] + cfr::read_bits(w.offsets, at, wd)];
      } else if (inside) {
        k = cfr::kTab.unrank[cfr::kTab.base[k]];
      }
    } else {
      rank0 = static_cast<uint32_t>(v.n - w.zeros[lvl]);
    }
  }
  if (inside) {  // k = the block's 15 bits now
    const uint32_t bit = 15u * (lane & 31u);
    uint32_t *pay = s_pay[wv][lane >> 5] + 1;
    atomicOr(pay + (bit >> 5), k << (bit & 31u));
    if ((bit & 31u) > 17u) atomicOr(pay + (bit >> 5) + 1, k >> (32u - (bit & 31u)));
  }
  __syncthreads();
  const uint32_t r = lane >> 4, j = lane & 15u, rec = 2u * sb + r;
  if (live && lane < 32u && rec < nrec) {
    const uint32_t word = j == 0 ? rank0 + (r ? static_cast<uint32_t>(ones) : 0u) : s_pay[wv][r][j];
    lines[(static_cast<size_t>(lvl) * nrec + rec) * 16u + j] = word;
  }
}

// lfb[c] = C[c] - e(c), one thread per symbol (the start-of-c chain on the RRR levels).
template <int LEVELS>
__global__ __launch_bounds__(kThreads) void fm_lines_lfb_kernel(cf_fm_view v, int32_t *__restrict__ lfb) {
  const int c = blockIdx.x * static_cast<int>(kThreads) + static_cast<int>(threadIdx.x);
  if (c >= v.sigma) return;
  const int L = LEVELS > 0 ? LEVELS : v.w.bits;
  int p = 0;
  for (int lvl = 0; lvl < L; ++lvl) {
    const int rp = cfr::rank1_lvl<false>(v.w, lvl, p, nullptr);
    p = (c >> (L - 1 - lvl)) & 1 ? v.w.zeros[lvl] + rp : p - rp;
  }
  lfb[c] = v.C[c] - p;
}

// One line record into registers (four 16-byte loads).
__device__ __forceinline__ void load_record(const uint32_t *__restrict__ rec, uint32_t (&w)[16]) {
  const uint4 *q = reinterpret_cast<const uint4 *>(rec);
  const uint4 a = q[0], b = q[1], c = q[2], d = q[3];
  w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
  w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
  w[8] = c.x; w[9] = c.y; w[10] = c.z; w[11] = c.w;
  w[12] = d.x; w[13] = d.y; w[14] = d.z; w[15] = d.w;
}

// Ones of the level before bit `off` of the record (word 0 + the payload's bits [0, off)); with kBit the bit at off.
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

struct LinesArgs {
  const uint32_t *rec;   // level records, [bits][nrec][16]
  const int32_t *lfb;    // [sigma]
  uint32_t nrec;
};

__host__ inline LinesArgs lines_args(const cf_fm_view &v, const uint32_t *lines) {
  const uint32_t nrec = lines_nrec(v.n);
  return {lines, reinterpret_cast<const int32_t *>(lines + static_cast<size_t>(v.w.bits) * nrec * 16u), nrec};
}

// One backward-search step on the line layout: [lo, hi) -> [lfb[c] + a_L, lfb[c] + b_L). When a and b fall in
// the same record (most steps once the interval is narrow) the second load hits the line the first brought in.
template <int LEVELS>
__device__ __forceinline__ void lines_step(const cf_fm_view &v, const LinesArgs &la, int c, int &lo, int &hi) {
  const int L = LEVELS > 0 ? LEVELS : v.w.bits;
  uint32_t a = static_cast<uint32_t>(lo), b = static_cast<uint32_t>(hi);
  for (int lvl = 0; lvl < L; ++lvl) {
    const uint32_t *lv = la.rec + static_cast<size_t>(lvl) * la.nrec * 16u;
    const uint32_t ra_rec = a / kLineBits, rb_rec = b / kLineBits;
    uint32_t wa[16], wb[16];
    load_record(lv + ra_rec * 16u, wa);
    load_record(lv + rb_rec * 16u, wb);
    const int ra = record_rank<false>(wa, a - ra_rec * kLineBits, nullptr);
    const int rb = record_rank<false>(wb, b - rb_rec * kLineBits, nullptr);
    if ((c >> (L - 1 - lvl)) & 1) {
      const uint32_t z = static_cast<uint32_t>(v.w.zeros[lvl]);
      a = z + ra;
      b = z + rb;
    } else {
      a -= ra;
      b -= rb;
    }
  }
  const int f = la.lfb[c];
  lo = f + static_cast<int>(a);
  hi = f + static_cast<int>(b);
}

// Backward search on the line layout. A workgroup owns `per` consecutive patterns and its lanes take the next one
// from an LDS counter whenever they finish one (pattern lengths vary); each loop iteration consumes one symbol
// (right to left, reference fm_search_device.cuh:31-48) or stores a result.
template <int LEVELS>
__global__ __launch_bounds__(kThreads) void fm_search_lines_kernel(cf_fm_view v, LinesArgs la,
                                                                   const int32_t *__restrict__ pat,
                                                                   const int32_t *__restrict__ pstart,
                                                                   const int32_t *__restrict__ plen, size_t npat,
                                                                   uint32_t *__restrict__ cnt_out,
                                                                   int32_t *__restrict__ lo_out,
                                                                   int32_t *__restrict__ hi_out) {
  __shared__ uint32_t s_next;
  const ItemQueue q = item_queue(npat, &s_next);
  size_t t = q.take();
  bool active = t < q.end;
  int st = 0, k = 0, lo = 0, hi = 0;
  if (active) {
    st = pstart[t];
    k = plen[t];
    hi = v.n;
  }
  while (__any(active)) {
    if (active) {
      if (k > 0) {
        --k;
        const int c = pat[st + k];
        if (c < 0 || c >= v.sigma) {
          lo = hi = 0;
        } else if (lo < hi) {
          lines_step<LEVELS>(v, la, c, lo, hi);
        }
      } else {
        if (cnt_out) cnt_out[t] = static_cast<uint32_t>(hi - lo);
        if (lo_out) {
          lo_out[t] = lo;
          hi_out[t] = hi;
        }
        t = q.take();
        active = t < q.end;
        if (active) {
          st = pstart[t];
          k = plen[t];
          lo = 0;
          hi = v.n;
        }
      }
    }
  }
}

// Locate on the line layout (reference fm_search_device.cuh:52-62): one LF step per loop iteration, c and LF(p)
// from one walk of p (the record's bit gives c's next bit, its rank the next position).
template <int LEVELS>
__global__ __launch_bounds__(kThreads) void fm_locate_lines_kernel(cf_fm_view v, LinesArgs la,
                                                                   const int32_t *__restrict__ rows,
                                                                   int32_t *__restrict__ out, size_t nocc) {
  __shared__ uint32_t s_next;
  const ItemQueue q = item_queue(nocc, &s_next);
  const int L = LEVELS > 0 ? LEVELS : v.w.bits;
  size_t t = q.take();
  bool active = t < q.end;
  int p = active ? rows[t] : 0, steps = 0;
  while (__any(active)) {
    if (active) {
      if ((v.mwords[p >> 5] >> (p & 31)) & 1u) {
        const int idx = cfp::rank1(v.mwords, v.msb, p);
        out[t] = static_cast<int32_t>((static_cast<int64_t>(v.sval[idx]) + steps) % v.n);
        t = q.take();
        active = t < q.end;
        if (active) {
          p = rows[t];
          steps = 0;
        }
      } else {
        uint32_t a = static_cast<uint32_t>(p);
        int c = 0;
        for (int lvl = 0; lvl < L; ++lvl) {
          const uint32_t rec = a / kLineBits;
          uint32_t w[16];
          load_record(la.rec + (static_cast<size_t>(lvl) * la.nrec + rec) * 16u, w);
          int bit;
          const int r = record_rank<true>(w, a - rec * kLineBits, &bit);
          c = (c << 1) | bit;
          a = bit ? static_cast<uint32_t>(v.w.zeros[lvl] + r) : a - static_cast<uint32_t>(r);
        }
        p = static_cast<int>(a) + la.lfb[c];
        ++steps;
      }
    }
  }
}

// Items per lane of a line-layout workgroup (the LDS queue balances within it; the hardware dispatcher across).
constexpr unsigned kLinesItemsPerLane = 4;

#define CF_FM_DISPATCH(LAUNCH) \
  switch (v.w.bits) {         \
    case 7: LAUNCH(7); break;  \
    case 15: LAUNCH(15); break; \
    case 16: LAUNCH(16); break; \
    default: LAUNCH(0); break; \
  }

}  // namespace

extern "C" cf_status cf_fm_count_async(cf_fm_view v, const int32_t *pat, const int32_t *pstart, const int32_t *plen,
                                       uint32_t *out, size_t npat, void *stream) {
  // reference src/cuda/fm_search.cu:53: null classes / pattern arrays / output rejected before any device call
  if (!v.w.classes || !pat || !pstart || !plen || !out) return CF_ERR_INVALID_ARGUMENT;
  if (npat == 0) return CF_OK;
  if (v.w.bits <= 0 || v.w.bits > 31 || v.n <= 0) return CF_ERR_INVALID_ARGUMENT;
  const hipStream_t s = cfd::as_stream(stream);
  CF_FM_STAGED(fm_count_staged_kernel, npat, v, pat, pstart, plen, out, npat);
  const unsigned blocks = cfd::grid_for(npat, kThreads);
#define CF_LAUNCH(L) fm_count_kernel<L><<<blocks, kThreads, 0, s>>>(v, pat, pstart, plen, out, npat)
  CF_FM_DISPATCH(CF_LAUNCH)
#undef CF_LAUNCH
  return cfd::launch_status();
}

extern "C" cf_status cf_fm_ranges_async(cf_fm_view v, const int32_t *pat, const int32_t *pstart,
                                        const int32_t *plen, int32_t *lo_out, int32_t *hi_out, size_t npat,
                                        void *stream) {
  // reference src/cuda/fm_search.cu:67
  if (!v.w.classes || !pat || !pstart || !plen || !lo_out || !hi_out) return CF_ERR_INVALID_ARGUMENT;
  if (npat == 0) return CF_OK;
  if (v.w.bits <= 0 || v.w.bits > 31 || v.n <= 0) return CF_ERR_INVALID_ARGUMENT;
  const hipStream_t s = cfd::as_stream(stream);
  CF_FM_STAGED(fm_ranges_staged_kernel, npat, v, pat, pstart, plen, lo_out, hi_out, npat);
  const unsigned blocks = cfd::grid_for(npat, kThreads);
#define CF_LAUNCH(L) fm_ranges_kernel<L><<<blocks, kThreads, 0, s>>>(v, pat, pstart, plen, lo_out, hi_out, npat)
  CF_FM_DISPATCH(CF_LAUNCH)
#undef CF_LAUNCH
  return cfd::launch_status();
}

extern "C" cf_status cf_fm_locate_async(cf_fm_view v, const int32_t *r_in, int32_t *out, size_t nocc,
                                        void *stream) {
  // reference src/cuda/fm_search.cu:80
  if (!v.w.classes || !r_in || !out) return CF_ERR_INVALID_ARGUMENT;
  if (nocc == 0) return CF_OK;
  if (v.w.bits <= 0 || v.w.bits > 31 || v.n <= 0 || !v.mwords || !v.msb || !v.sval || !v.C)
    return CF_ERR_INVALID_ARGUMENT;
  const hipStream_t s = cfd::as_stream(stream);
  CF_FM_STAGED(fm_locate_staged_kernel, nocc, v, r_in, out, nocc);
  const unsigned blocks = cfd::grid_for(nocc, kThreads);
#define CF_LAUNCH(L) fm_locate_kernel<L><<<blocks, kThreads, 0, s>>>(v, r_in, out, nocc)
  CF_FM_DISPATCH(CF_LAUNCH)
#undef CF_LAUNCH
  return cfd::launch_status();
}

// ---- line layout entry points (chromofold_index.h) ----
extern "C" uint64_t cf_fm_lines_bytes(cf_fm_view v) {
  if (v.w.bits <= 0 || v.w.bits > 31 || v.n <= 0 || v.sigma <= 0) return 0;
  return (static_cast<uint64_t>(v.w.bits) * lines_nrec(v.n) * 16u + static_cast<uint64_t>(v.sigma)) * 4u;
}

// The view fields the line-layout kernels read, and a 16-byte aligned `lines` (records are read as uint4).
static bool lines_view_ok(const cf_fm_view &v, const uint32_t *lines) {
  return lines && (reinterpret_cast<uintptr_t>(lines) & 15u) == 0 && v.w.classes && v.w.bits > 0 &&
         v.w.bits <= 31 && v.n > 0 && v.sigma > 0 && v.C && v.w.zeros && (v.sigma - 1) >> v.w.bits == 0;
}

extern "C" cf_status cf_fm_lines_build_async(cf_fm_view v, uint32_t *lines, uint64_t bytes, void *stream) {
  if (!lines_view_ok(v, lines) || !v.w.offsets || !v.w.rank_a || !v.w.rank_d || !v.w.off_a || !v.w.off_d ||
      !v.w.offbase)
    return CF_ERR_INVALID_ARGUMENT;
  if (bytes < cf_fm_lines_bytes(v)) return CF_ERR_INVALID_ARGUMENT;
  const hipStream_t s = cfd::as_stream(stream);
  const uint32_t nrec = lines_nrec(v.n), npairs = (nrec + 1) / 2;
  const uint64_t waves = static_cast<uint64_t>(v.w.bits) * npairs;
  const uint64_t blocks = (waves + kLinesBuildThreads / 64 - 1) / (kLinesBuildThreads / 64);
  if (blocks > 0x7fffffffu) return CF_ERR_INVALID_ARGUMENT;
  fm_lines_build_kernel<<<static_cast<unsigned>(blocks), kLinesBuildThreads, 0, s>>>(v, lines, nrec, npairs);
  int32_t *lfb = reinterpret_cast<int32_t *>(lines + static_cast<size_t>(v.w.bits) * nrec * 16u);
  const unsigned g = cfd::grid_for(static_cast<size_t>(v.sigma), kThreads);
#define CF_LAUNCH(L) fm_lines_lfb_kernel<L><<<g, kThreads, 0, s>>>(v, lfb)
  CF_FM_DISPATCH(CF_LAUNCH)
#undef CF_LAUNCH
  return cfd::launch_status();
}

static unsigned lines_grid(size_t count) {
  const size_t per = static_cast<size_t>(kThreads) * kLinesItemsPerLane;
  return static_cast<unsigned>((count + per - 1) / per);
}

extern "C" cf_status cf_fm_count_lines_async(cf_fm_view v, const uint32_t *lines, const int32_t *pat,
                                             const int32_t *pstart, const int32_t *plen, uint32_t *out, size_t npat,
                                             void *stream) {
  if (!pat || !pstart || !plen || !out || !lines_view_ok(v, lines)) return CF_ERR_INVALID_ARGUMENT;
  if (npat == 0) return CF_OK;
  if (npat > (static_cast<size_t>(1) << 40)) return CF_ERR_INVALID_ARGUMENT;
  const hipStream_t s = cfd::as_stream(stream);
  const LinesArgs la = lines_args(v, lines);
  const unsigned g = lines_grid(npat);
#define CF_LAUNCH(L) \
  fm_search_lines_kernel<L><<<g, kThreads, 0, s>>>(v, la, pat, pstart, plen, npat, out, nullptr, nullptr)
  CF_FM_DISPATCH(CF_LAUNCH)
#undef CF_LAUNCH
  return cfd::launch_status();
}

extern "C" cf_status cf_fm_ranges_lines_async(cf_fm_view v, const uint32_t *lines, const int32_t *pat,
                                              const int32_t *pstart, const int32_t *plen, int32_t *lo_out,
                                              int32_t *hi_out, size_t npat, void *stream) {
  if (!pat || !pstart || !plen || !lo_out || !hi_out || !lines_view_ok(v, lines)) return CF_ERR_INVALID_ARGUMENT;
  if (npat == 0) return CF_OK;
  if (npat > (static_cast<size_t>(1) << 40)) return CF_ERR_INVALID_ARGUMENT;
  const hipStream_t s = cfd::as_stream(stream);
  const LinesArgs la = lines_args(v, lines);
  const unsigned g = lines_grid(npat);
#define CF_LAUNCH(L) \
  fm_search_lines_kernel<L><<<g, kThreads, 0, s>>>(v, la, pat, pstart, plen, npat, nullptr, lo_out, hi_out)
  CF_FM_DISPATCH(CF_LAUNCH)
#undef CF_LAUNCH
  return cfd::launch_status();
}

extern "C" cf_status cf_fm_locate_lines_async(cf_fm_view v, const uint32_t *lines, const int32_t *r_in, int32_t *out,
                                              size_t nocc, void *stream) {
  if (!r_in || !out || !lines_view_ok(v, lines) || !v.mwords || !v.msb || !v.sval) return CF_ERR_INVALID_ARGUMENT;
  if (nocc == 0) return CF_OK;
  if (nocc > (static_cast<size_t>(1) << 40)) return CF_ERR_INVALID_ARGUMENT;
  const hipStream_t s = cfd::as_stream(stream);
  const LinesArgs la = lines_args(v, lines);
  const unsigned g = lines_grid(nocc);
#define CF_LAUNCH(L) fm_locate_lines_kernel<L><<<g, kThreads, 0, s>>>(v, la, r_in, out, nocc)
  CF_FM_DISPATCH(CF_LAUNCH)
#undef CF_LAUNCH
  return cfd::launch_status();
}
