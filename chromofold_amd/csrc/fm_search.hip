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
#include "lines_core.hpp"
#include "quads_core.hpp"

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

// ---- the derived layouts (chromofold_index.h cf_fm_lines_*, cf_fm_quads_*). With lfb[c] = C[c] - e(c), e(c) the end
// of the walk of c from position 0, an LF step is LF(i) = walk(i) + lfb[c], so backward search walks lo and hi
// (one record per level each) and an LF step of locate walks once (the access walk of i is the rank walk of i for
// c = BWT[i]); every result equals the RRR kernels' above.
//   line layout (lines_core.hpp): the binary levels, `bits` records per walk;
//   4-ary layout (quads_core.hpp): base-4 digits, ceil(bits / 2) records per walk.
struct WalkArgs {
  const uint32_t *rec;  // level records, [levels][nrec][16]
  const int32_t *lfb;   // [sigma]
  const uint32_t *Z;    // 4-ary layout: digit bucket starts [levels][4]
  uint32_t nrec;
};

__host__ inline WalkArgs lines_args(const cf_fm_view &v, const uint32_t *lines) {
  const uint32_t nrec = cfl::nrec_for(static_cast<uint64_t>(v.n));
  return {lines, reinterpret_cast<const int32_t *>(lines + static_cast<size_t>(v.w.bits) * nrec * cfl::kRecWords),
          nullptr, nrec};
}

__host__ inline WalkArgs quads_args(const cf_fm_view &v, const uint32_t *quads) {
  const cfq::Layout L = cfq::layout(v.w.bits, static_cast<uint64_t>(v.n), v.sigma);
  const uint32_t *Z = quads + L.rec_words;
  return {quads, reinterpret_cast<const int32_t *>(Z + L.z_words), Z, L.nrec};
}

template <int LEVELS>
struct LinesWalk {
  // One backward-search step: [lo, hi) -> [lfb[c] + a_L, lfb[c] + b_L). When a and b fall in the same record (most
  // steps once the interval is narrow) the second load hits the line the first brought in.
  __device__ static __forceinline__ void range(const cf_fm_view &v, const WalkArgs &la, int c, int &lo, int &hi) {
    const int L = LEVELS > 0 ? LEVELS : v.w.bits;
    uint32_t a = static_cast<uint32_t>(lo), b = static_cast<uint32_t>(hi);
    for (int lvl = 0; lvl < L; ++lvl) {
      // both records' loads issued before either rank is counted (two latencies per level would serialise)
      const uint32_t *lv = la.rec + static_cast<size_t>(lvl) * la.nrec * cfl::kRecWords;
      const uint32_t ra_rec = min(a / cfl::kLineBits, la.nrec - 1u), rb_rec = min(b / cfl::kLineBits, la.nrec - 1u);
      uint32_t wa[16], wb[16];
      cfl::load_record(lv + ra_rec * cfl::kRecWords, wa);
      cfl::load_record(lv + rb_rec * cfl::kRecWords, wb);
      const int ra = cfl::record_rank<false>(wa, a - ra_rec * cfl::kLineBits, nullptr);
      const int rb = cfl::record_rank<false>(wb, b - rb_rec * cfl::kLineBits, nullptr);
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
  // LF(p): c's bits and the next position from one walk of p (each record's bit at the position).
  __device__ static __forceinline__ int lf(const cf_fm_view &v, const WalkArgs &la, int p) {
    const int L = LEVELS > 0 ? LEVELS : v.w.bits;
    uint32_t a = static_cast<uint32_t>(p);
    int c = 0;
    for (int lvl = 0; lvl < L; ++lvl) {
      int bit;
      const int r = cfl::rank1<true>(la.rec, la.nrec, lvl, a, &bit);
      c = (c << 1) | bit;
      a = bit ? static_cast<uint32_t>(v.w.zeros[lvl] + r) : a - static_cast<uint32_t>(r);
    }
    return static_cast<int>(a) + la.lfb[c];
  }
};

template <int L4>
struct QuadsWalk {
  __device__ static __forceinline__ void range(const cf_fm_view &v, const WalkArgs &la, int c, int &lo, int &hi) {
    const uint32_t L = L4 > 0 ? static_cast<uint32_t>(L4) : cfq::levels_for(v.w.bits);
    uint32_t a = static_cast<uint32_t>(lo), b = static_cast<uint32_t>(hi);
    for (uint32_t l = 0; l < L; ++l) {
      const uint32_t d = (static_cast<uint32_t>(c) >> (2u * (L - 1u - l))) & 3u;
      const uint32_t *lv = la.rec + static_cast<size_t>(l) * la.nrec * cfq::kRecWords;
      const uint32_t ra_rec = min(a / cfq::kDigits, la.nrec - 1u), rb_rec = min(b / cfq::kDigits, la.nrec - 1u);
      uint32_t wa[16], wb[16];
      cfq::load_record(lv + ra_rec * cfq::kRecWords, wa);
      cfq::load_record(lv + rb_rec * cfq::kRecWords, wb);
      const uint32_t z = la.Z[4 * l + d];
      a = z + cfq::record_rank(wa, ra_rec * cfq::kDigits, min(a - ra_rec * cfq::kDigits, cfq::kDigits), d);
      b = z + cfq::record_rank(wb, rb_rec * cfq::kDigits, min(b - rb_rec * cfq::kDigits, cfq::kDigits), d);
    }
    const int f = la.lfb[c];
    lo = f + static_cast<int>(a);
    hi = f + static_cast<int>(b);
  }
  __device__ static __forceinline__ int lf(const cf_fm_view &v, const WalkArgs &la, int p) {
    const uint32_t L = L4 > 0 ? static_cast<uint32_t>(L4) : cfq::levels_for(v.w.bits);
    uint32_t a = static_cast<uint32_t>(p), c = 0;
    for (uint32_t l = 0; l < L; ++l) {
      uint32_t d;
      a = cfq::step<true>(la.rec, la.nrec, la.Z, l, a, 0u, &d);
      c = (c << 2) | d;
    }
    return static_cast<int>(a) + la.lfb[c];
  }
};

// Backward search on a derived layout. A workgroup owns `per` consecutive patterns and its lanes take the next one
// from an LDS counter whenever they finish one (pattern lengths vary); each loop iteration consumes one symbol
// (right to left, reference fm_search_device.cuh:31-48) or stores a result.
template <typename Walk>
__global__ __launch_bounds__(kThreads) void fm_search_walk_kernel(cf_fm_view v, WalkArgs la,
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
          Walk::range(v, la, c, lo, hi);
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

// Locate on a derived layout (reference fm_search_device.cuh:52-62): one LF step per loop iteration.
template <typename Walk>
__global__ __launch_bounds__(kThreads) void fm_locate_walk_kernel(cf_fm_view v, WalkArgs la,
                                                                  const int32_t *__restrict__ rows,
                                                                  int32_t *__restrict__ out, size_t nocc) {
  __shared__ uint32_t s_next;
  const ItemQueue q = item_queue(nocc, &s_next);
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
        p = Walk::lf(v, la, p);
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
  return (static_cast<uint64_t>(v.w.bits) * cfl::nrec_for(static_cast<uint64_t>(v.n)) * cfl::kRecWords +
          static_cast<uint64_t>(v.sigma)) * 4u;
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
  const uint32_t nblocks = static_cast<uint32_t>((static_cast<int64_t>(v.n) + cfd::kRrrT - 1) / cfd::kRrrT);
  return cfl::build(v.w, lines, cfl::nrec_for(static_cast<uint64_t>(v.n)), nblocks, v.n, v.sigma, v.C,
                    cfd::as_stream(stream));
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
  const WalkArgs la = lines_args(v, lines);
  const unsigned g = lines_grid(npat);
#define CF_LAUNCH(L) \
  fm_search_walk_kernel<LinesWalk<L>><<<g, kThreads, 0, s>>>(v, la, pat, pstart, plen, npat, out, nullptr, nullptr)
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
  const WalkArgs la = lines_args(v, lines);
  const unsigned g = lines_grid(npat);
#define CF_LAUNCH(L) \
  fm_search_walk_kernel<LinesWalk<L>><<<g, kThreads, 0, s>>>(v, la, pat, pstart, plen, npat, nullptr, lo_out, hi_out)
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
  const WalkArgs la = lines_args(v, lines);
  const unsigned g = lines_grid(nocc);
#define CF_LAUNCH(L) fm_locate_walk_kernel<LinesWalk<L>><<<g, kThreads, 0, s>>>(v, la, r_in, out, nocc)
  CF_FM_DISPATCH(CF_LAUNCH)
#undef CF_LAUNCH
  return cfd::launch_status();
}

// ---- 4-ary layout entry points (chromofold_index.h) ----
static bool quads_fm_ok(const cf_fm_view &v) {
  return v.w.classes && v.w.bits > 0 && v.w.bits <= 24 && v.n > 0 && v.sigma > 0 && v.C && v.w.zeros &&
         (v.sigma - 1) >> v.w.bits == 0 && static_cast<uint64_t>(v.n) <= static_cast<uint64_t>(v.w.nsb) * 960u;
}

extern "C" uint64_t cf_fm_quads_bytes(cf_fm_view v) {
  if (!quads_fm_ok(v)) return 0;
  return cfq::layout(v.w.bits, static_cast<uint64_t>(v.n), v.sigma).bytes();
}

extern "C" uint64_t cf_fm_quads_workspace_bytes(cf_fm_view v) {
  if (!quads_fm_ok(v)) return 0;
  return cfq::workspace_bytes(static_cast<uint64_t>(v.n), cfq::nrec_for(static_cast<uint64_t>(v.n)));
}

extern "C" cf_status cf_fm_quads_build_async(cf_fm_view v, uint32_t *quads, uint64_t bytes, void *workspace,
                                             uint64_t workspace_bytes, void *stream) {
  if (!quads_fm_ok(v) || !quads || (reinterpret_cast<uintptr_t>(quads) & 15u) != 0 || !workspace ||
      (reinterpret_cast<uintptr_t>(workspace) & 255u) != 0 || !v.w.offsets || !v.w.rank_a || !v.w.rank_d ||
      !v.w.off_a || !v.w.off_d || !v.w.offbase)
    return CF_ERR_INVALID_ARGUMENT;
  if (bytes < cf_fm_quads_bytes(v) || workspace_bytes < cf_fm_quads_workspace_bytes(v)) return CF_ERR_INVALID_ARGUMENT;
  return cfq::build(v.w, static_cast<uint64_t>(v.n), v.sigma, v.C, quads, workspace, cfd::as_stream(stream));
}

static bool quads_ptr_ok(const cf_fm_view &v, const uint32_t *quads) {
  return quads && (reinterpret_cast<uintptr_t>(quads) & 15u) == 0 && quads_fm_ok(v);
}

#define CF_QUADS_DISPATCH(LAUNCH)           \
  if (cfq::levels_for(v.w.bits) == 8) {     \
    LAUNCH(QuadsWalk<8>);                   \
  } else {                                  \
    LAUNCH(QuadsWalk<0>);                   \
  }

extern "C" cf_status cf_fm_count_quads_async(cf_fm_view v, const uint32_t *quads, const int32_t *pat,
                                             const int32_t *pstart, const int32_t *plen, uint32_t *out, size_t npat,
                                             void *stream) {
  if (!pat || !pstart || !plen || !out || !quads_ptr_ok(v, quads)) return CF_ERR_INVALID_ARGUMENT;
  if (npat == 0) return CF_OK;
  if (npat > (static_cast<size_t>(1) << 40)) return CF_ERR_INVALID_ARGUMENT;
  const hipStream_t s = cfd::as_stream(stream);
  const WalkArgs la = quads_args(v, quads);
  const unsigned g = lines_grid(npat);
#define CF_LAUNCH(W) fm_search_walk_kernel<W><<<g, kThreads, 0, s>>>(v, la, pat, pstart, plen, npat, out, nullptr, nullptr)
  CF_QUADS_DISPATCH(CF_LAUNCH)
#undef CF_LAUNCH
  return cfd::launch_status();
}

extern "C" cf_status cf_fm_ranges_quads_async(cf_fm_view v, const uint32_t *quads, const int32_t *pat,
                                              const int32_t *pstart, const int32_t *plen, int32_t *lo_out,
                                              int32_t *hi_out, size_t npat, void *stream) {
  if (!pat || !pstart || !plen || !lo_out || !hi_out || !quads_ptr_ok(v, quads)) return CF_ERR_INVALID_ARGUMENT;
  if (npat == 0) return CF_OK;
  if (npat > (static_cast<size_t>(1) << 40)) return CF_ERR_INVALID_ARGUMENT;
  const hipStream_t s = cfd::as_stream(stream);
  const WalkArgs la = quads_args(v, quads);
  const unsigned g = lines_grid(npat);
#define CF_LAUNCH(W) \
  fm_search_walk_kernel<W><<<g, kThreads, 0, s>>>(v, la, pat, pstart, plen, npat, nullptr, lo_out, hi_out)
  CF_QUADS_DISPATCH(CF_LAUNCH)
#undef CF_LAUNCH
  return cfd::launch_status();
}

extern "C" cf_status cf_fm_locate_quads_async(cf_fm_view v, const uint32_t *quads, const int32_t *r_in, int32_t *out,
                                              size_t nocc, void *stream) {
  if (!r_in || !out || !quads_ptr_ok(v, quads) || !v.mwords || !v.msb || !v.sval) return CF_ERR_INVALID_ARGUMENT;
  if (nocc == 0) return CF_OK;
  if (nocc > (static_cast<size_t>(1) << 40)) return CF_ERR_INVALID_ARGUMENT;
  const hipStream_t s = cfd::as_stream(stream);
  const WalkArgs la = quads_args(v, quads);
  const unsigned g = lines_grid(nocc);
#define CF_LAUNCH(W) fm_locate_walk_kernel<W><<<g, kThreads, 0, s>>>(v, la, r_in, out, nocc)
  CF_QUADS_DISPATCH(CF_LAUNCH)
#undef CF_LAUNCH
  return cfd::launch_status();
}
