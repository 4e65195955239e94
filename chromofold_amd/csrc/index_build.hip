// index_build.hip — on-device construction of the compressed-domain search indexes (gfx950): the RRR wavelet matrix
// of a token array (the .cfrw arrays) and the FM-index side arrays of a text and its suffix array (BWT, C table,
// sampled-SA mark plane with its rank directory, sampled SA values).
//
// Output layout is the reference builder's, byte for byte (reference tools/build_index.cpp:90-218 RRR blocks,
// classes, offsets, samples and two-level split; :368-371 BWT of s = (tokens + 1) ++ [0]; :455-469 C / marks / msb /
// sval). The reference builds on the CPU, level after level; here every level is a handful of wide kernels:
//   plane    wave ballots pack the level's bit of 64 tokens per instruction;
//   blocks   one lane per 8 RRR blocks (one class word): class = popcount of the 15-bit block, offset = its
//            combinatorial-number-system rank, width from the fixed table;
//   scans    hipCUB exclusive sums of widths and classes give every block's offset bit and rank base;
//   pack     one lane per block ORs its offset into the level's offset words (global atomics: blocks share words);
//   samples  one lane per superblock writes the anchor / 16-bit delta pairs;
//   split    the stable zeros-then-ones partition for the next level: an exclusive scan of the zero flags, then a
//            scatter.
// The offset stream of a level is data dependent in length, so levels are built into worst-case slots of the
// workspace; cf_rrrw_build reads the per-level totals back once at the end (one synchronisation) and
// cf_rrrw_build_copy packs the slots into the caller's arrays.
#include <hipcub/hipcub.hpp>

#include <vector>

#include "cf_device.hpp"
#include "chromofold/chromofold_index.h"

namespace {

constexpr unsigned kThreads = 256;
constexpr int kT = cfd::kRrrT, kS = cfd::kRrrS, kK = cfd::kRrrK;

struct Binom {
  uint16_t c[16][16];
};
constexpr Binom make_binom() {
  Binom b{};
  for (int n = 0; n < 16; ++n) {
    b.c[n][0] = 1;
    for (int k = 1; k <= n; ++k) b.c[n][k] = static_cast<uint16_t>(b.c[n - 1][k - 1] + (k <= n - 1 ? b.c[n - 1][k] : 0));
  }
  return b;
}
__device__ const Binom kBinom = make_binom();

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

struct Geo {  // sizes fixed by (n, bits)
  uint64_t n;
  uint32_t bits, nblocks, cwords, nsb, na, owords_max;
};

Geo geo_of(uint64_t n, uint32_t bits) {
  Geo g{};
  g.n = n;
  g.bits = bits;
  g.nblocks = static_cast<uint32_t>((n + kT - 1) / kT);
  g.cwords = static_cast<uint32_t>((static_cast<uint64_t>(g.nblocks) * 4 + 31) / 32 + 1);
  g.nsb = (g.nblocks + kS - 1) / kS;
  g.na = (g.nsb + 1 + kK - 1) / kK;
  g.owords_max = static_cast<uint32_t>((static_cast<uint64_t>(g.nblocks) * 13 + 31) / 32 + 2);
  return g;
}

struct WsLayout {
  size_t cur, nxt, plane, width, ones, obit, ccum, zflag, zpos, scan_tmp, classes, rank_a, rank_d, off_a, off_d,
      offbase, zeros, level_bits, offsets, total;
};

WsLayout ws_layout(const Geo &g) {
  WsLayout L{};
  size_t scan_bytes = 0, scan2 = 0;
  // temp-storage size queries: a failure leaves the size 0 and the checked scan that uses it fails
  uint32_t *const none = nullptr;
  static_cast<void>(hipcub::DeviceScan::ExclusiveSum(nullptr, scan_bytes, none, none, static_cast<int>(g.nblocks + 1)));
  static_cast<void>(hipcub::DeviceScan::ExclusiveSum(nullptr, scan2, none, none, static_cast<int>(g.n)));
  scan_bytes = std::max(scan_bytes, scan2);
  size_t at = 0;
  auto take = [&](size_t bytes) {
    const size_t here = at;
    at += align256(bytes);
    return here;
  };
  const uint64_t nwords64 = (g.n + kThreads - 1) / kThreads * (kThreads / 64) + 1;  // every word a ballot writes + 1
  L.cur = take(4 * g.n);
  L.nxt = take(4 * g.n);
  L.plane = take(8 * nwords64);
  L.width = take(4ull * (g.nblocks + 1));
  L.ones = take(4ull * (g.nblocks + 1));
  L.obit = take(4ull * (g.nblocks + 1));
  L.ccum = take(4ull * (g.nblocks + 1));
  L.zflag = take(4 * g.n);
  L.zpos = take(4 * g.n);
  L.scan_tmp = take(scan_bytes);
  L.classes = take(4ull * g.bits * g.cwords);
  L.rank_a = take(4ull * g.bits * g.na);
  L.rank_d = take(2ull * g.bits * (g.nsb + 1));
  L.off_a = take(4ull * g.bits * g.na);
  L.off_d = take(2ull * g.bits * (g.nsb + 1));
  L.offbase = take(4ull * g.bits);
  L.zeros = take(4ull * g.bits);
  L.level_bits = take(8ull * g.bits);
  L.offsets = take(4ull * g.bits * g.owords_max);
  L.total = at;
  return L;
}

template <typename T>
T *at(void *ws, size_t off) {
  return reinterpret_cast<T *>(static_cast<uint8_t *>(ws) + off);
}

__global__ void fill_u32(uint32_t *p, size_t n, uint32_t v) {
  for (size_t i = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * kThreads)
    p[i] = v;
}

// bit `shift` of every token, 64 tokens per ballot; also the zero flags of the partition
__global__ void plane_kernel(const uint32_t *__restrict__ cur, uint64_t n, int shift, uint64_t *__restrict__ plane,
                             uint32_t *__restrict__ zflag) {
  const uint64_t i = blockIdx.x * static_cast<uint64_t>(kThreads) + threadIdx.x;
  const uint32_t b = i < n ? (cur[i] >> shift) & 1u : 0u;
  const uint64_t word = __ballot(b);
  if ((threadIdx.x & 63u) == 0) plane[i >> 6] = word;
  if (i < n) zflag[i] = b ^ 1u;
}

__device__ __forceinline__ uint32_t bits15(const uint64_t *__restrict__ plane, uint64_t pos) {
  const uint64_t w = pos >> 6;
  const int b = static_cast<int>(pos & 63);
  uint64_t v = plane[w] >> b;
  if (b > 64 - kT) v |= plane[w + 1] << (64 - b);
  return static_cast<uint32_t>(v & ((1u << kT) - 1u));
}

// one lane per class word (8 blocks): classes, per-block widths / ones / enumerative offsets
__global__ void blocks_kernel(const uint64_t *__restrict__ plane, uint32_t nblocks, uint32_t *__restrict__ classes,
                              uint32_t *__restrict__ width, uint32_t *__restrict__ ones, uint32_t *__restrict__ offs) {
  const uint32_t g = blockIdx.x * kThreads + threadIdx.x;
  const uint32_t ncw = (nblocks + 7) / 8;
  if (g >= ncw) return;
  uint32_t cw = 0;
  for (int e = 0; e < 8; ++e) {
    const uint32_t j = g * 8 + e;
    if (j >= nblocks) break;
    const uint32_t v = bits15(plane, static_cast<uint64_t>(j) * kT);  // bits past n are zero in the plane
    int k = 0;
    uint32_t o = 0;
    for (int c = 0; c < kT; ++c)
      if ((v >> c) & 1u) {
        ++k;
        o += kBinom.c[c][k];
      }
    cw |= static_cast<uint32_t>(k) << (4 * e);
    width[j] = static_cast<uint32_t>(cfd::width_of(k));
    ones[j] = static_cast<uint32_t>(k);
    offs[j] = o;
  }
  classes[g] = cw;
}

// offsets LSB-first at the block's scanned bit position (blocks share words: atomic OR)
__global__ void pack_kernel(const uint32_t *__restrict__ width, const uint32_t *__restrict__ obit,
                            const uint32_t *__restrict__ offs, uint32_t nblocks, uint32_t *__restrict__ words) {
  const uint32_t j = blockIdx.x * kThreads + threadIdx.x;
  if (j >= nblocks) return;
  const uint32_t w = width[j];
  if (!w) return;
  const uint32_t p = obit[j];
  const uint64_t v = static_cast<uint64_t>(offs[j]) << (p & 31);
  atomicOr(words + (p >> 5), static_cast<uint32_t>(v));
  if ((p & 31) + w > 32) atomicOr(words + (p >> 5) + 1, static_cast<uint32_t>(v >> 32));
}

// two-level samples of one level: anchors every kK superblocks (i32) + 16-bit deltas, for ranks and offsets
__global__ void samples_kernel(const uint32_t *__restrict__ ccum, const uint32_t *__restrict__ obit, uint32_t nblocks,
                               uint32_t nsb, uint32_t na, int32_t *__restrict__ rank_a, uint16_t *__restrict__ rank_d,
                               int32_t *__restrict__ off_a, uint16_t *__restrict__ off_d) {
  const uint32_t i = blockIdx.x * kThreads + threadIdx.x;
  if (i > nsb) return;
  const uint32_t b = min(i * kS, nblocks), a = i / kK, ba = min(a * kK * kS, nblocks);
  rank_d[i] = static_cast<uint16_t>(ccum[b] - ccum[ba]);
  off_d[i] = static_cast<uint16_t>(obit[b] - obit[ba]);
  if (i % kK == 0) {
    rank_a[a] = static_cast<int32_t>(ccum[b]);
    off_a[a] = static_cast<int32_t>(obit[b]);
  }
  (void)na;
}

__global__ void level_totals(const uint32_t *__restrict__ ccum, const uint32_t *__restrict__ obit, uint32_t nblocks,
                             uint64_t n, int lvl, int32_t *__restrict__ zeros, uint64_t *__restrict__ level_bits) {
  zeros[lvl] = static_cast<int32_t>(n - ccum[nblocks]);
  level_bits[lvl] = obit[nblocks];
}

// stable zeros-then-ones partition: zeros go to their scanned rank, ones after all zeros
__global__ void split_kernel(const uint32_t *__restrict__ cur, const uint32_t *__restrict__ zflag,
                             const uint32_t *__restrict__ zpos, const int32_t *__restrict__ zeros, int lvl, uint64_t n,
                             uint32_t *__restrict__ nxt) {
  const uint64_t i = blockIdx.x * static_cast<uint64_t>(kThreads) + threadIdx.x;
  if (i >= n) return;
  const uint64_t z = static_cast<uint32_t>(zeros[lvl]);
  nxt[zflag[i] ? zpos[i] : z + (i - zpos[i])] = cur[i];
}

// ------------------------------------------------------------------------------------------------ FM side arrays
__global__ void bwt_kernel(const int32_t *__restrict__ s, const int32_t *__restrict__ sa, int32_t n,
                           uint32_t *__restrict__ bwt) {
  const int i = blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  const int p = sa[i];
  bwt[i] = static_cast<uint32_t>(s[p == 0 ? n - 1 : p - 1]);
}

__global__ void marks_kernel(const int32_t *__restrict__ sa, int32_t n, int32_t sample, uint32_t *__restrict__ mwords,
                             uint32_t *__restrict__ wcount) {
  const int w = blockIdx.x * kThreads + threadIdx.x;
  const int nw = (n + 31) / 32;
  if (w >= nw) return;
  uint32_t m = 0;
  for (int b = 0; b < 32; ++b) {
    const int i = w * 32 + b;
    if (i < n && sa[i] % sample == 0) m |= 1u << b;
  }
  mwords[w] = m;
  wcount[w] = __popc(m);
}

__global__ void sval_kernel(const int32_t *__restrict__ sa, int32_t n, const uint32_t *__restrict__ mwords,
                            const uint32_t *__restrict__ wbase, int32_t *__restrict__ sval) {
  const int i = blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  const uint32_t m = mwords[i >> 5];
  if (!((m >> (i & 31)) & 1u)) return;
  sval[wbase[i >> 5] + __popc(m & ((1u << (i & 31)) - 1u))] = sa[i];
}

__global__ void msb_kernel(const uint32_t *__restrict__ wbase, int32_t nw, int32_t nb, int32_t *__restrict__ msb) {
  const int j = blockIdx.x * kThreads + threadIdx.x;
  if (j > nb) return;
  msb[j] = static_cast<int32_t>(wbase[min(j * 8, nw)]);
}

// C[c] = number of text symbols < c = the first suffix-array row whose suffix starts with a symbol >= c (rows are
// sorted by first symbol). Row i writes C[c] for every c in (first[i-1], first[i]]; the last row also fills up to
// sigma - 1. No histogram, no atomics (a Zipf text makes per-symbol atomic counters contend heavily).
__global__ void c_table_kernel(const int32_t *__restrict__ s, const int32_t *__restrict__ sa, int32_t n, int32_t sigma,
                               int32_t *__restrict__ C) {
  const int i = blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  const int f = s[sa[i]];
  const int prev = i == 0 ? -1 : s[sa[i - 1]];
  for (int c = prev + 1; c <= f && c < sigma; ++c) C[c] = i;
  if (i == n - 1)
    for (int c = f + 1; c < sigma; ++c) C[c] = n;
}

}  // namespace

extern "C" uint64_t cf_rrrw_build_workspace_bytes(uint64_t n, uint32_t bits) {
  if (n == 0 || bits == 0 || bits > 31 || n >= (1ull << 31)) return 0;
  return ws_layout(geo_of(n, bits)).total;
}

extern "C" cf_status cf_rrrw_build(const uint32_t *tokens, uint64_t n, uint32_t bits, void *ws, uint64_t ws_bytes,
                                   cf_rrrw_layout *layout, void *stream) {
  if (!tokens || !ws || !layout || n == 0 || bits == 0) return CF_ERR_INVALID_ARGUMENT;
  if (bits > 31 || n >= (1ull << 31)) return CF_ERR_UNSUPPORTED;
  const Geo g = geo_of(n, bits);
  const WsLayout L = ws_layout(g);
  if (ws_bytes < L.total) return CF_ERR_INVALID_ARGUMENT;
  const hipStream_t st = cfd::as_stream(stream);
  uint32_t *cur = at<uint32_t>(ws, L.cur), *nxt = at<uint32_t>(ws, L.nxt);
  uint64_t *plane = at<uint64_t>(ws, L.plane);
  uint32_t *width = at<uint32_t>(ws, L.width), *ones = at<uint32_t>(ws, L.ones);
  uint32_t *obit = at<uint32_t>(ws, L.obit), *ccum = at<uint32_t>(ws, L.ccum);
  uint32_t *zflag = at<uint32_t>(ws, L.zflag), *zpos = at<uint32_t>(ws, L.zpos);
  uint32_t *offs = zpos;  // per-block enumerative offsets share the partition scratch (disjoint in time)
  int32_t *zeros = at<int32_t>(ws, L.zeros);
  uint64_t *level_bits = at<uint64_t>(ws, L.level_bits);
  const unsigned gn = cfd::grid_for(n, kThreads), gb = cfd::grid_for(g.nblocks, kThreads);
  if (hipMemcpyAsync(cur, tokens, 4 * n, hipMemcpyDeviceToDevice, st) != hipSuccess) return CF_ERR_CUDA;
  fill_u32<<<1024, kThreads, 0, st>>>(at<uint32_t>(ws, L.offsets), static_cast<size_t>(g.bits) * g.owords_max, 0u);
  fill_u32<<<1, kThreads, 0, st>>>(at<uint32_t>(ws, L.plane) + 2 * (static_cast<uint64_t>(gn) * (kThreads / 64)), 2,
                                   0u);  // the word past the last ballot (read by the last block's straddle)
  for (uint32_t lvl = 0; lvl < bits; ++lvl) {
    plane_kernel<<<gn, kThreads, 0, st>>>(cur, n, static_cast<int>(bits - 1 - lvl), plane, zflag);
    blocks_kernel<<<cfd::grid_for((g.nblocks + 7) / 8, kThreads), kThreads, 0, st>>>(
        plane, g.nblocks, at<uint32_t>(ws, L.classes) + static_cast<size_t>(lvl) * g.cwords, width, ones, offs);
    fill_u32<<<1, kThreads, 0, st>>>(at<uint32_t>(ws, L.classes) + static_cast<size_t>(lvl) * g.cwords +
                                         (g.nblocks + 7) / 8,
                                     g.cwords - (g.nblocks + 7) / 8, 0u);  // trailing class word(s)
    fill_u32<<<1, 1, 0, st>>>(width + g.nblocks, 1, 0u);
    fill_u32<<<1, 1, 0, st>>>(ones + g.nblocks, 1, 0u);
    size_t tb = 0;
    static_cast<void>(hipcub::DeviceScan::ExclusiveSum(nullptr, tb, width, obit, static_cast<int>(g.nblocks + 1), st));
    if (hipcub::DeviceScan::ExclusiveSum(at<uint8_t>(ws, L.scan_tmp), tb, width, obit,
                                         static_cast<int>(g.nblocks + 1), st) != hipSuccess ||
        hipcub::DeviceScan::ExclusiveSum(at<uint8_t>(ws, L.scan_tmp), tb, ones, ccum,
                                         static_cast<int>(g.nblocks + 1), st) != hipSuccess)
      return CF_ERR_CUDA;
    pack_kernel<<<gb, kThreads, 0, st>>>(width, obit, offs, g.nblocks,
                                         at<uint32_t>(ws, L.offsets) + static_cast<size_t>(lvl) * g.owords_max);
    samples_kernel<<<cfd::grid_for(g.nsb + 1, kThreads), kThreads, 0, st>>>(
        ccum, obit, g.nblocks, g.nsb, g.na, at<int32_t>(ws, L.rank_a) + static_cast<size_t>(lvl) * g.na,
        at<uint16_t>(ws, L.rank_d) + static_cast<size_t>(lvl) * (g.nsb + 1),
        at<int32_t>(ws, L.off_a) + static_cast<size_t>(lvl) * g.na,
        at<uint16_t>(ws, L.off_d) + static_cast<size_t>(lvl) * (g.nsb + 1));
    level_totals<<<1, 1, 0, st>>>(ccum, obit, g.nblocks, n, static_cast<int>(lvl), zeros, level_bits);
    if (lvl + 1 < bits) {
      size_t tz = 0;
      static_cast<void>(hipcub::DeviceScan::ExclusiveSum(nullptr, tz, zflag, zpos, static_cast<int>(n), st));
      if (hipcub::DeviceScan::ExclusiveSum(at<uint8_t>(ws, L.scan_tmp), tz, zflag, zpos, static_cast<int>(n), st) !=
          hipSuccess)
        return CF_ERR_CUDA;
      split_kernel<<<gn, kThreads, 0, st>>>(cur, zflag, zpos, zeros, static_cast<int>(lvl), n, nxt);
      std::swap(cur, nxt);
    }
  }
  std::vector<uint64_t> lb(bits);
  if (hipMemcpyAsync(lb.data(), level_bits, 8ull * bits, hipMemcpyDeviceToHost, st) != hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess)
    return CF_ERR_CUDA;
  cf_rrrw_layout out{};
  out.n = n;
  out.bits = bits;
  out.nblocks = g.nblocks;
  out.cwords = g.cwords;
  out.nsb = g.nsb;
  out.na = g.na;
  uint64_t ow = 0, stored = 0;
  std::vector<int32_t> offbase(bits);
  for (uint32_t l = 0; l < bits; ++l) {
    offbase[l] = static_cast<int32_t>(ow * 32);
    out.level_owords[l] = static_cast<uint32_t>((lb[l] + 31) / 32 + 2);
    ow += out.level_owords[l];
    stored += static_cast<uint64_t>(g.nblocks) * 4 + lb[l];
  }
  if (ow * 32 > 0x7FFFFFFFull) return CF_ERR_UNSUPPORTED;
  out.owords = static_cast<uint32_t>(ow);
  out.rrr_bytes = stored / 8 + (2ull * bits * g.na) * 4 + (2ull * bits * (g.nsb + 1)) * 2;
  if (hipMemcpy(at<int32_t>(ws, L.offbase), offbase.data(), 4ull * bits, hipMemcpyHostToDevice) != hipSuccess)
    return CF_ERR_CUDA;
  *layout = out;
  return cfd::launch_status();
}

extern "C" cf_status cf_rrrw_build_copy(const void *ws, const cf_rrrw_layout *layout, const cf_rrrw_arrays *out,
                                        void *stream) {
  if (!ws || !layout || !out || !out->classes || !out->offsets || !out->rank_a || !out->rank_d || !out->off_a ||
      !out->off_d || !out->offbase || !out->zeros)
    return CF_ERR_INVALID_ARGUMENT;
  const Geo g = geo_of(layout->n, layout->bits);
  const WsLayout L = ws_layout(g);
  const hipStream_t st = cfd::as_stream(stream);
  void *w = const_cast<void *>(ws);
  auto cp = [&](void *dst, size_t off, size_t bytes) {
    return hipMemcpyAsync(dst, at<uint8_t>(w, off), bytes, hipMemcpyDeviceToDevice, st) == hipSuccess;
  };
  bool ok = cp(out->classes, L.classes, 4ull * g.bits * g.cwords) && cp(out->rank_a, L.rank_a, 4ull * g.bits * g.na) &&
            cp(out->rank_d, L.rank_d, 2ull * g.bits * (g.nsb + 1)) && cp(out->off_a, L.off_a, 4ull * g.bits * g.na) &&
            cp(out->off_d, L.off_d, 2ull * g.bits * (g.nsb + 1)) && cp(out->offbase, L.offbase, 4ull * g.bits) &&
            cp(out->zeros, L.zeros, 4ull * g.bits);
  uint64_t ow = 0;
  for (uint32_t l = 0; ok && l < g.bits; ++l) {
    ok = hipMemcpyAsync(out->offsets + ow, at<uint32_t>(w, L.offsets) + static_cast<size_t>(l) * g.owords_max,
                        4ull * layout->level_owords[l], hipMemcpyDeviceToDevice, st) == hipSuccess;
    ow += layout->level_owords[l];
  }
  return ok ? cfd::launch_status() : CF_ERR_CUDA;
}

extern "C" uint64_t cf_fm_build_workspace_bytes(int32_t n, int32_t sigma) {
  if (n <= 0 || sigma <= 0) return 0;
  const size_t nw = (static_cast<size_t>(n) + 31) / 32;
  size_t scan_bytes = 0, s2 = 0;
  // temp-storage size queries: a failure leaves the size 0 and the checked scan that uses it fails
  uint32_t *const none = nullptr;
  static_cast<void>(hipcub::DeviceScan::ExclusiveSum(nullptr, scan_bytes, none, none, static_cast<int>(nw + 1)));
  static_cast<void>(hipcub::DeviceScan::ExclusiveSum(nullptr, s2, none, none, sigma));
  return align256(4 * (nw + 1)) * 2 + align256(4ull * sigma) + align256(std::max(scan_bytes, s2));
}

extern "C" cf_status cf_fm_build_aux(const int32_t *s, const int32_t *sa, int32_t n, int32_t sigma, int32_t sa_sample,
                                     uint32_t *bwt, int32_t *C, uint32_t *mwords, int32_t *msb, int32_t *sval,
                                     int32_t *sval_count, void *ws, uint64_t ws_bytes, void *stream) {
  if (!s || !sa || !bwt || !C || !mwords || !msb || !sval || !sval_count || !ws || n <= 0 || sigma <= 0 ||
      sa_sample <= 0)
    return CF_ERR_INVALID_ARGUMENT;
  if (ws_bytes < cf_fm_build_workspace_bytes(n, sigma)) return CF_ERR_INVALID_ARGUMENT;
  const hipStream_t st = cfd::as_stream(stream);
  const int nw = (n + 31) / 32, nb = (nw + 7) / 8;
  uint8_t *w = static_cast<uint8_t *>(ws);
  uint32_t *wcount = reinterpret_cast<uint32_t *>(w);
  uint32_t *wbase = reinterpret_cast<uint32_t *>(w + align256(4 * (static_cast<size_t>(nw) + 1)));
  uint8_t *tmp = w + 2 * align256(4 * (static_cast<size_t>(nw) + 1)) + align256(4ull * sigma);
  const unsigned gn = cfd::grid_for(n, kThreads);
  bwt_kernel<<<gn, kThreads, 0, st>>>(s, sa, n, bwt);
  c_table_kernel<<<gn, kThreads, 0, st>>>(s, sa, n, sigma, C);
  size_t tb = 0;
  marks_kernel<<<cfd::grid_for(nw, kThreads), kThreads, 0, st>>>(sa, n, sa_sample, mwords, wcount);
  fill_u32<<<1, 1, 0, st>>>(wcount + nw, 1, 0u);
  static_cast<void>(hipcub::DeviceScan::ExclusiveSum(nullptr, tb, wcount, wbase, nw + 1, st));
  if (hipcub::DeviceScan::ExclusiveSum(tmp, tb, wcount, wbase, nw + 1, st) != hipSuccess) return CF_ERR_CUDA;
  msb_kernel<<<cfd::grid_for(nb + 1, kThreads), kThreads, 0, st>>>(wbase, nw, nb, msb);
  sval_kernel<<<gn, kThreads, 0, st>>>(sa, n, mwords, wbase, sval);
  uint32_t total = 0;
  if (hipMemcpyAsync(&total, wbase + nw, 4, hipMemcpyDeviceToHost, st) != hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess)
    return CF_ERR_CUDA;
  *sval_count = static_cast<int32_t>(total);
  return cfd::launch_status();
}
