// rrr_wavelet.hip — access/rank over an RRR-compressed wavelet matrix on gfx950.
//
// Replaces reference src/cuda/rrr_wavelet.cu:25-67 and the device inlines of
// include/chromofold/detail/rrr_wavelet_device.cuh:40-149 behind the unchanged cf_rrrw_* C ABI.
//
// Design (one lane per query, 64 queries per wave):
//   * the per-superblock class scan (up to 63 four-bit classes) is done a class word at a time with SWAR
//     arithmetic: the class sum and the offset-width sum of 8 blocks cost a handful of popcounts, instead of a
//     per-block loop with a width-table load;
//   * the enumerative block decode is a single lookup in a 64 KiB compile-time unrank table (every 15-bit word
//     indexed by class and rank), replacing the reference's data-dependent Pascal-triangle walk;
//   * the class words of a superblock are fetched independently of the rank/offset samples, so each level costs
//     two dependent memory round trips (samples + classes in parallel, then the offset word and unrank entry).
// The caller's width/binom tables are part of the view for ABI compatibility; the kernels use the identical
// compile-time tables (the values are fixed by the format).
#include "chromofold/chromofold_search.h"
#include "cf_device.hpp"
#include "rrr_core.hpp"
#include "lines_core.hpp"
#include "quads_core.hpp"
#include "gather_core.hpp"
#include "chromofold/chromofold_index.h"

namespace {

template <int LEVELS>
__global__ __launch_bounds__(256) void rrrw_access_kernel(cf_rrrw_view v, const uint32_t *__restrict__ pos,
                                                          uint32_t *__restrict__ out, size_t count) {
  const size_t t = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
  if (t >= count) return;
  out[t] = cfr::access_one<LEVELS>(v, static_cast<int>(pos[t]));
}

template <int LEVELS>
__global__ __launch_bounds__(256) void rrrw_rank_kernel(cf_rrrw_view v, const uint32_t *__restrict__ sym,
                                                        const uint32_t *__restrict__ pos,
                                                        uint32_t *__restrict__ out, size_t count) {
  const size_t t = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
  if (t >= count) return;
  out[t] = cfr::rank_one<LEVELS>(v, static_cast<int>(sym[t]), static_cast<int>(pos[t]));
}

constexpr unsigned kThreads = 256;

// ---- persistent variant with the per-superblock samples and the unrank table staged in LDS
// One 1024-thread workgroup per CU copies rank_a/off_a, rank_d/off_d of every level and the 64 KiB unrank table
// (with its class starts) into LDS once, then walks its share of the queries; each rank1 then reads global memory only for the class words
// (two 16-byte loads) and the offset bits. Used when the tables fit and the batch is large enough to amortise the
// copy; results are identical to the kernels above.
constexpr unsigned kLdsThreads = 1024;

template <int LEVELS>
__global__ __launch_bounds__(kLdsThreads) void rrrw_access_lds_kernel(cf_rrrw_view v, const uint32_t *__restrict__ pos,
                                                                      uint32_t *__restrict__ out, size_t count) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const auto tb = cfr::stage_tables<true>(v, smem, kLdsThreads);
  for (size_t q = blockIdx.x * static_cast<size_t>(kLdsThreads) + threadIdx.x; q < count;
       q += static_cast<size_t>(gridDim.x) * kLdsThreads)
    out[q] = cfr::access_one_t<LEVELS, cfr::StagedTables<true>, true>(v, tb, static_cast<int>(pos[q]));
}

template <int LEVELS>
__global__ __launch_bounds__(kLdsThreads) void rrrw_rank_lds_kernel(cf_rrrw_view v, const uint32_t *__restrict__ sym,
                                                                    const uint32_t *__restrict__ pos,
                                                                    uint32_t *__restrict__ out, size_t count) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const auto tb = cfr::stage_tables<true>(v, smem, kLdsThreads);
  for (size_t q = blockIdx.x * static_cast<size_t>(kLdsThreads) + threadIdx.x; q < count;
       q += static_cast<size_t>(gridDim.x) * kLdsThreads)
    out[q] = cfr::rank_one_t<LEVELS, cfr::StagedTables<true>, true>(v, tb, static_cast<int>(sym[q]),
                                                                     static_cast<int>(pos[q]));
}

// ---- the line layout (lines_core.hpp, chromofold_index.h cf_rrrw_lines_*): access walks one record per level;
// rank(c, i) = a_L(i) + base[c] with base[c] = -e(c), one record per level instead of the RRR walk's two rank1.
// One lane per query; results equal the kernels above for every position in [0, n].
template <int LEVELS>
__global__ __launch_bounds__(kThreads) void rrrw_access_lines_kernel(cf_rrrw_view v, const uint32_t *__restrict__ lines,
                                                                     uint32_t nrec, const uint32_t *__restrict__ pos,
                                                                     uint32_t *__restrict__ out, size_t count) {
  const size_t t = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x;
  if (t >= count) return;
  const int L = LEVELS > 0 ? LEVELS : v.bits;
  uint32_t a = pos[t], val = 0;
  for (int lvl = 0; lvl < L; ++lvl) {
    int bit;
    const int r = cfl::rank1<true>(lines, nrec, lvl, a, &bit);
    val = (val << 1) | static_cast<uint32_t>(bit);
    a = bit ? static_cast<uint32_t>(v.zeros[lvl] + r) : a - static_cast<uint32_t>(r);
  }
  out[t] = val;
}

// cf_sparse_gather_fused_async over the line layout: lane = query (its access walk, one record per level), then the
// wave copies its 64 rows (gather_core.hpp).
template <int LEVELS, bool VEC>
__global__ __launch_bounds__(kThreads) void sparse_fused_lines_kernel(cf_rrrw_view v, const uint32_t *__restrict__ lines,
                                                                      uint32_t nrec, const float *__restrict__ emb,
                                                                      int dim, const uint32_t *__restrict__ pos,
                                                                      float *__restrict__ out, size_t count) {
  const size_t q0 = (blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x) & ~size_t(63);
  if (q0 >= count) return;  // wave-uniform
  const size_t t = q0 + (threadIdx.x & 63u);
  const int L = LEVELS > 0 ? LEVELS : v.bits;
  uint32_t a = t < count ? pos[t] : 0u, id = 0;
  for (int lvl = 0; lvl < L; ++lvl) {
    int bit;
    const int r = cfl::rank1<true>(lines, nrec, lvl, a, &bit);
    id = (id << 1) | static_cast<uint32_t>(bit);
    a = bit ? static_cast<uint32_t>(v.zeros[lvl] + r) : a - static_cast<uint32_t>(r);
  }
  const int nq = static_cast<int>(count - q0 < 64 ? count - q0 : 64);
  cfg::copy_rows<VEC>(id, nq, emb, static_cast<uint64_t>(dim), out, q0);
}

// Access and rank over the 4-ary layout (quads_core.hpp): L4 records per query.
template <int L4>
__global__ __launch_bounds__(kThreads) void rrrw_access_quads_kernel(const uint32_t *__restrict__ quads, uint32_t nrec,
                                                                     uint32_t nlev, const uint32_t *__restrict__ pos,
                                                                     uint32_t *__restrict__ out, size_t count) {
  const size_t t = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x;
  if (t >= count) return;
  const uint32_t L = L4 > 0 ? static_cast<uint32_t>(L4) : nlev;
  const uint32_t *Z = quads + static_cast<size_t>(L) * nrec * cfq::kRecWords;
  uint32_t a = pos[t], val = 0;
  for (uint32_t l = 0; l < L; ++l) {
    uint32_t d;
    a = cfq::step<true>(quads, nrec, Z, l, a, 0u, &d);
    val = (val << 2) | d;
  }
  out[t] = val;
}

template <int L4>
__global__ __launch_bounds__(kThreads) void rrrw_rank_quads_kernel(const uint32_t *__restrict__ quads, uint32_t nrec,
                                                                   uint32_t nlev, uint32_t mask,
                                                                   const uint32_t *__restrict__ sym,
                                                                   const uint32_t *__restrict__ pos,
                                                                   uint32_t *__restrict__ out, size_t count) {
  const size_t t = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x;
  if (t >= count) return;
  const uint32_t L = L4 > 0 ? static_cast<uint32_t>(L4) : nlev;
  const uint32_t *Z = quads + static_cast<size_t>(L) * nrec * cfq::kRecWords;
  const uint32_t c = sym[t] & mask;  // the RRR walk reads the symbol's low `bits` bits only
  uint32_t a = pos[t];
  for (uint32_t l = 0; l < L; ++l) a = cfq::step<false>(quads, nrec, Z, l, a, (c >> (2u * (L - 1u - l))) & 3u, nullptr);
  const int32_t *base = reinterpret_cast<const int32_t *>(Z + 4u * L);
  out[t] = static_cast<uint32_t>(static_cast<int32_t>(a) + base[c]);
}

// cf_sparse_gather_fused_async over the 4-ary layout: lane = query (its access walk, one record per 4-ary level),
// then the wave copies its 64 rows (gather_core.hpp).
template <int L4, bool VEC>
__global__ __launch_bounds__(kThreads) void sparse_fused_quads_kernel(const uint32_t *__restrict__ quads, uint32_t nrec,
                                                                      uint32_t nlev, const float *__restrict__ emb,
                                                                      int dim, const uint32_t *__restrict__ pos,
                                                                      float *__restrict__ out, size_t count) {
  const size_t q0 = (blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x) & ~size_t(63);
  if (q0 >= count) return;  // wave-uniform
  const size_t t = q0 + (threadIdx.x & 63u);
  const uint32_t L = L4 > 0 ? static_cast<uint32_t>(L4) : nlev;
  const uint32_t *Z = quads + static_cast<size_t>(L) * nrec * cfq::kRecWords;
  uint32_t a = t < count ? pos[t] : 0u, id = 0;
  for (uint32_t l = 0; l < L; ++l) {
    uint32_t d;
    a = cfq::step<true>(quads, nrec, Z, l, a, 0u, &d);
    id = (id << 2) | d;
  }
  const int nq = static_cast<int>(count - q0 < 64 ? count - q0 : 64);
  cfg::copy_rows<VEC>(id, nq, emb, static_cast<uint64_t>(dim), out, q0);
}

template <int LEVELS>
__global__ __launch_bounds__(kThreads) void rrrw_rank_lines_kernel(cf_rrrw_view v, const uint32_t *__restrict__ lines,
                                                                   uint32_t nrec, const uint32_t *__restrict__ sym,
                                                                   const uint32_t *__restrict__ pos,
                                                                   uint32_t *__restrict__ out, size_t count) {
  const size_t t = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x;
  if (t >= count) return;
  const int L = LEVELS > 0 ? LEVELS : v.bits;
  const uint32_t c = sym[t] & ((1u << L) - 1u);  // the RRR walk reads the symbol's low L bits only
  uint32_t a = pos[t];
  for (int lvl = 0; lvl < L; ++lvl) {
    const int r = cfl::rank1<false>(lines, nrec, lvl, a, nullptr);
    a = (c >> (L - 1 - lvl)) & 1u ? static_cast<uint32_t>(v.zeros[lvl] + r) : a - static_cast<uint32_t>(r);
  }
  const int32_t *base = reinterpret_cast<const int32_t *>(lines + static_cast<size_t>(L) * nrec * cfl::kRecWords);
  out[t] = a + static_cast<uint32_t>(base[c]);
}

}  // namespace

// Records per level of the wavelet line layout: positions up to 960 * nsb resolve (n <= 960 * nsb).
static uint32_t rrrw_nrec(const cf_rrrw_view &v) { return 2u * static_cast<uint32_t>(v.nsb) + 1u; }
constexpr int kLinesMaxBits = 24;  // the per-symbol table has 2^bits entries

extern "C" uint64_t cf_rrrw_lines_bytes(cf_rrrw_view v) {
  if (v.bits <= 0 || v.bits > kLinesMaxBits || v.nsb < 0 || v.na <= (v.nsb >> 5)) return 0;
  return (static_cast<uint64_t>(v.bits) * rrrw_nrec(v) * cfl::kRecWords + (uint64_t{1} << v.bits)) * 4u;
}

static bool rrrw_lines_ok(const cf_rrrw_view &v, const uint32_t *lines) {
  return lines && (reinterpret_cast<uintptr_t>(lines) & 15u) == 0 && v.zeros && cf_rrrw_lines_bytes(v) != 0;
}

extern "C" cf_status cf_rrrw_lines_build_async(cf_rrrw_view v, uint32_t *lines, uint64_t bytes, void *stream) {
  if (!rrrw_lines_ok(v, lines) || !v.classes || !v.offsets || !v.rank_a || !v.rank_d || !v.off_a || !v.off_d ||
      !v.offbase || v.cwords < 0)
    return CF_ERR_INVALID_ARGUMENT;
  if (bytes < cf_rrrw_lines_bytes(v)) return CF_ERR_INVALID_ARGUMENT;
  // blocks past the last real one have class nibble 0 in the zero-padded class words
  return cfl::build(v, lines, rrrw_nrec(v), 8u * static_cast<uint32_t>(v.cwords), -1, int32_t{1} << v.bits,
                    nullptr, cfd::as_stream(stream));
}

extern "C" cf_status cf_rrrw_access_lines_async(cf_rrrw_view v, const uint32_t *lines, const uint32_t *positions,
                                                uint32_t *out, size_t count, void *stream) {
  if (!rrrw_lines_ok(v, lines) || !positions || !out) return CF_ERR_INVALID_ARGUMENT;
  if (count == 0) return CF_OK;
  const hipStream_t s = cfd::as_stream(stream);
  const unsigned g = cfd::grid_for(count, kThreads);
  const uint32_t nrec = rrrw_nrec(v);
  switch (v.bits) {
    case 15: rrrw_access_lines_kernel<15><<<g, kThreads, 0, s>>>(v, lines, nrec, positions, out, count); break;
    case 16: rrrw_access_lines_kernel<16><<<g, kThreads, 0, s>>>(v, lines, nrec, positions, out, count); break;
    default: rrrw_access_lines_kernel<0><<<g, kThreads, 0, s>>>(v, lines, nrec, positions, out, count); break;
  }
  return cfd::launch_status();
}

// ---- the 4-ary layout (quads_core.hpp): n is the sequence's length (the view does not hold it)
static bool rrrw_ok(const cf_rrrw_view &v) {  // the arrays the binary access walk reads
  return v.classes && v.offsets && v.rank_a && v.rank_d && v.off_a && v.off_d && v.offbase && v.zeros;
}

static bool quads_view_ok(const cf_rrrw_view &v, uint64_t n) {
  return v.bits > 0 && v.bits <= kLinesMaxBits && v.nsb >= 0 && n < (uint64_t{1} << 31) &&
         n <= static_cast<uint64_t>(v.nsb) * 960u;
}

extern "C" uint64_t cf_rrrw_quads_bytes(cf_rrrw_view v, uint64_t n) {
  if (!quads_view_ok(v, n)) return 0;
  return cfq::layout(v.bits, n, int32_t{1} << v.bits).bytes();
}

extern "C" uint64_t cf_rrrw_quads_workspace_bytes(cf_rrrw_view v, uint64_t n) {
  if (!quads_view_ok(v, n)) return 0;
  return cfq::workspace_bytes(n, cfq::nrec_for(n));
}

extern "C" cf_status cf_rrrw_quads_build_async(cf_rrrw_view v, uint64_t n, uint32_t *quads, uint64_t bytes,
                                               void *workspace, uint64_t workspace_bytes, void *stream) {
  if (!quads_view_ok(v, n) || !quads || (reinterpret_cast<uintptr_t>(quads) & 15u) != 0 || !workspace ||
      (reinterpret_cast<uintptr_t>(workspace) & 255u) != 0 || !rrrw_ok(v))
    return CF_ERR_INVALID_ARGUMENT;
  if (bytes < cf_rrrw_quads_bytes(v, n) || workspace_bytes < cf_rrrw_quads_workspace_bytes(v, n))
    return CF_ERR_INVALID_ARGUMENT;
  return cfq::build(v, n, int32_t{1} << v.bits, nullptr, quads, workspace, cfd::as_stream(stream));
}

extern "C" cf_status cf_rrrw_access_quads_async(cf_rrrw_view v, uint64_t n, const uint32_t *quads,
                                                const uint32_t *positions, uint32_t *out, size_t count, void *stream) {
  if (!quads_view_ok(v, n) || !quads || (reinterpret_cast<uintptr_t>(quads) & 15u) != 0 || !positions || !out)
    return CF_ERR_INVALID_ARGUMENT;
  if (count == 0) return CF_OK;
  const hipStream_t s = cfd::as_stream(stream);
  const unsigned g = cfd::grid_for(count, kThreads);
  const uint32_t nrec = cfq::nrec_for(n), L4 = cfq::levels_for(v.bits);
  if (L4 == 8)
    rrrw_access_quads_kernel<8><<<g, kThreads, 0, s>>>(quads, nrec, L4, positions, out, count);
  else
    rrrw_access_quads_kernel<0><<<g, kThreads, 0, s>>>(quads, nrec, L4, positions, out, count);
  return cfd::launch_status();
}

extern "C" cf_status cf_rrrw_rank_quads_async(cf_rrrw_view v, uint64_t n, const uint32_t *quads,
                                              const uint32_t *symbols, const uint32_t *positions, uint32_t *out,
                                              size_t count, void *stream) {
  if (!quads_view_ok(v, n) || !quads || (reinterpret_cast<uintptr_t>(quads) & 15u) != 0 || !symbols || !positions ||
      !out)
    return CF_ERR_INVALID_ARGUMENT;
  if (count == 0) return CF_OK;
  const hipStream_t s = cfd::as_stream(stream);
  const unsigned g = cfd::grid_for(count, kThreads);
  const uint32_t nrec = cfq::nrec_for(n), L4 = cfq::levels_for(v.bits), mask = (1u << v.bits) - 1u;
  if (L4 == 8)
    rrrw_rank_quads_kernel<8><<<g, kThreads, 0, s>>>(quads, nrec, L4, mask, symbols, positions, out, count);
  else
    rrrw_rank_quads_kernel<0><<<g, kThreads, 0, s>>>(quads, nrec, L4, mask, symbols, positions, out, count);
  return cfd::launch_status();
}

extern "C" cf_status cf_sparse_gather_fused_quads_async(cf_rrrw_view v, uint64_t n, const uint32_t *quads,
                                                        const float *emb, int dim, const uint32_t *pos, float *out,
                                                        size_t count, void *stream) {
  if (!quads_view_ok(v, n) || !quads || (reinterpret_cast<uintptr_t>(quads) & 15u) != 0 || !emb || !pos || !out)
    return CF_ERR_INVALID_ARGUMENT;
  if (count == 0 || dim <= 0) return CF_OK;
  const hipStream_t s = cfd::as_stream(stream);
  const unsigned g = cfd::grid_for(count, kThreads);
  const uint32_t nrec = cfq::nrec_for(n), L4 = cfq::levels_for(v.bits);
  const bool vec = cfg::vec4_ok(emb, out, static_cast<uint64_t>(dim));
#define CF_FUSED(L, V) sparse_fused_quads_kernel<L, V><<<g, kThreads, 0, s>>>(quads, nrec, L4, emb, dim, pos, out, count)
  if (L4 == 8) {
    if (vec) CF_FUSED(8, true); else CF_FUSED(8, false);
  } else {
    if (vec) CF_FUSED(0, true); else CF_FUSED(0, false);
  }
#undef CF_FUSED
  return cfd::launch_status();
}

extern "C" cf_status cf_sparse_gather_fused_lines_async(cf_rrrw_view v, const uint32_t *lines, const float *emb,
                                                        int dim, const uint32_t *pos, float *out, size_t count,
                                                        void *stream) {
  if (!rrrw_lines_ok(v, lines) || !emb || !pos || !out) return CF_ERR_INVALID_ARGUMENT;
  if (count == 0 || dim <= 0) return CF_OK;
  const hipStream_t s = cfd::as_stream(stream);
  const unsigned g = cfd::grid_for(count, kThreads);
  const uint32_t nrec = rrrw_nrec(v);
  const bool vec = cfg::vec4_ok(emb, out, static_cast<uint64_t>(dim));
#define CF_FUSED(L, V) sparse_fused_lines_kernel<L, V><<<g, kThreads, 0, s>>>(v, lines, nrec, emb, dim, pos, out, count)
  switch (v.bits) {
    case 15: if (vec) CF_FUSED(15, true); else CF_FUSED(15, false); break;
    case 16: if (vec) CF_FUSED(16, true); else CF_FUSED(16, false); break;
    default: if (vec) CF_FUSED(0, true); else CF_FUSED(0, false); break;
  }
#undef CF_FUSED
  return cfd::launch_status();
}

extern "C" cf_status cf_rrrw_rank_lines_async(cf_rrrw_view v, const uint32_t *lines, const uint32_t *symbols,
                                              const uint32_t *positions, uint32_t *out, size_t count, void *stream) {
  if (!rrrw_lines_ok(v, lines) || !symbols || !positions || !out) return CF_ERR_INVALID_ARGUMENT;
  if (count == 0) return CF_OK;
  const hipStream_t s = cfd::as_stream(stream);
  const unsigned g = cfd::grid_for(count, kThreads);
  const uint32_t nrec = rrrw_nrec(v);
  switch (v.bits) {
    case 15: rrrw_rank_lines_kernel<15><<<g, kThreads, 0, s>>>(v, lines, nrec, symbols, positions, out, count); break;
    case 16: rrrw_rank_lines_kernel<16><<<g, kThreads, 0, s>>>(v, lines, nrec, symbols, positions, out, count); break;
    default: rrrw_rank_lines_kernel<0><<<g, kThreads, 0, s>>>(v, lines, nrec, symbols, positions, out, count); break;
  }
  return cfd::launch_status();
}

extern "C" cf_status cf_rrrw_access_async(cf_rrrw_view v, const uint32_t *positions, uint32_t *out, size_t count,
                                          void *stream) {
  // reference src/cuda/rrr_wavelet.cu:25-27: null classes/positions/out is rejected before any device call
  if (!v.classes || !positions || !out) return CF_ERR_INVALID_ARGUMENT;
  if (count == 0) return CF_OK;
  if (v.bits <= 0 || v.bits > 31) return CF_ERR_INVALID_ARGUMENT;
  const hipStream_t s = cfd::as_stream(stream);
  unsigned g = 0;
  if (cfr::staged_mode(v, count, kLdsThreads, g) == 2) {
    const size_t lb = cfr::stage_layout(v, true).bytes;
    if (v.bits == 15) return cfr::launch_staged(kLdsThreads, rrrw_access_lds_kernel<15>, g, lb, s, v, positions, out, count);
    if (v.bits == 16) return cfr::launch_staged(kLdsThreads, rrrw_access_lds_kernel<16>, g, lb, s, v, positions, out, count);
    return cfr::launch_staged(kLdsThreads, rrrw_access_lds_kernel<0>, g, lb, s, v, positions, out, count);
  }
  const unsigned blocks = cfd::grid_for(count, kThreads);
  switch (v.bits) {
    case 7: rrrw_access_kernel<7><<<blocks, kThreads, 0, s>>>(v, positions, out, count); break;
    case 8: rrrw_access_kernel<8><<<blocks, kThreads, 0, s>>>(v, positions, out, count); break;
    case 15: rrrw_access_kernel<15><<<blocks, kThreads, 0, s>>>(v, positions, out, count); break;
    case 16: rrrw_access_kernel<16><<<blocks, kThreads, 0, s>>>(v, positions, out, count); break;
    default: rrrw_access_kernel<0><<<blocks, kThreads, 0, s>>>(v, positions, out, count); break;
  }
  return cfd::launch_status();
}

extern "C" cf_status cf_rrrw_rank_async(cf_rrrw_view v, const uint32_t *symbols, const uint32_t *positions,
                                        uint32_t *out, size_t count, void *stream) {
  // reference src/cuda/rrr_wavelet.cu:47-50
  if (!v.classes || !symbols || !positions || !out) return CF_ERR_INVALID_ARGUMENT;
  if (count == 0) return CF_OK;
  if (v.bits <= 0 || v.bits > 31) return CF_ERR_INVALID_ARGUMENT;
  const hipStream_t s = cfd::as_stream(stream);
  unsigned g = 0;
  if (cfr::staged_mode(v, count, kLdsThreads, g) == 2) {
    const size_t lb = cfr::stage_layout(v, true).bytes;
    if (v.bits == 15) return cfr::launch_staged(kLdsThreads, rrrw_rank_lds_kernel<15>, g, lb, s, v, symbols, positions, out, count);
    if (v.bits == 16) return cfr::launch_staged(kLdsThreads, rrrw_rank_lds_kernel<16>, g, lb, s, v, symbols, positions, out, count);
    return cfr::launch_staged(kLdsThreads, rrrw_rank_lds_kernel<0>, g, lb, s, v, symbols, positions, out, count);
  }
  const unsigned blocks = cfd::grid_for(count, kThreads);
  switch (v.bits) {
    case 7: rrrw_rank_kernel<7><<<blocks, kThreads, 0, s>>>(v, symbols, positions, out, count); break;
    case 8: rrrw_rank_kernel<8><<<blocks, kThreads, 0, s>>>(v, symbols, positions, out, count); break;
    case 15: rrrw_rank_kernel<15><<<blocks, kThreads, 0, s>>>(v, symbols, positions, out, count); break;
    case 16: rrrw_rank_kernel<16><<<blocks, kThreads, 0, s>>>(v, symbols, positions, out, count); break;
    default: rrrw_rank_kernel<0><<<blocks, kThreads, 0, s>>>(v, symbols, positions, out, count); break;
  }
  return cfd::launch_status();
}
