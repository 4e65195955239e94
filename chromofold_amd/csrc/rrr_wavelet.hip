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

}  // namespace

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
