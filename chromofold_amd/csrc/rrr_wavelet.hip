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

}  // namespace

extern "C" cf_status cf_rrrw_access_async(cf_rrrw_view v, const uint32_t *positions, uint32_t *out, size_t count,
                                          void *stream) {
  // reference src/cuda/rrr_wavelet.cu:25-27: null classes/positions/out is rejected before any device call
  if (!v.classes || !positions || !out) return CF_ERR_INVALID_ARGUMENT;
  if (count == 0) return CF_OK;
  if (v.bits <= 0 || v.bits > 31) return CF_ERR_INVALID_ARGUMENT;
  const hipStream_t s = cfd::as_stream(stream);
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
