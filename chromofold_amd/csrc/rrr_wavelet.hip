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
constexpr size_t kLdsLimit = 160 * 1024;

struct LdsLayout {
  size_t unrank, base, rank_d, off_d, rank_a, off_a, bytes;
};

__host__ __device__ inline size_t align16(size_t x) { return (x + 15) & ~static_cast<size_t>(15); }

__host__ __device__ inline LdsLayout lds_layout(const cf_rrrw_view &v) {
  LdsLayout l{};
  const size_t nd = static_cast<size_t>(v.bits) * (v.nsb + 1), na = static_cast<size_t>(v.bits) * v.na;
  l.unrank = 0;
  l.base = align16(sizeof(cfd::RrrTables::unrank));
  l.rank_d = l.base + align16(sizeof(cfd::RrrTables::base));
  l.off_d = l.rank_d + align16(nd * 2);
  l.rank_a = l.off_d + align16(nd * 2);
  l.off_a = l.rank_a + align16(na * 4);
  l.bytes = l.off_a + align16(na * 4);
  return l;
}

__device__ cfr::LdsTables stage_tables(const cf_rrrw_view &v, uint8_t *smem) {
  const LdsLayout l = lds_layout(v);
  const int t = threadIdx.x;
  {  // unrank table: 16-byte copies
    const uint4 *src = reinterpret_cast<const uint4 *>(cfr::kTab.unrank);
    uint4 *dst = reinterpret_cast<uint4 *>(smem + l.unrank);
    for (size_t i = t; i < sizeof(cfd::RrrTables::unrank) / 16; i += kLdsThreads) dst[i] = src[i];
  }
  int32_t *bs = reinterpret_cast<int32_t *>(smem + l.base);
  if (t < 17) bs[t] = cfr::kTab.base[t];
  const size_t nd = static_cast<size_t>(v.bits) * (v.nsb + 1), na = static_cast<size_t>(v.bits) * v.na;
  uint16_t *rd = reinterpret_cast<uint16_t *>(smem + l.rank_d), *od = reinterpret_cast<uint16_t *>(smem + l.off_d);
  int32_t *ra = reinterpret_cast<int32_t *>(smem + l.rank_a), *oa = reinterpret_cast<int32_t *>(smem + l.off_a);
  for (size_t i = t; i < nd; i += kLdsThreads) {
    rd[i] = v.rank_d[i];
    od[i] = v.off_d[i];
  }
  for (size_t i = t; i < na; i += kLdsThreads) {
    ra[i] = v.rank_a[i];
    oa[i] = v.off_a[i];
  }
  __syncthreads();
  return cfr::LdsTables{ra, oa, rd, od, reinterpret_cast<const uint16_t *>(smem + l.unrank), bs};
}

template <int LEVELS>
__global__ __launch_bounds__(kLdsThreads) void rrrw_access_lds_kernel(cf_rrrw_view v, const uint32_t *__restrict__ pos,
                                                                      uint32_t *__restrict__ out, size_t count) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const cfr::LdsTables tb = stage_tables(v, smem);
  for (size_t q = blockIdx.x * static_cast<size_t>(kLdsThreads) + threadIdx.x; q < count;
       q += static_cast<size_t>(gridDim.x) * kLdsThreads)
    out[q] = cfr::access_one_t<LEVELS, cfr::LdsTables, true>(v, tb, static_cast<int>(pos[q]));
}

template <int LEVELS>
__global__ __launch_bounds__(kLdsThreads) void rrrw_rank_lds_kernel(cf_rrrw_view v, const uint32_t *__restrict__ sym,
                                                                    const uint32_t *__restrict__ pos,
                                                                    uint32_t *__restrict__ out, size_t count) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const cfr::LdsTables tb = stage_tables(v, smem);
  for (size_t q = blockIdx.x * static_cast<size_t>(kLdsThreads) + threadIdx.x; q < count;
       q += static_cast<size_t>(gridDim.x) * kLdsThreads)
    out[q] = cfr::rank_one_t<LEVELS, cfr::LdsTables, true>(v, tb, static_cast<int>(sym[q]), static_cast<int>(pos[q]));
}

// Workgroups for the persistent kernels (one per CU), or 0 when the LDS path does not apply: the tables must fit and
// the batch must give every lane of the grid at least one query (each workgroup copies ~135 KB first).
unsigned lds_grid(const cf_rrrw_view &v, size_t count) {
  static int cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) !=
                                                 hipSuccess)
      return 0;
    return n;
  }();
  if (cus <= 0 || v.bits <= 0 || v.nsb < 0 || v.na < 0 || lds_layout(v).bytes > kLdsLimit) return 0;
  if (count < static_cast<size_t>(cus) * kLdsThreads) return 0;
  return static_cast<unsigned>(cus);
}

template <class K>
cf_status launch_lds(K kernel, unsigned grid, size_t bytes, hipStream_t s, const auto &...args) {
  if (hipFuncSetAttribute(reinterpret_cast<const void *>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          static_cast<int>(bytes)) != hipSuccess)
    return CF_ERR_CUDA;
  kernel<<<grid, kLdsThreads, bytes, s>>>(args...);
  return cfd::launch_status();
}

}  // namespace

extern "C" cf_status cf_rrrw_access_async(cf_rrrw_view v, const uint32_t *positions, uint32_t *out, size_t count,
                                          void *stream) {
  // reference src/cuda/rrr_wavelet.cu:25-27: null classes/positions/out is rejected before any device call
  if (!v.classes || !positions || !out) return CF_ERR_INVALID_ARGUMENT;
  if (count == 0) return CF_OK;
  if (v.bits <= 0 || v.bits > 31) return CF_ERR_INVALID_ARGUMENT;
  const hipStream_t s = cfd::as_stream(stream);
  if (const unsigned g = lds_grid(v, count)) {
    const size_t lb = lds_layout(v).bytes;
    if (v.bits == 15) return launch_lds(rrrw_access_lds_kernel<15>, g, lb, s, v, positions, out, count);
    if (v.bits == 16) return launch_lds(rrrw_access_lds_kernel<16>, g, lb, s, v, positions, out, count);
    return launch_lds(rrrw_access_lds_kernel<0>, g, lb, s, v, positions, out, count);
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
  if (const unsigned g = lds_grid(v, count)) {
    const size_t lb = lds_layout(v).bytes;
    if (v.bits == 15) return launch_lds(rrrw_rank_lds_kernel<15>, g, lb, s, v, symbols, positions, out, count);
    if (v.bits == 16) return launch_lds(rrrw_rank_lds_kernel<16>, g, lb, s, v, symbols, positions, out, count);
    return launch_lds(rrrw_rank_lds_kernel<0>, g, lb, s, v, symbols, positions, out, count);
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
