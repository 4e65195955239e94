// rrr_gather.hip — single RRR bitvector rank1 and the RRR-wavelet sparse consumers on gfx950.
//
//   cf_rrr_rank_async            reference src/cuda/rrr.cu:59-85
//   cf_sparse_gather_fused_async reference src/cuda/sparse_gather.cu:55-66 (access + embedding-row gather, fused)
//   cf_sparse_decode_all_async   reference src/cuda/sparse_gather.cu:68-79 (every token id, the materialised path)
//   cf_sparse_gather_async       reference src/cuda/sparse_gather.cu:81-91 (gather through decoded ids)
// Outputs are bit-identical to the reference. The binomial/width tables the reference reads from caller memory are
// fixed by the RRR format (T = 15) and compiled into the code object here, so those two arguments are accepted for
// signature compatibility and not read. Row copies are wave-cooperative (gather_core.hpp).
#include "cf_device.hpp"
#include "chromofold/chromofold_extra.h"
#include "gather_core.hpp"
#include "rrr_core.hpp"

namespace {

constexpr unsigned kThreads = 256;

__global__ void __launch_bounds__(kThreads) rrr_rank_kernel(const uint32_t *__restrict__ cls,
                                                            const uint32_t *__restrict__ offsets,
                                                            const int32_t *__restrict__ sbrank,
                                                            const int32_t *__restrict__ sboff,
                                                            const uint32_t *__restrict__ pos, uint32_t *__restrict__ out,
                                                            size_t count) {
  const size_t t = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x;
  if (t < count) out[t] = static_cast<uint32_t>(cfr::rank1_plain(cls, offsets, sbrank, sboff, static_cast<int>(pos[t])));
}

template <int LEVELS, bool VEC>
__global__ void __launch_bounds__(kThreads) sparse_fused_kernel(cf_rrrw_view v, const float *__restrict__ emb, int dim,
                                                                const uint32_t *__restrict__ pos,
                                                                float *__restrict__ out, size_t count) {
  const size_t q0 = (blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x) & ~size_t(63);
  if (q0 >= count) return;  // wave-uniform
  const size_t t = q0 + (threadIdx.x & 63u);
  const uint32_t id = t < count ? cfr::access_one<LEVELS>(v, static_cast<int>(pos[t])) : 0u;
  const int nq = static_cast<int>(count - q0 < 64 ? count - q0 : 64);
  cfg::copy_rows<VEC>(id, nq, emb, static_cast<uint64_t>(dim), out, q0);
}

template <int LEVELS>
__global__ void __launch_bounds__(kThreads) decode_all_kernel(cf_rrrw_view v, uint32_t *__restrict__ ids, size_t n) {
  const size_t t = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x;
  if (t < n) ids[t] = cfr::access_one<LEVELS>(v, static_cast<int>(t));
}

template <bool VEC>
__global__ void __launch_bounds__(kThreads) id_gather_kernel(const uint32_t *__restrict__ ids,
                                                             const float *__restrict__ emb, int dim,
                                                             const uint32_t *__restrict__ pos,
                                                             float *__restrict__ out, size_t count) {
  const size_t q0 = (blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x) & ~size_t(63);
  if (q0 >= count) return;
  const size_t t = q0 + (threadIdx.x & 63u);
  const uint32_t id = t < count ? ids[pos[t]] : 0u;
  const int nq = static_cast<int>(count - q0 < 64 ? count - q0 : 64);
  cfg::copy_rows<VEC>(id, nq, emb, static_cast<uint64_t>(dim), out, q0);
}

// level-count specialisations of the reference's sparse kernels (2, 4, 6, 7, 8, 16, 17) plus the dynamic walk
#define CF_BITS_SWITCH(bits, LAUNCH) \
  switch (bits) {                    \
    case 2: LAUNCH(2); break;        \
    case 4: LAUNCH(4); break;        \
    case 6: LAUNCH(6); break;        \
    case 7: LAUNCH(7); break;        \
    case 8: LAUNCH(8); break;        \
    case 15: LAUNCH(15); break;      \
    case 16: LAUNCH(16); break;      \
    case 17: LAUNCH(17); break;      \
    default: LAUNCH(0); break;       \
  }

bool rrrw_ok(const cf_rrrw_view &v) {
  return v.classes && v.offsets && v.rank_a && v.rank_d && v.off_a && v.off_d && v.offbase && v.zeros;
}

}  // namespace

extern "C" cf_status cf_rrr_rank_async(const uint32_t *classes, const uint32_t *offsets, const int32_t *sbrank,
                                       const int32_t *sboff, const int * /*width*/, const int * /*binom*/,
                                       const uint32_t *positions, uint32_t *out, size_t count, void *stream) {
  if (!classes || !offsets || !positions || !out) return CF_ERR_INVALID_ARGUMENT;
  if (count == 0) return CF_OK;
  if (!sbrank || !sboff) return CF_ERR_INVALID_ARGUMENT;
  rrr_rank_kernel<<<cfd::grid_for(count, kThreads), kThreads, 0, cfd::as_stream(stream)>>>(
      classes, offsets, sbrank, sboff, positions, out, count);
  return cfd::launch_status();
}

extern "C" cf_status cf_sparse_gather_fused_async(cf_rrrw_view v, const float *emb, int dim, const uint32_t *pos,
                                                  float *out, size_t K, void *stream) {
  if (!v.classes || !emb || !pos || !out) return CF_ERR_INVALID_ARGUMENT;
  if (K == 0 || dim <= 0) return CF_OK;
  if (!rrrw_ok(v)) return CF_ERR_INVALID_ARGUMENT;
  const hipStream_t st = cfd::as_stream(stream);
  const unsigned blocks = cfd::grid_for(K, kThreads);
  if (cfg::vec4_ok(emb, out, static_cast<uint64_t>(dim))) {
#define L_(N) sparse_fused_kernel<N, true><<<blocks, kThreads, 0, st>>>(v, emb, dim, pos, out, K)
    CF_BITS_SWITCH(v.bits, L_)
#undef L_
  } else {
#define L_(N) sparse_fused_kernel<N, false><<<blocks, kThreads, 0, st>>>(v, emb, dim, pos, out, K)
    CF_BITS_SWITCH(v.bits, L_)
#undef L_
  }
  return cfd::launch_status();
}

extern "C" cf_status cf_sparse_decode_all_async(cf_rrrw_view v, uint32_t *ids, size_t n, void *stream) {
  if (!v.classes || !ids) return CF_ERR_INVALID_ARGUMENT;
  if (n == 0) return CF_OK;
  if (!rrrw_ok(v)) return CF_ERR_INVALID_ARGUMENT;
  const hipStream_t st = cfd::as_stream(stream);
  const unsigned blocks = cfd::grid_for(n, kThreads);
#define L_(N) decode_all_kernel<N><<<blocks, kThreads, 0, st>>>(v, ids, n)
  CF_BITS_SWITCH(v.bits, L_)
#undef L_
  return cfd::launch_status();
}

extern "C" cf_status cf_sparse_gather_async(const uint32_t *ids, const float *emb, int dim, const uint32_t *pos,
                                            float *out, size_t K, void *stream) {
  if (!ids || !emb || !pos || !out) return CF_ERR_INVALID_ARGUMENT;
  if (K == 0 || dim <= 0) return CF_OK;
  const hipStream_t st = cfd::as_stream(stream);
  const unsigned blocks = cfd::grid_for(K, kThreads);
  if (cfg::vec4_ok(emb, out, static_cast<uint64_t>(dim)))
    id_gather_kernel<true><<<blocks, kThreads, 0, st>>>(ids, emb, dim, pos, out, K);
  else
    id_gather_kernel<false><<<blocks, kThreads, 0, st>>>(ids, emb, dim, pos, out, K);
  return cfd::launch_status();
}
