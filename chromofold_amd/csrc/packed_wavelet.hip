// packed_wavelet.hip — packed-bitplane wavelet matrix on gfx950: batched access, rank (linear and two-level
// directory) and the fused access + embedding-row gather.
//
// Semantics (outputs bit for bit, status codes, argument checks):
//   cf_access_async                reference src/cuda/access.cu:21-47
//   cf_rank_async / cf_rank2_async reference src/cuda/rank.cu:34-52, 54-111
//   cf_embedding_gather_async      reference src/cuda/fused_embedding.cu:68-90
//   cf_embedding_gather_tpq_async  reference src/cuda/fused_embedding.cu:41-66 (same output as the fused gather)
// One lane per query for the index walks (the per-level rank1 is a short dependent chain; 64 queries per wave keep
// the memory pipeline full); the gathers then copy rows wave-cooperatively with 16-byte accesses (gather_core.hpp)
// instead of one workgroup per query.
#include "cf_device.hpp"
#include "chromofold/chromofold_extra.h"
#include "gather_core.hpp"
#include "packed_core.hpp"

namespace {

constexpr unsigned kThreads = 256;

template <int LEVELS>
__global__ void __launch_bounds__(kThreads) access_kernel(cf_wavelet_view v, const uint32_t *__restrict__ pos,
                                                          uint32_t *__restrict__ out, size_t count) {
  const size_t t = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x;
  if (t < count) out[t] = cfp::access_one<LEVELS>(v, static_cast<int>(pos[t]));
}

template <int LEVELS>
__global__ void __launch_bounds__(kThreads) rank_kernel(cf_wavelet_view v, const uint32_t *__restrict__ sym,
                                                        const uint32_t *__restrict__ pos, uint32_t *__restrict__ out,
                                                        size_t count) {
  const size_t t = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x;
  if (t < count) out[t] = cfp::rank_one<LEVELS>(v, static_cast<int>(sym[t]), static_cast<int>(pos[t]));
}

// two-level directory: coarse i32 sample every CB words + u16 within-sample prefix per word (+1 sentinel per level)
struct Rank2 {
  const int32_t *coarse;
  const uint16_t *fine;
  int ncoarse, cb;
};

__device__ __forceinline__ int rank1_2level(const uint32_t *__restrict__ w, const int32_t *__restrict__ coarse,
                                            const uint16_t *__restrict__ fine, int cb, int pos) {
  const int word = pos >> 5, bit = pos & 31;
  int r = coarse[word / cb] + static_cast<int>(fine[word]);
  if (bit) r += __popc(w[word] & ((1u << bit) - 1u));
  return r;
}

template <int LEVELS>
__global__ void __launch_bounds__(kThreads) rank2_kernel(cf_wavelet_view v, Rank2 d, const uint32_t *__restrict__ sym,
                                                         const uint32_t *__restrict__ pos, uint32_t *__restrict__ out,
                                                         size_t count) {
  const size_t t = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x;
  if (t >= count) return;
  const int L = LEVELS > 0 ? LEVELS : static_cast<int>(v.levels);
  const int c = static_cast<int>(sym[t]);
  int p = 0, q = static_cast<int>(pos[t]);
  for (int lvl = 0; lvl < L; ++lvl) {
    const uint32_t *w = v.bitplanes + static_cast<size_t>(lvl) * v.nwords;
    const int32_t *co = d.coarse + static_cast<size_t>(lvl) * d.ncoarse;
    const uint16_t *fi = d.fine + static_cast<size_t>(lvl) * (v.nwords + 1);
    const int rp = rank1_2level(w, co, fi, d.cb, p), rq = rank1_2level(w, co, fi, d.cb, q);
    if ((c >> (L - 1 - lvl)) & 1) {
      p = v.zero_counts[lvl] + rp;
      q = v.zero_counts[lvl] + rq;
    } else {
      p -= rp;
      q -= rq;
    }
  }
  out[t] = static_cast<uint32_t>(q - p);
}

// 64 queries per wave: lane = query for the access walk, then all lanes copy the 64 rows
template <int LEVELS, bool VEC>
__global__ void __launch_bounds__(kThreads) gather_kernel(cf_wavelet_view v, const float *__restrict__ emb,
                                                          uint32_t dim, const uint32_t *__restrict__ pos,
                                                          float *__restrict__ out, size_t count) {
  const size_t q0 = (blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x) & ~size_t(63);
  if (q0 >= count) return;  // wave-uniform
  const size_t t = q0 + (threadIdx.x & 63u);
  const uint32_t id = t < count ? cfp::access_one<LEVELS>(v, static_cast<int>(pos[t])) : 0u;
  const int nq = static_cast<int>(count - q0 < 64 ? count - q0 : 64);
  cfg::copy_rows<VEC>(id, nq, emb, dim, out, q0);
}

// level-count specialisations of the reference (2, 4, 8, 15, 16, 17) plus the dynamic fallback (LEVELS = 0)
#define CF_LEVEL_SWITCH(levels, LAUNCH) \
  switch (levels) {                     \
    case 2: LAUNCH(2); break;           \
    case 4: LAUNCH(4); break;           \
    case 8: LAUNCH(8); break;           \
    case 15: LAUNCH(15); break;         \
    case 16: LAUNCH(16); break;         \
    case 17: LAUNCH(17); break;         \
    default: LAUNCH(0); break;          \
  }

}  // namespace

extern "C" cf_status cf_access_async(cf_wavelet_view v, const uint32_t *pos, uint32_t *out, size_t count,
                                     void *stream) {
  if (!v.bitplanes || !v.superblocks || !v.zero_counts || !pos || !out) return CF_ERR_INVALID_ARGUMENT;
  if (count == 0) return CF_OK;
  const hipStream_t st = cfd::as_stream(stream);
  const unsigned blocks = cfd::grid_for(count, kThreads);
#define L_(N) access_kernel<N><<<blocks, kThreads, 0, st>>>(v, pos, out, count)
  CF_LEVEL_SWITCH(v.levels, L_)
#undef L_
  return cfd::launch_status();
}

extern "C" cf_status cf_rank_async(cf_wavelet_view v, const uint32_t *sym, const uint32_t *pos, uint32_t *out,
                                   size_t count, void *stream) {
  if (!v.bitplanes || !sym || !pos || !out) return CF_ERR_INVALID_ARGUMENT;
  if (count == 0) return CF_OK;
  if (!v.superblocks || !v.zero_counts) return CF_ERR_INVALID_ARGUMENT;
  const hipStream_t st = cfd::as_stream(stream);
  const unsigned blocks = cfd::grid_for(count, kThreads);
#define L_(N) rank_kernel<N><<<blocks, kThreads, 0, st>>>(v, sym, pos, out, count)
  CF_LEVEL_SWITCH(v.levels, L_)
#undef L_
  return cfd::launch_status();
}

extern "C" cf_status cf_rank2_async(cf_wavelet_view v, const int32_t *coarse, const uint16_t *fine, int ncoarse,
                                    int CB, const uint32_t *sym, const uint32_t *pos, uint32_t *out, size_t count,
                                    void *stream) {
  if (count == 0) return CF_OK;
  if (!v.bitplanes || !v.zero_counts || !coarse || !fine || !sym || !pos || !out || CB <= 0 || ncoarse < 0)
    return CF_ERR_INVALID_ARGUMENT;
  const hipStream_t st = cfd::as_stream(stream);
  const unsigned blocks = cfd::grid_for(count, kThreads);
  const Rank2 d{coarse, fine, ncoarse, CB};
#define L_(N) rank2_kernel<N><<<blocks, kThreads, 0, st>>>(v, d, sym, pos, out, count)
  CF_LEVEL_SWITCH(v.levels, L_)
#undef L_
  return cfd::launch_status();
}

namespace {
cf_status launch_gather(cf_wavelet_view v, const float *emb, uint32_t dim, const uint32_t *pos, float *out,
                        size_t count, void *stream) {
  const hipStream_t st = cfd::as_stream(stream);
  const unsigned blocks = cfd::grid_for(count, kThreads);
  if (cfg::vec4_ok(emb, out, dim)) {
#define L_(N) gather_kernel<N, true><<<blocks, kThreads, 0, st>>>(v, emb, dim, pos, out, count)
    CF_LEVEL_SWITCH(v.levels, L_)
#undef L_
  } else {
#define L_(N) gather_kernel<N, false><<<blocks, kThreads, 0, st>>>(v, emb, dim, pos, out, count)
    CF_LEVEL_SWITCH(v.levels, L_)
#undef L_
  }
  return cfd::launch_status();
}
}  // namespace

extern "C" cf_status cf_embedding_gather_async(cf_wavelet_view v, const float *emb, uint32_t dim,
                                               const uint32_t *pos, float *out, size_t count, void *stream) {
  if (!v.bitplanes || !emb || !pos || !out) return CF_ERR_INVALID_ARGUMENT;
  if (count == 0 || dim == 0) return CF_OK;
  if (!v.superblocks || !v.zero_counts) return CF_ERR_INVALID_ARGUMENT;
  return launch_gather(v, emb, dim, pos, out, count, stream);
}

extern "C" cf_status cf_embedding_gather_tpq_async(cf_wavelet_view v, const float *emb, uint32_t dim,
                                                   const uint32_t *pos, float *out, size_t count, void *stream) {
  if (count == 0 || dim == 0) return CF_OK;
  if (!v.bitplanes || !v.superblocks || !v.zero_counts || !emb || !pos || !out) return CF_ERR_INVALID_ARGUMENT;
  return launch_gather(v, emb, dim, pos, out, count, stream);
}
