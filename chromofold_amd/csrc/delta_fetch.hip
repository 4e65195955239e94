// delta_fetch.hip — delta-cluster fetch on gfx950: value at (leaf, pos) = base[pos] (or -1 past the shared base),
// overridden by the leaf's own delta when its sorted delta positions hold pos. Semantics of reference
// src/cuda/delta_apply.cu:12-43, bit for bit. One lane per query; the binary search over a leaf's deltas is a
// short dependent chain, so 64 independent queries per wave hide its latency.
#include "cf_device.hpp"
#include "chromofold/chromofold_extra.h"

namespace {

constexpr unsigned kThreads = 256;

__global__ void __launch_bounds__(kThreads) delta_fetch_kernel(const int32_t *__restrict__ base, int nbase,
                                                               const int32_t *__restrict__ dpos,
                                                               const int32_t *__restrict__ dval,
                                                               const int32_t *__restrict__ dstart,
                                                               const int32_t *__restrict__ dlen,
                                                               const int32_t *__restrict__ leaf_in,
                                                               const int32_t *__restrict__ pos_in,
                                                               int32_t *__restrict__ out, size_t count) {
  const size_t t = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x;
  if (t >= count) return;
  const int leaf = leaf_in[t], pos = pos_in[t];
  int res = (pos < nbase) ? base[pos] : -1;
  const int ds = dstart[leaf], dl = dlen[leaf];
  int lo = 0, hi = dl;  // first delta position >= pos
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (dpos[ds + mid] < pos)
      lo = mid + 1;
    else
      hi = mid;
  }
  if (lo < dl && dpos[ds + lo] == pos) res = dval[ds + lo];
  out[t] = res;
}

}  // namespace

extern "C" cf_status cf_delta_fetch_async(const int32_t *base, int nbase, const int32_t *dpos, const int32_t *dval,
                                          const int32_t *dstart, const int32_t *dlen, const int32_t *leaf,
                                          const int32_t *pos, int32_t *out, size_t count, void *stream) {
  if (!base || !dstart || !dlen || !leaf || !pos || !out) return CF_ERR_INVALID_ARGUMENT;
  if (count == 0) return CF_OK;
  delta_fetch_kernel<<<cfd::grid_for(count, kThreads), kThreads, 0, cfd::as_stream(stream)>>>(
      base, nbase, dpos, dval, dstart, dlen, leaf, pos, out, count);
  return cfd::launch_status();
}
