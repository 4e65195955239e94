// delta_fetch.hip — delta-cluster fetch on gfx950.
//
// Result for query t (semantics of reference src/cuda/delta_apply.cu:12-43): the leaf's own delta value when the
// leaf's sorted delta positions contain pos, else the shared base value base[pos], or -1 past the base. With
// repeated positions the first one's value wins (the lowest index holding pos).
//
// Design: one lane per query. The lookup in the leaf's sorted positions is a 4-way search: each round loads the
// three pivots that cut the remaining range into quarters together (three loads in flight per lane instead of one
// dependent load per halving), counts the pivots below pos and keeps that quarter; at most three entries remain for
// a final scan. For a leaf of n deltas that is about log4(n) load rounds: 3 for 64 deltas, where a halving search
// makes 6 dependent trips to memory. The base load is issued before the search so that it overlaps it.
#include "cf_device.hpp"
#include "chromofold/chromofold_extra.h"

namespace {

constexpr unsigned kThreads = 256;

// First index i in [0, n) with p[i] >= pos, or n when every entry is below pos (p sorted ascending).
__device__ __forceinline__ int lower_bound_4way(const int32_t *__restrict__ p, int n, int pos) {
  int lo = 0, len = n;
  while (len > 3) {
    const int q = len >> 2;  // quarters [lo, lo+q), [lo+q, lo+2q), [lo+2q, lo+3q), [lo+3q, lo+len)
    const int32_t a = p[lo + q - 1], b = p[lo + 2 * q - 1], c = p[lo + 3 * q - 1];
    const int below = (a < pos) + (b < pos) + (c < pos);  // pivots are sorted, so this picks the quarter
    lo += below * q;
    len = below == 3 ? len - 3 * q : q;
  }
  for (; len > 0 && p[lo] < pos; --len) ++lo;
  return lo;
}

__global__ void __launch_bounds__(kThreads) delta_fetch_kernel(const int32_t *__restrict__ base, int nbase,
                                                               const int32_t *__restrict__ dpos,
                                                               const int32_t *__restrict__ dval,
                                                               const int32_t *__restrict__ dstart,
                                                               const int32_t *__restrict__ dlen,
                                                               const int32_t *__restrict__ leaf,
                                                               const int32_t *__restrict__ pos,
                                                               int32_t *__restrict__ out, size_t count) {
  const size_t q = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x;
  if (q >= count) return;
  const int32_t lf = leaf[q], p = pos[q];
  // a negative position is treated like one past the base (the reference would read before the array)
  const int32_t shared = (p >= 0 && p < nbase) ? base[p] : -1;
  const int32_t first = dstart[lf], n = dlen[lf];
  const int32_t *run = dpos + first;
  const int i = lower_bound_4way(run, n, p);
  out[q] = (i < n && run[i] == p) ? dval[first + i] : shared;
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
