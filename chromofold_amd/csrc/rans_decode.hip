// rans_decode.hip — whole-tensor block-rANS value decode on gfx950 (cf_rans_decode_async).
//
// Format and decode semantics of reference src/cuda/rans.cu:11-50, bit for bit: 12-bit probabilities (M = 4096),
// 32-bit state, byte-wise renormalisation to L = 2^23 reading data[] upward from byte_off[b], one independent
// stream per block of `block` symbols (the last block may be short).
//
// gfx950 mapping: one lane per block (the state chain is serial by construction); the per-slot decode entries —
// symbol, its frequency and the slot's bias (slot - cum[symbol]) — are gathered once per workgroup into LDS, so the
// serial chain reads one LDS row per symbol instead of three dependent global loads. The renormalisation loop is
// bounded at 4 byte reads per symbol: a non-zero state reaches L within 3, so well-formed streams decode exactly as
// in the reference, and a corrupt all-zero state cannot spin forever.
#include "cf_device.hpp"
#include "chromofold/chromofold_extra.h"

namespace {

constexpr unsigned kThreads = 256;
constexpr int kProbBits = 12;
constexpr uint32_t kM = 1u << kProbBits;
constexpr uint32_t kL = 1u << 23;

__global__ void __launch_bounds__(kThreads) rans_decode_kernel(const uint8_t *__restrict__ data,
                                                               const int32_t *__restrict__ byte_off,
                                                               const uint32_t *__restrict__ state0,
                                                               const int32_t *__restrict__ slot2sym,
                                                               const int32_t *__restrict__ freq,
                                                               const int32_t *__restrict__ cum, int block, int n,
                                                               int32_t *__restrict__ out) {
  __shared__ int32_t s_sym[kM];
  __shared__ uint32_t s_freq[kM];
  __shared__ uint32_t s_bias[kM];
  for (uint32_t slot = threadIdx.x; slot < kM; slot += kThreads) {
    const int32_t s = slot2sym[slot];
    s_sym[slot] = s;
    s_freq[slot] = static_cast<uint32_t>(freq[s]);
    s_bias[slot] = static_cast<uint32_t>(static_cast<int32_t>(slot) - cum[s]);
  }
  __syncthreads();
  const int64_t b = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t base = b * block;
  if (base >= n) return;
  const int cnt = static_cast<int>(n - base < block ? n - base : block);
  int64_t pos = byte_off[b];
  uint32_t x = state0[b];
  int32_t *__restrict__ o = out + base;
  for (int j = 0; j < cnt; ++j) {
    const uint32_t slot = x & (kM - 1u);
    o[j] = s_sym[slot];
    x = s_freq[slot] * (x >> kProbBits) + s_bias[slot];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (x >= kL) break;
      x = (x << 8) | data[pos++];
    }
  }
}

}  // namespace

extern "C" cf_status cf_rans_decode_async(const uint8_t *data, const int32_t *byte_off, const uint32_t *state0,
                                          const int32_t *slot2sym, const int32_t *freq, const int32_t *cum, int block,
                                          int n, int32_t *out, void *stream) {
  if (!data || !byte_off || !state0 || !slot2sym || !freq || !cum || !out) return CF_ERR_INVALID_ARGUMENT;
  if (n == 0) return CF_OK;
  if (n < 0 || block <= 0) return CF_ERR_INVALID_ARGUMENT;
  const int64_t nblocks = (static_cast<int64_t>(n) + block - 1) / block;
  rans_decode_kernel<<<cfd::grid_for(static_cast<size_t>(nblocks), kThreads), kThreads, 0,
                       cfd::as_stream(stream)>>>(data, byte_off, state0, slot2sym, freq, cum, block, n, out);
  return cfd::launch_status();
}
