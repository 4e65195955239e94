// stream_read.hip — read-only HBM streaming kernel (chromofold_measure.h): the achievable read bandwidth of the
// device (16-byte non-temporal loads, coalesced, each byte read once).
//
// One workgroup per 64 KiB chunk, read front to back with four 16-byte loads in flight per lane. Per-workgroup
// contiguous chunks reach ~7.1 TB/s on MI355X where a grid-stride walk over the whole buffer (a few workgroups per
// CU, their loads 4 KiB apart at any moment) stays near 6.0 TB/s, and non-temporal loads add ~12 % over ordinary
// ones. The data is folded into one XOR per workgroup, which is stored to the sink only when it equals kKey: the
// loads cannot be removed, and no workgroup waits on an atomic to one address (one atomic per workgroup cost 40 %
// of the rate at this grid size).
#include "cf_device.hpp"
#include "chromofold/chromofold_measure.h"

namespace {

constexpr int kThreads = 256;
constexpr uint64_t kChunk16 = 4096;  // 16-byte units per chunk (64 KiB)
constexpr uint32_t kKey = CF_MEASURE_FOLD_KEY;  // a workgroup fold equal to this is stored (keeps the loads alive)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// The workgroup's XOR of `acc`, stored to *sink if it equals kKey.
__device__ void fold_out(uint32_t acc, uint32_t *sink) {
  __shared__ uint32_t s_acc;
  if (threadIdx.x == 0) s_acc = 0;
  __syncthreads();
  atomicXor(&s_acc, acc);
  __syncthreads();
  if (threadIdx.x == 0 && s_acc == kKey) *sink = s_acc;
}

__global__ void __launch_bounds__(kThreads) stream_read_kernel(const u32x4 *__restrict__ src, uint64_t n16,
                                                               uint32_t *__restrict__ sink) {
  const uint64_t chunks = (n16 + kChunk16 - 1) / kChunk16;
  uint32_t acc = 0;
  for (uint64_t c = blockIdx.x; c < chunks; c += gridDim.x) {
    const uint64_t hi = min((c + 1) * kChunk16, n16);
    uint64_t i = c * kChunk16 + threadIdx.x;
    for (; i + 3 * kThreads < hi; i += 4 * kThreads) {
      const u32x4 a = __builtin_nontemporal_load(src + i), b = __builtin_nontemporal_load(src + i + kThreads);
      const u32x4 e = __builtin_nontemporal_load(src + i + 2 * kThreads);
      const u32x4 f = __builtin_nontemporal_load(src + i + 3 * kThreads);
      acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ e.x ^ e.y ^ e.z ^ e.w ^ f.x ^ f.y ^ f.z ^ f.w;
    }
    for (; i < hi; i += kThreads) {
      const u32x4 a = __builtin_nontemporal_load(src + i);
      acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
  }
  fold_out(acc, sink);
}

// Cached re-reads: `passes` passes over n16 16-byte units with ordinary loads. Pass p gives workgroup b the chunk of
// workgroup (b + 8 p) mod gridDim.x — same XCD under round-robin dispatch (so its L2 holds it after the first pass),
// a different CU (so the CU's own L1 does not).
__global__ void __launch_bounds__(kThreads) cache_read_kernel(const u32x4 *__restrict__ src, uint64_t n16,
                                                              uint32_t passes, uint32_t *__restrict__ sink) {
  const uint64_t chunk = (n16 + gridDim.x - 1) / gridDim.x;
  uint32_t acc = 0;
  for (uint32_t p = 0; p < passes; ++p) {
    const uint64_t b = (blockIdx.x + 8ull * p) % gridDim.x;
    const uint64_t lo = b * chunk, hi = lo + chunk < n16 ? lo + chunk : n16;
    uint64_t i = lo + threadIdx.x;
    for (; i + 3 * kThreads < hi; i += 4 * kThreads) {
      const u32x4 a = src[i], c = src[i + kThreads], e = src[i + 2 * kThreads], f = src[i + 3 * kThreads];
      acc ^= a.x ^ a.y ^ a.z ^ a.w ^ c.x ^ c.y ^ c.z ^ c.w ^ e.x ^ e.y ^ e.z ^ e.w ^ f.x ^ f.y ^ f.z ^ f.w;
    }
    for (; i < hi; i += kThreads) {
      const u32x4 a = src[i];
      acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
  }
  fold_out(acc, sink);
}

// LDS reads: each workgroup fills 64 KiB of LDS, then reads it `passes` times with 16-byte ds_read (lane i of a
// wavefront at 16 i + 1 KiB steps: every bank busy, no conflicts).
constexpr int kLdsBytes = 64 * 1024;
__global__ void __launch_bounds__(kThreads) lds_read_kernel(uint32_t passes, uint32_t *__restrict__ sink) {
  __shared__ u32x4 s_buf[kLdsBytes / 16];
  for (int i = threadIdx.x; i < kLdsBytes / 16; i += kThreads)
    s_buf[i] = u32x4{static_cast<uint32_t>(i), static_cast<uint32_t>(i) * 3u, blockIdx.x, 7u};
  __syncthreads();
  uint32_t acc = 0;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (uint32_t p = 0; p < passes; ++p) {
#pragma unroll 8
    for (int k = 0; k < kLdsBytes / 16 / 64; k += 4) {  // 4 waves cover 4 KiB per step
      const u32x4 a = s_buf[((k + wave) * 64 + lane) % (kLdsBytes / 16)];
      acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    acc = (acc << 1) | (acc >> 31);  // keeps each pass's loads alive
  }
  fold_out(acc, sink);
}

int device_cus() {
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  return cus;
}

}  // namespace

extern "C" cf_status cf_cache_read_async(const void *src, uint64_t bytes, uint32_t passes, uint32_t *sink,
                                         void *stream) {
  if (!src || !sink || bytes % 16 != 0 || reinterpret_cast<uintptr_t>(src) % 16 != 0 || passes == 0)
    return CF_ERR_INVALID_ARGUMENT;
  if (bytes == 0) return CF_OK;
  const unsigned blocks = static_cast<unsigned>(8 * device_cus());
  cache_read_kernel<<<blocks, kThreads, 0, cfd::as_stream(stream)>>>(static_cast<const u32x4 *>(src), bytes / 16,
                                                                    passes, sink);
  return cfd::launch_status();
}

extern "C" cf_status cf_lds_read_async(uint32_t passes, uint32_t *sink, void *stream) {
  if (!sink || passes == 0) return CF_ERR_INVALID_ARGUMENT;
  const unsigned blocks = static_cast<unsigned>(2 * device_cus());
  lds_read_kernel<<<blocks, kThreads, 0, cfd::as_stream(stream)>>>(passes, sink);
  return cfd::launch_status();
}

extern "C" uint64_t cf_lds_read_bytes(uint32_t passes) {
  return static_cast<uint64_t>(2 * device_cus()) * kLdsBytes * passes;
}

extern "C" cf_status cf_stream_read_async(const void *src, uint64_t bytes, uint32_t *sink, void *stream) {
  if (!src || !sink || bytes % 16 != 0 || reinterpret_cast<uintptr_t>(src) % 16 != 0) return CF_ERR_INVALID_ARGUMENT;
  if (bytes == 0) return CF_OK;
  const uint64_t n16 = bytes / 16;
  const uint64_t chunks = (n16 + kChunk16 - 1) / kChunk16;
  const unsigned blocks = static_cast<unsigned>(chunks < 0x7FFFFFFFull ? chunks : 0x7FFFFFFFull);
  stream_read_kernel<<<blocks, kThreads, 0, cfd::as_stream(stream)>>>(static_cast<const u32x4 *>(src), n16, sink);
  return cfd::launch_status();
}
