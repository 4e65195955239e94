// stream_read.hip — read-only HBM streaming kernel (chromofold_measure.h): the achievable read bandwidth of the
// device, measured with the access pattern the decode kernels use for their pools (16-byte loads, coalesced, each
// byte read once).
//
// A grid of a few workgroups per CU walks the buffer in a grid-stride loop with four 16-byte loads in flight per
// lane; the data is folded into one XOR per lane so the loads cannot be removed, and one atomic XOR per workgroup
// writes the result.
#include "cf_device.hpp"
#include "chromofold/chromofold_measure.h"

namespace {

constexpr int kThreads = 256;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(kThreads) stream_read_kernel(const u32x4 *__restrict__ src, uint64_t n16,
                                                               uint32_t *__restrict__ sink) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads;
  uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
  uint32_t acc = 0;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const u32x4 a = __builtin_nontemporal_load(src + i), b = __builtin_nontemporal_load(src + i + stride);
    const u32x4 c = __builtin_nontemporal_load(src + i + 2 * stride), d = __builtin_nontemporal_load(src + i + 3 * stride);
    acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
  }
  for (; i < n16; i += stride) {
    const u32x4 a = __builtin_nontemporal_load(src + i);
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  __shared__ uint32_t s_acc;
  if (threadIdx.x == 0) s_acc = 0;
  __syncthreads();
  atomicXor(&s_acc, acc);
  __syncthreads();
  if (threadIdx.x == 0) atomicXor(sink, s_acc);
}

}  // namespace

extern "C" cf_status cf_stream_read_async(const void *src, uint64_t bytes, uint32_t *sink, void *stream) {
  if (!src || !sink || bytes % 16 != 0 || reinterpret_cast<uintptr_t>(src) % 16 != 0) return CF_ERR_INVALID_ARGUMENT;
  if (bytes == 0) return CF_OK;
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  const uint64_t n16 = bytes / 16;
  const uint64_t want = (n16 + 4ull * kThreads - 1) / (4ull * kThreads);
  const unsigned blocks = static_cast<unsigned>(want < 8ull * cus ? (want ? want : 1) : 8ull * cus);
  stream_read_kernel<<<blocks, kThreads, 0, cfd::as_stream(stream)>>>(static_cast<const u32x4 *>(src), n16, sink);
  return cfd::launch_status();
}
