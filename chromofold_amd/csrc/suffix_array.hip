// suffix_array.hip — GPU suffix-array construction (prefix doubling) for the FM-index build, gfx950.
//
// Replaces reference src/cuda/suffix_array.cu:42-65 (thrust prefix doubling). Same algorithm: each round sorts
// the suffixes by the pair (rank[i], rank[i+k] + 1 or 0 past the end) and re-ranks by adjacent-key differences;
// the suffix array of a sentinel-terminated string is unique, so the result equals the CPU suffix array bit for
// bit. MI355X-side choices: the pair key is packed into 2*bits(n+1) bits and the LSD radix sort only visits those
// bits; the key gather for round k is fused with the previous ranks so no separate key array per suffix start is
// materialised; all scratch lives in one caller-provided workspace.
#include <hipcub/hipcub.hpp>

#include <vector>

#include "cf_device.hpp"
#include "chromofold/chromofold_index.h"

namespace {

constexpr unsigned kThreads = 256;

int bits_for(uint32_t v) {
  int b = 0;
  while (b < 32 && (1ull << b) <= v) ++b;
  return b;
}

// gkey[j] = rank[sa[j]] << sh | (sa[j]+k < n ? rank[sa[j]+k] + 1 : 0)
__global__ void sa_keys(const int32_t *__restrict__ sa, const int32_t *__restrict__ rank, int n, int k, int sh,
                        uint64_t *__restrict__ key) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= n) return;
  const int i = sa[j];
  const uint64_t hi = static_cast<uint32_t>(rank[i]);
  const uint64_t lo = (i + k < n) ? static_cast<uint64_t>(static_cast<uint32_t>(rank[i + k]) + 1u) : 0ull;
  key[j] = (hi << sh) | lo;
}

__global__ void sa_flags(const uint64_t *__restrict__ key, int n, int32_t *__restrict__ flag) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= n) return;
  flag[j] = (j > 0 && key[j] != key[j - 1]) ? 1 : 0;
}

__global__ void sa_scatter(const int32_t *__restrict__ sa, const int32_t *__restrict__ pos, int n,
                           int32_t *__restrict__ rank) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= n) return;
  rank[sa[j]] = pos[j];
}

__global__ void sa_init(const int32_t *__restrict__ s, int n, int32_t *__restrict__ sa, int32_t *__restrict__ rank) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= n) return;
  sa[j] = j;
  rank[j] = s[j];
}

struct Layout {
  size_t sa, sa2, rank, pos, key, key2, sort_tmp, scan_tmp, total;
};

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

Layout layout(int n, int key_bits) {
  Layout L{};
  size_t sort_bytes = 0, scan_bytes = 0;
  static_cast<void>(hipcub::DeviceRadixSort::SortPairs(nullptr, sort_bytes, static_cast<uint64_t *>(nullptr),
                                     static_cast<uint64_t *>(nullptr), static_cast<int32_t *>(nullptr),
                                     static_cast<int32_t *>(nullptr), n, 0, key_bits));
  static_cast<void>(hipcub::DeviceScan::InclusiveSum(nullptr, scan_bytes, static_cast<int32_t *>(nullptr),
                                   static_cast<int32_t *>(nullptr), n));
  size_t at = 0;
  auto take = [&](size_t bytes) {
    const size_t here = at;
    at += align256(bytes);
    return here;
  };
  L.sa = take(4ull * n);
  L.sa2 = take(4ull * n);
  L.rank = take(4ull * n);
  L.pos = take(4ull * n);
  L.key = take(8ull * n);
  L.key2 = take(8ull * n);
  L.sort_tmp = take(sort_bytes);
  L.scan_tmp = take(scan_bytes);
  L.total = at;
  return L;
}

int key_bits_for(int n, int32_t max_symbol) {
  const uint32_t top = static_cast<uint32_t>(std::max<int64_t>(n, static_cast<int64_t>(max_symbol) + 1));
  return bits_for(top) + bits_for(static_cast<uint32_t>(n) + 1);
}

}  // namespace

extern "C" uint64_t cf_suffix_array_workspace_bytes(int32_t n, int32_t max_symbol) {
  if (n <= 0 || max_symbol < 0) return 0;
  const int kb = key_bits_for(n, max_symbol);
  if (kb > 64) return 0;
  return layout(n, kb).total;
}

extern "C" cf_status cf_suffix_array(const int32_t *s, int32_t n, int32_t max_symbol, int32_t *sa_out,
                                     void *workspace, uint64_t workspace_bytes, void *stream) {
  if (!s || !sa_out || n <= 0 || max_symbol < 0) return CF_ERR_INVALID_ARGUMENT;
  const int kb = key_bits_for(n, max_symbol);
  if (kb > 64) return CF_ERR_UNSUPPORTED;
  const Layout L = layout(n, kb);
  if (!workspace || workspace_bytes < L.total) return CF_ERR_INVALID_ARGUMENT;
  const hipStream_t st = cfd::as_stream(stream);
  uint8_t *ws = static_cast<uint8_t *>(workspace);
  int32_t *sa = reinterpret_cast<int32_t *>(ws + L.sa), *sa2 = reinterpret_cast<int32_t *>(ws + L.sa2);
  int32_t *rank = reinterpret_cast<int32_t *>(ws + L.rank), *pos = reinterpret_cast<int32_t *>(ws + L.pos);
  uint64_t *key = reinterpret_cast<uint64_t *>(ws + L.key), *key2 = reinterpret_cast<uint64_t *>(ws + L.key2);
  const int sh = bits_for(static_cast<uint32_t>(n) + 1);
  const unsigned blocks = cfd::grid_for(n, kThreads);
  sa_init<<<blocks, kThreads, 0, st>>>(s, n, sa, rank);
  if (hipPeekAtLastError() != hipSuccess) return CF_ERR_CUDA;
  for (int64_t k = 1;; k <<= 1) {
    sa_keys<<<blocks, kThreads, 0, st>>>(sa, rank, n, static_cast<int>(std::min<int64_t>(k, n)), sh, key);
    size_t sort_bytes = 0;
    static_cast<void>(hipcub::DeviceRadixSort::SortPairs(nullptr, sort_bytes, key, key2, sa, sa2, n, 0, kb, st));
    if (hipcub::DeviceRadixSort::SortPairs(ws + L.sort_tmp, sort_bytes, key, key2, sa, sa2, n, 0, kb, st) !=
        hipSuccess)
      return CF_ERR_CUDA;
    std::swap(sa, sa2);
    sa_flags<<<blocks, kThreads, 0, st>>>(key2, n, pos);
    size_t scan_bytes = 0;
    static_cast<void>(hipcub::DeviceScan::InclusiveSum(nullptr, scan_bytes, pos, pos, n, st));
    if (hipcub::DeviceScan::InclusiveSum(ws + L.scan_tmp, scan_bytes, pos, pos, n, st) != hipSuccess)
      return CF_ERR_CUDA;
    sa_scatter<<<blocks, kThreads, 0, st>>>(sa, pos, n, rank);
    int32_t last = 0;
    if (hipMemcpyAsync(&last, pos + (n - 1), 4, hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
      return CF_ERR_CUDA;
    if (last == n - 1 || k >= n) break;  // all ranks distinct: sa is the suffix array
  }
  if (hipMemcpyAsync(sa_out, sa, 4ull * n, hipMemcpyDeviceToDevice, st) != hipSuccess) return CF_ERR_CUDA;
  return cfd::launch_status();
}

// Host-vector convenience with the reference's C++ signature (reference src/cuda/suffix_array.cu:42). Allocates
// its device buffers (it is the offline index builder, not a hot-path entry point) and synchronises.
void cf_gpu_suffix_array(const std::vector<int> &s, std::vector<int> &out) {
  const int n = static_cast<int>(s.size());
  out.assign(n, 0);
  if (n == 0) return;
  int32_t mx = 0;
  for (int v : s) mx = std::max(mx, v);
  const uint64_t wsb = cf_suffix_array_workspace_bytes(n, mx);
  void *d_s = nullptr, *d_sa = nullptr, *d_ws = nullptr;
  if (hipMalloc(&d_s, 4ull * n) != hipSuccess || hipMalloc(&d_sa, 4ull * n) != hipSuccess ||
      hipMalloc(&d_ws, wsb) != hipSuccess) {
    static_cast<void>(hipFree(d_s));
    static_cast<void>(hipFree(d_sa));
    out.clear();
    return;
  }
  if (hipMemcpy(d_s, s.data(), 4ull * n, hipMemcpyHostToDevice) == hipSuccess &&
      cf_suffix_array(static_cast<const int32_t *>(d_s), n, mx, static_cast<int32_t *>(d_sa), d_ws, wsb, nullptr) ==
          CF_OK &&
      hipMemcpy(out.data(), d_sa, 4ull * n, hipMemcpyDeviceToHost) == hipSuccess) {
  } else {
    out.clear();
  }
  static_cast<void>(hipFree(d_s));
  static_cast<void>(hipFree(d_sa));
  static_cast<void>(hipFree(d_ws));
}
