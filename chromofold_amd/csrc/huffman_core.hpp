// huffman_core.hpp — per-lane canonical-Huffman LUT decode of an MSB-first bit stream (the block-Huffman format of
// the reference: codes length-limited to `maxlen`, lut[look] = symbol | code_length << 8 over a `maxlen`-bit
// lookahead, reference include/chromofold/detail/block_huffman_device.cuh:12-19).
//
// The reference assembles the lookahead one bit (one global load) at a time. Here a lane keeps a 64-bit window of
// the stream in registers and refills it one 32-bit word at a time, only when the lookahead needs bits it does not
// hold — so exactly the words the reference touches are read, never one beyond them.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace cfh {

// random-access decode at bit `pos`: returns sym | len << 8
__device__ __forceinline__ int huff_at(const uint32_t *__restrict__ words, const int32_t *__restrict__ lut, int maxlen,
                                       int64_t pos) {
  const int64_t wi = pos >> 5;
  const int b = static_cast<int>(pos & 31);
  uint64_t v = static_cast<uint64_t>(words[wi]) << 32;
  if (b + maxlen > 32) v |= words[wi + 1];
  const uint32_t look = static_cast<uint32_t>((v << b) >> (64 - maxlen));
  return lut[look];
}

// sequential decoder: `buf` holds `nb` valid stream bits, MSB-aligned
struct BitReader {
  const uint32_t *__restrict__ words;
  int64_t next;  // index of the next word to load
  uint64_t buf;
  int nb;

  __device__ __forceinline__ BitReader(const uint32_t *__restrict__ w, int64_t pos) : words(w) {
    next = (pos >> 5) + 1;
    const int b = static_cast<int>(pos & 31);
    buf = (static_cast<uint64_t>(w[pos >> 5]) << 32) << b;
    nb = 32 - b;
  }
  // symbol | len << 8 of the code at the read position; advances past it
  __device__ __forceinline__ int decode(const int32_t *__restrict__ lut, int maxlen) {
    if (nb < maxlen) {
      buf |= static_cast<uint64_t>(words[next++]) << (32 - nb);
      nb += 32;
    }
    const int e = lut[static_cast<uint32_t>(buf >> (64 - maxlen))];
    const int len = e >> 8;
    buf <<= len;
    nb -= len;
    return e;
  }
};

}  // namespace cfh
