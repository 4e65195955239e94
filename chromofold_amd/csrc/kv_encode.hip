// kv_encode.hip — device-side sealing: quantise and entropy-code KV page groups on the GPU.
//
// The device twin of the host encoder cf_kv_encode_groups (kv_codec.cpp): same group blob format
// (kv_codec_ext.h), same chain pairs, same pool packing and offsets, byte for byte. It replaces the host quantise +
// encode step of the append path (reference src/runtime/compressed_kv_cache.cu:89-109 seals pages on the host), so
// K/V that the model produced in HBM never leave the device. Three launches on the caller's stream, nothing
// allocated:
//   1. table_prep_kernel: one workgroup per table blob derives the compact (freq, cum) pairs of its 256 joint
//      symbols (last slot with offset 0 wins, exactly the host loader's rule) and whether the table is usable;
//      workgroup 0 also clears the status word.
//   2. encode_kernel: one 8-wavefront workgroup per chain unit (a group alone, or a group and the group that
//      continues its chain; the workgroup of a continuing group only checks its flag). The unit's fields all
//      depend only on the group index, so they are requested at once, and every wavefront issues its page's K/V
//      loads before the first barrier (two memory latencies before any compute, not one per field). Phase 1:
//      wavefront 4 X + G quantises page G of group X (absmax over the page's present tokens, IEEE division, round
//      half to even) into LDS symbol tiles laid out for the later reads (K token-major, V dim-major, both padded to
//      odd word strides). Phase 2: wavefronts 0 and 1 rANS-code the K and V chains across the unit's coded groups in
//      reverse (64 interleaved states each); the renormalisation words of one step are placed with a ballot prefix
//      count, written from the top of an LDS buffer down so that the reversed stream needs no second pass. At the
//      same time wavefronts 2-5 write the raw words of the (group, stream) pairs (frame-rotated nibbles, crumbs and
//      signs). Phase 3 writes the headers and word streams (or the INT8 blob of a group holding -128) into
//      fixed-capacity staging slots, and each blob's size in 16-byte units.
//   3. an exclusive scan of the sizes (hipcub), then pack_kernel copies every blob to pool[pool_at + offset],
//      writes offsets_out and *pool_end — or nothing at all when any group or the pool capacity failed, in which
//      case the status word holds CF_ERR_INVALID_ARGUMENT.
#include <hipcub/hipcub.hpp>

#include <cstdint>

#include "cf_device.hpp"
#include "chromofold/kv_codec_ext.h"

namespace {

constexpr int kEncThreads = 512;  // encode_kernel: 8 wavefronts, one per page of the unit's (up to) two groups
constexpr uint32_t kHeader = 64;
constexpr uint32_t kStateBytes = 2 * 64 * 4;
constexpr uint32_t kMaxDim = CF_KV_MAX_HEAD_DIM;
constexpr uint32_t kStreamCap = CF_KV_RANS_MAX_GROUP_WORDS / 2;  // per stream and group: 64 lanes x D/8 steps
constexpr int kKStride = kMaxDim / 4 + 1;              // words per K token row (odd: conflict-free lane reads)
constexpr int kVStride = 5;                            // words per V dim row (4 token quads + 1)
constexpr uint32_t kTableBytes = CF_KV_RANS_TABLE_BYTES;
constexpr uint32_t kFrame[8] = {0, 4, 2, 6, 1, 5, 3, 7};  // frame of quad k of a sign group
constexpr uint32_t kNWord[8] = {0, 0, 1, 1, 3, 3, 4, 4};  // raw word holding quad k's nibbles (N0 N1 C0 N2 N3 C1 S)

__host__ __device__ inline uint64_t align16(uint64_t v) { return (v + 15) & ~uint64_t(15); }

bool dim_ok(uint32_t codec, uint32_t d) {
  if (d == 0 || d > kMaxDim) return false;
  return codec == CF_KV_CODEC_RANS_HYBRID ? d % 32 == 0 : d % 16 == 0;
}

uint64_t stage_cap(uint32_t codec, uint32_t head_dim) {
  return align16(cf_kv_group_blob_max_bytes(codec, head_dim));
}

// lrint(float) as the x86-64 host encoder computes it, then clamped to int8 and offset: rint (half to even); a
// result outside the range of long, or NaN, is the "integer indefinite" LONG_MIN, which clamps to -128.
__device__ __forceinline__ uint32_t quant8(float x, float scale) {
  const float r = __builtin_rintf(x / scale);
  if (!(__builtin_fabsf(r) < 9.223372036854775808e18f)) return 0u;
  return static_cast<uint32_t>(static_cast<int>(__builtin_fminf(__builtin_fmaxf(r, -128.0f), 127.0f)) + 128);
}

__device__ __forceinline__ float wave_max(float m) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m = __builtin_fmaxf(m, __shfl_xor(m, o));
  return m;
}

__device__ __forceinline__ uint32_t rotl(uint32_t v, uint32_t r) { return r ? (v << r) | (v >> (32 - r)) : v; }

// ------------------------------------------------------------------------------------------------ 1. tables
__global__ void __launch_bounds__(256) table_prep_kernel(const uint8_t *__restrict__ tables, uint32_t table_count,
                                                         uint32_t *__restrict__ ctab, uint32_t *__restrict__ tvalid,
                                                         uint32_t *__restrict__ status, uint32_t *__restrict__ units,
                                                         uint64_t ngroups) {
  __shared__ int s_last[256];
  __shared__ uint32_t s_total, s_bad;
  const int tid = threadIdx.x;
  if (blockIdx.x == 0 && tid == 0) {
    *status = CF_OK;
    units[ngroups] = 0;  // the scan's extra element: its exclusive sum is the pool total
  }
  if (blockIdx.x >= table_count) return;
  const uint32_t *blob = reinterpret_cast<const uint32_t *>(tables + static_cast<uint64_t>(blockIdx.x) * kTableBytes);
  s_last[tid] = -1;
  if (tid == 0) s_total = s_bad = 0;
  __syncthreads();
  for (int s = tid; s < 2048; s += 256) {
    const uint32_t lo = blob[2 * s];
    if (((lo >> 11) & 2047u) == 0) atomicMax(&s_last[(lo >> 22) & 255u], s);
  }
  __syncthreads();
  const int s = s_last[tid];
  const uint32_t f = s < 0 ? 0u : (blob[2 * s] & 2047u);
  if (f == 0) atomicOr(&s_bad, 1u);
  atomicAdd(&s_total, f);
  ctab[blockIdx.x * 256 + tid] = f | static_cast<uint32_t>(s < 0 ? 0 : s) << 16;
  __syncthreads();
  if (tid == 0) tvalid[blockIdx.x] = (!s_bad && s_total == 2048u) ? 1u : 0u;
}

// ------------------------------------------------------------------------------------------------ 2. encode
struct EncodeArgs {
  const float *keys, *values;
  const uint64_t *first_page;
  const uint32_t *page_counts, *token_counts, *heads;
  const uint8_t *continues;
  const uint32_t *ctab, *tvalid;
  uint64_t ngroups;
  uint32_t table_count;
  uint32_t codec, head_dim;
  uint8_t *stage;
  uint64_t cap;
  uint32_t *units, *status;
};

// Symbol word (4 symbols q + 128, symbol i in byte i) of lane (G, t), quad q, in the lane order of kv_codec_ext.h.
__device__ __forceinline__ uint32_t k_word(const uint32_t *kS, int G, int t, int q) {
  return kS[(G * 16 + t) * kKStride + q];
}
__device__ __forceinline__ uint32_t v_word(const uint32_t *vT, int G, int t, int q, int ng) {
  return vT[(G * kMaxDim + t + 16 * (q % ng)) * kVStride + q / ng];
}

// big bits (|q| >= 64: symbol >= 192 or <= 64) of the 4 symbols of a word, bit i for symbol i
__device__ __forceinline__ uint32_t bigs_of(uint32_t w) {
  uint32_t j = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t b = (w >> (8 * i)) & 255u;
    j |= (b >= 192u || b <= 64u ? 1u : 0u) << i;
  }
  return j;
}

__global__ void __launch_bounds__(kEncThreads) encode_kernel(EncodeArgs a) {
  __shared__ uint32_t kS[2][4 * 16 * kKStride];
  __shared__ uint32_t vT[2][4 * kMaxDim * kVStride];
  __shared__ uint16_t s_words[2][2][kStreamCap];  // [stream][group of the unit]
  __shared__ uint32_t s_tab[2][256];
  __shared__ float s_scale[2][2][4];               // [group][K, V][page]
  __shared__ uint32_t s_tc[2][4], s_count[2][2], s_bad, s_minus[2];

  // Group of this workgroup: the even groups first, then the odd ones. Chain units usually start at even groups
  // (pairs 2k, 2k + 1), and the workgroup of a continuing group ends almost at once. With g = blockIdx.x the two kinds
  // alternate in dispatch order, and the dispatcher's round-robin over the CUs of an XCD then placed every unit on
  // the same half of the CUs (measured: units on 128 of 256 CUs, the near-empty workgroups on the other 128); this
  // order dispatches the units over every CU first. A bijection on [0, ngroups).
  const uint64_t half = (a.ngroups + 1) / 2, b = blockIdx.x;
  const uint64_t g = b < half ? 2 * b : 2 * (b - half) + 1;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t D = a.head_dim, nq = D / 4, ng = D / 16;
  const bool rans = a.codec == CF_KV_CODEC_RANS_HYBRID;
  // Every per-unit field depends only on g, so all of them are requested at once (one memory latency), and each
  // wavefront starts loading its page's K/V right after (a second one) before any barrier.
  const uint32_t head = a.heads ? a.heads[g] : 0u;
  const bool cont = a.continues && a.continues[g];
  const bool cont_next = a.continues && g + 1 < a.ngroups && a.continues[g + 1];
  if (cont) {  // the group before this one codes it: only check that it may
    if (tid == 0 && (g == 0 || a.continues[g - 1] || (a.heads && a.heads[g - 1] != head))) {
      *a.status = CF_ERR_INVALID_ARGUMENT;
      a.units[g] = 0;
    }
    return;
  }
  const uint32_t ngu = cont_next ? 2u : 1u;  // groups of the unit
  // wavefront w quantises page G = w % 4 of group X = w / 4 of the unit
  const uint32_t X1 = static_cast<uint32_t>(wave) >> 2, G1 = static_cast<uint32_t>(wave) & 3u;
  const uint32_t pc1 = X1 < ngu ? a.page_counts[g + X1] : 0u;
  const uint64_t p01 = X1 < ngu ? a.first_page[g + X1] : 0u;
  const bool page_ok = G1 < pc1 && pc1 <= 4;  // the page exists (pc1 > 4 fails the unit below)
  const uint64_t page_vals = 16ull * D;
  const float *kp = a.keys + (p01 + G1) * page_vals;
  const float *vp = a.values + (p01 + G1) * page_vals;
  // K: float4 index i = r * 64 + lane -> token i / nq, quad i % nq (4 * D float4 per page, <= 8 per lane); all 16
  // token slots of the page are read (page-major [*][16][D] arrays), tokens past its count are masked below
  float4 kx[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const uint32_t i = r * 64 + lane;
    kx[r] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (page_ok && i < 4 * D) kx[r] = *reinterpret_cast<const float4 *>(kp + 4ull * i);
  }
  // V: lane owns dims d = lane, lane + 64; 16 tokens each
  float vx[2][16];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const uint32_t d = r * 64 + lane;
#pragma unroll
    for (int t = 0; t < 16; ++t) vx[r][t] = (page_ok && d < D) ? vp[static_cast<uint64_t>(t) * D + d] : 0.0f;
  }
  if (tid < 8) {  // thread 4 X + G checks page G of group X
    const uint32_t X = static_cast<uint32_t>(tid) >> 2, G = static_cast<uint32_t>(tid) & 3u;
    bool bad = false;
    uint32_t tc = 0;
    if (X < ngu) {
      const uint32_t pc = a.page_counts[g + X];
      bad = pc == 0 || pc > 4;
      if (!bad && G < pc) {
        tc = a.token_counts ? a.token_counts[a.first_page[g + X] + G] : 16u;
        bad = tc == 0 || tc > 16;
      }
      s_tc[X][G] = tc;
      if (G == 0) s_minus[X] = 0;
    }
    if (tid == 0 && rans && (2ull * head + 1 >= a.table_count || !a.tvalid[2 * head] || !a.tvalid[2 * head + 1]))
      bad = true;
    const uint64_t any = __ballot(bad);
    if (tid == 0) s_bad = any != 0 ? 1u : 0u;
  }
  __syncthreads();
  if (s_bad) {
    if (tid == 0) {
      *a.status = CF_ERR_INVALID_ARGUMENT;
      for (uint32_t X = 0; X < ngu; ++X) a.units[g + X] = 0;
    }
    return;
  }
  if (rans) {  // head validated above: tables 2 head and 2 head + 1 exist
    for (int i = tid; i < 512; i += kEncThreads)
      s_tab[i >> 8][i & 255] = a.ctab[(2ull * head + (i >> 8)) * 256 + (i & 255)];
  }

  // ---- phase 1: wavefront (X, G) quantises page G of K and V of group X of the unit
  if (X1 < ngu) {
    const uint32_t X = X1, G = G1;
    const uint32_t tc = s_tc[X][G];
    bool minus = false;  // a symbol 0 (q = -128) among the present tokens
    float m = 0.0f;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const uint32_t i = r * 64 + lane;
      if (i < 4 * D && i / nq < tc) {
        m = __builtin_fmaxf(m, __builtin_fabsf(kx[r].x));
        m = __builtin_fmaxf(m, __builtin_fabsf(kx[r].y));
        m = __builtin_fmaxf(m, __builtin_fabsf(kx[r].z));
        m = __builtin_fmaxf(m, __builtin_fabsf(kx[r].w));
      }
    }
    m = wave_max(m);
    const float ks = m == 0.0f ? 1.0f : m / 127.0f;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const uint32_t i = r * 64 + lane;
      if (i < 4 * D) {
        const uint32_t t = i / nq, q = i % nq;
        uint32_t w = 0x80808080u;
        if (t < tc) {
          const uint32_t b0 = quant8(kx[r].x, ks), b1 = quant8(kx[r].y, ks), b2 = quant8(kx[r].z, ks),
                         b3 = quant8(kx[r].w, ks);
          minus |= b0 == 0 || b1 == 0 || b2 == 0 || b3 == 0;
          w = b0 | b1 << 8 | b2 << 16 | b3 << 24;
        }
        kS[X][(G * 16 + t) * kKStride + q] = w;
      }
    }
    m = 0.0f;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const uint32_t d = r * 64 + lane;
#pragma unroll
      for (int t = 0; t < 16; ++t)
        if (d < D && static_cast<uint32_t>(t) < tc) m = __builtin_fmaxf(m, __builtin_fabsf(vx[r][t]));
    }
    m = wave_max(m);
    const float vs = m == 0.0f ? 1.0f : m / 127.0f;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const uint32_t d = r * 64 + lane;
      if (d < D) {
#pragma unroll
        for (int tq = 0; tq < 4; ++tq) {
          uint32_t w = 0;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t t = 4 * tq + i;
            const uint32_t b = t < tc ? quant8(vx[r][t], vs) : 128u;
            minus |= b == 0;
            w |= b << (8 * i);
          }
          vT[X][(G * kMaxDim + d) * kVStride + tq] = w;
        }
      }
    }
    if (__ballot(minus) != 0 && lane == 0) atomicOr(&s_minus[X], 1u);
    if (lane == 0) {
      s_scale[X][0][G] = tc ? ks : 1.0f;
      s_scale[X][1][G] = tc ? vs : 1.0f;
    }
  }
  __syncthreads();

  // the unit's coded groups, in chain order (a group holding -128 is stored INT8 instead)
  uint32_t list[2], nlist = 0;
  for (uint32_t X = 0; X < ngu; ++X)
    if (rans && !s_minus[X]) list[nlist++] = X;
  const uint32_t sgroups = D / 32, raw_words = 7 * sgroups * 64;
  auto blob_of = [&](uint32_t X) { return a.stage + (g + X) * a.cap; };
  auto raw_at = [&](uint32_t X) { return kHeader + (nlist && X == list[0] ? kStateBytes : 0u); };
  const int G = lane >> 4, t = lane & 15;
  if (wave < 2 && nlist) {
    // ---- phase 2: rANS of stream `wave` over the chain, encoded in reverse (last group, last step first)
    const int s = wave;
    uint32_t x = 1u << 16;
    for (int li = static_cast<int>(nlist) - 1; li >= 0; --li) {
      const uint32_t X = list[li];
      uint32_t base = 0;
      for (int p = static_cast<int>(D / 8) - 1; p >= 0; --p) {
        const uint32_t w0 = s == 0 ? k_word(kS[X], G, t, 2 * p) : v_word(vT[X], G, t, 2 * p, ng);
        const uint32_t w1 = s == 0 ? k_word(kS[X], G, t, 2 * p + 1) : v_word(vT[X], G, t, 2 * p + 1, ng);
        const uint32_t e = s_tab[s][bigs_of(w0) | bigs_of(w1) << 4];
        const uint32_t f = e & 0xFFFFu, cum = e >> 16;
        const bool emit = static_cast<uint64_t>(x) >= (static_cast<uint64_t>(f) << 21);  // (2^16 >> 11) << 16
        const uint64_t mask = __ballot(emit);
        if (emit) {
          const uint32_t above = __popcll(mask & ~((2ull << lane) - 1ull));  // emitters at higher lanes go first
          s_words[s][X][kStreamCap - 1 - (base + above)] = static_cast<uint16_t>(x & 0xFFFFu);
          x >>= 16;
        }
        base += __popcll(mask);
        x = ((x / f) << CF_KV_RANS_PROB_BITS) + (x % f) + cum;
      }
      if (lane == 0) s_count[s][X] = base;
    }
    *reinterpret_cast<uint32_t *>(blob_of(list[0]) + kHeader + 4 * (s * 64 + lane)) = x;
  } else if (wave >= 2 && wave < 6 && static_cast<uint32_t>(wave - 2) / 2 < nlist) {
    // ---- raw words of stream s of coded group list[li]: nibbles, crumbs and signs in their quads' frames
    const int s = (wave - 2) & 1;
    const uint32_t X = list[(wave - 2) / 2];
    uint32_t *out = reinterpret_cast<uint32_t *>(blob_of(X) + raw_at(X)) + s * raw_words;
    for (uint32_t sg = 0; sg < sgroups; ++sg) {
      uint32_t wd[7] = {0, 0, 0, 0, 0, 0, 0};
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int q = 8 * sg + k;
        const uint32_t w = s == 0 ? k_word(kS[X], G, t, q) : v_word(vT[X], G, t, q, ng);
        uint32_t nib = 0, cr = 0, sn = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t b = (w >> (8 * i)) & 255u;
          const uint32_t mag = b >= 128u ? b - 128u : 128u - b;
          nib |= (mag & 15u) << (8 * i);
          cr |= ((mag >> 4) & 3u) << (8 * i + 4);
          sn |= (b < 128u ? 1u : 0u) << (8 * i + 7);
        }
        wd[kNWord[k]] |= rotl(nib, kFrame[k]);
        wd[k < 4 ? 2 : 5] |= rotl(cr, kFrame[k]);
        wd[6] |= rotl(sn, kFrame[k]);
      }
#pragma unroll
      for (int w = 0; w < 7; ++w) out[(7 * sg + w) * 64 + lane] = wd[w];
    }
  }
  __syncthreads();

  // ---- phase 3: word streams and headers of the coded groups, INT8 blobs of the others
  for (uint32_t X = 0; X < ngu; ++X) {
    uint8_t *blob = blob_of(X);
    const bool coded = rans && !s_minus[X];
    uint64_t size;
    uint32_t wc[2] = {0, 0};
    if (!coded) {
      // INT8: word (q * 64 + L) of stream s = the 4 symbols of quad q of lane L
      uint32_t *out = reinterpret_cast<uint32_t *>(blob + kHeader);
      for (uint32_t i = tid; i < 2 * nq * 64; i += kEncThreads) {
        const uint32_t s = i / (nq * 64), r = i % (nq * 64), q = r / 64, L = r % 64;
        out[i] = s == 0 ? k_word(kS[X], L >> 4, L & 15, q) : v_word(vT[X], L >> 4, L & 15, q, ng);
      }
      size = kHeader + 2ull * nq * 64 * 4;
    } else {
      wc[0] = s_count[0][X];
      wc[1] = s_count[1][X];
      const uint64_t wat = raw_at(X) + 2ull * raw_words * 4;  // first rANS word of the blob
      uint16_t *wo = reinterpret_cast<uint16_t *>(blob + wat);  // K stream, then V
      for (uint32_t i = tid; i < wc[0] + wc[1]; i += kEncThreads) {
        const uint32_t s = i < wc[0] ? 0u : 1u, at = i - (s ? wc[0] : 0u);
        wo[i] = s_words[s][X][kStreamCap - wc[s] + at];
      }
      const uint64_t end = wat + 2ull * (wc[0] + wc[1]);
      size = align16(end);
      for (uint64_t b = end + tid; b < size; b += kEncThreads) blob[b] = 0;
    }
    if (tid == 0) {
      cf_kv_group_header h{};
      h.codec = coded ? CF_KV_CODEC_RANS_HYBRID : CF_KV_CODEC_INT8;
      h.word_count[0] = static_cast<uint16_t>(wc[0]);
      h.word_count[1] = static_cast<uint16_t>(wc[1]);
      h.chain = static_cast<uint16_t>(coded && X == list[0] ? 1 : 0);
      for (int i = 0; i < 4; ++i) {
        h.token_count[i] = static_cast<uint16_t>(s_tc[X][i]);
        h.k_scale[i] = s_scale[X][0][i];
        h.v_scale[i] = s_scale[X][1][i];
      }
      h.head_dim = static_cast<uint16_t>(D);
      h.page_count = static_cast<uint16_t>(a.page_counts[g + X]);
      h.k_table = 2 * head;
      h.v_table = 2 * head + 1;
      const uint32_t *src = reinterpret_cast<const uint32_t *>(&h);
      uint32_t *dst = reinterpret_cast<uint32_t *>(blob);
#pragma unroll
      for (int i = 0; i < 16; ++i) dst[i] = src[i];
      a.units[g + X] = static_cast<uint32_t>(size / 16);
    }
  }
}

// ------------------------------------------------------------------------------------------------ 3. pack
__global__ void __launch_bounds__(256) pack_kernel(const uint8_t *__restrict__ stage, uint64_t cap,
                                                   const uint32_t *__restrict__ offs16, uint64_t ngroups,
                                                   uint8_t *__restrict__ pool, uint64_t pool_capacity, uint64_t pool_at,
                                                   uint32_t *__restrict__ offsets_out, uint64_t *__restrict__ pool_end,
                                                   uint32_t *__restrict__ status) {
  if (*status != CF_OK) return;
  const uint64_t g = blockIdx.x;
  const uint64_t end = pool_at + 16ull * offs16[ngroups];
  const uint64_t last_start = pool_at + 16ull * offs16[ngroups - 1];
  if (end > pool_capacity || last_start / 16 > 0xFFFFFFFFull) {
    if (g == 0 && threadIdx.x == 0) *status = CF_ERR_INVALID_ARGUMENT;
    return;
  }
  const uint64_t at = pool_at + 16ull * offs16[g];
  const uint32_t n16 = offs16[g + 1] - offs16[g];
  const uint4 *src = reinterpret_cast<const uint4 *>(stage + g * cap);
  uint4 *dst = reinterpret_cast<uint4 *>(pool + at);
  for (uint32_t i = threadIdx.x; i < n16; i += 256) dst[i] = src[i];
  if (threadIdx.x == 0) {
    offsets_out[g] = static_cast<uint32_t>(at / 16);
    if (g == ngroups - 1) *pool_end = end;
  }
}

// ------------------------------------------------------------------------------------------------ workspace
struct Layout {
  uint64_t ctab, tvalid, units, offs, scan, stage, total, cap, scan_bytes;
};

Layout layout_of(uint32_t codec, uint32_t head_dim, uint64_t ngroups, uint32_t table_count) {
  Layout L{};
  L.cap = stage_cap(codec, head_dim);
  size_t scan_bytes = 0;
  (void)hipcub::DeviceScan::ExclusiveSum(nullptr, scan_bytes, static_cast<uint32_t *>(nullptr),
                                         static_cast<uint32_t *>(nullptr), static_cast<int>(ngroups + 1));
  L.scan_bytes = scan_bytes;
  uint64_t at = 0;
  auto take = [&](uint64_t bytes) {
    const uint64_t o = at;
    at = (at + bytes + 255) & ~uint64_t(255);
    return o;
  };
  L.ctab = take(static_cast<uint64_t>(table_count) * 256 * 4);
  L.tvalid = take(static_cast<uint64_t>(table_count) * 4);
  L.units = take((ngroups + 1) * 4);
  L.offs = take((ngroups + 1) * 4);
  L.scan = take(scan_bytes);
  L.stage = take(ngroups * L.cap);
  L.total = at;
  return L;
}

}  // namespace

extern "C" uint64_t cf_kv_encode_groups_workspace_bytes(uint32_t codec, uint32_t head_dim, uint64_t ngroups,
                                                        uint32_t table_count) {
  if (codec != CF_KV_CODEC_INT8 && codec != CF_KV_CODEC_RANS_HYBRID) return 0;
  if (!dim_ok(codec, head_dim) || ngroups == 0 || ngroups >= (1ull << 31)) return 0;
  return layout_of(codec, head_dim, ngroups, codec == CF_KV_CODEC_RANS_HYBRID ? table_count : 0).total;
}

extern "C" cf_status cf_kv_encode_groups_async(uint32_t codec, const float *keys, const float *values,
                                               uint64_t ngroups, const uint64_t *first_page,
                                               const uint32_t *page_counts, const uint32_t *token_counts,
                                               uint32_t head_dim, const uint8_t *tables, uint32_t table_count,
                                               const uint32_t *heads, const uint8_t *continues, uint8_t *pool,
                                               uint64_t pool_capacity,
                                               uint64_t pool_at, uint32_t *offsets_out, uint64_t *pool_end,
                                               uint32_t *status, void *workspace, uint64_t workspace_bytes,
                                               void *stream) {
  if (!keys || !values || !first_page || !page_counts || !pool || !offsets_out || !pool_end || !status ||
      !workspace || pool_at % 16 != 0 || ngroups == 0 || ngroups >= (1ull << 31) ||
      reinterpret_cast<uintptr_t>(keys) % 16 != 0 || reinterpret_cast<uintptr_t>(values) % 16 != 0 ||
      reinterpret_cast<uintptr_t>(pool) % 16 != 0)
    return CF_ERR_INVALID_ARGUMENT;
  if (codec != CF_KV_CODEC_INT8 && codec != CF_KV_CODEC_RANS_HYBRID) return CF_ERR_UNSUPPORTED;
  if (!dim_ok(codec, head_dim)) return CF_ERR_UNSUPPORTED;
  const bool rans = codec == CF_KV_CODEC_RANS_HYBRID;
  if (rans && (!tables || table_count < 2)) return CF_ERR_INVALID_ARGUMENT;
  if (!rans) table_count = 0;
  const Layout L = layout_of(codec, head_dim, ngroups, table_count);
  if (workspace_bytes < L.total) return CF_ERR_INVALID_ARGUMENT;
  if (ngroups * (L.cap / 16) >= (1ull << 32)) return CF_ERR_UNSUPPORTED;  // 16-byte unit sums stay in u32
  hipStream_t st = cfd::as_stream(stream);
  uint8_t *ws = static_cast<uint8_t *>(workspace);
  uint32_t *ctab = reinterpret_cast<uint32_t *>(ws + L.ctab);
  uint32_t *tvalid = reinterpret_cast<uint32_t *>(ws + L.tvalid);
  uint32_t *units = reinterpret_cast<uint32_t *>(ws + L.units);
  uint32_t *offs = reinterpret_cast<uint32_t *>(ws + L.offs);

  table_prep_kernel<<<table_count ? table_count : 1, 256, 0, st>>>(tables, table_count, ctab, tvalid, status, units,
                                                                   ngroups);
  if (cfd::launch_status() != CF_OK) return CF_ERR_CUDA;
  EncodeArgs a{keys, values, first_page, page_counts, token_counts, heads, continues, ctab, tvalid, ngroups,
               table_count, codec, head_dim, ws + L.stage, L.cap, units, status};
  encode_kernel<<<static_cast<unsigned>(ngroups), kEncThreads, 0, st>>>(a);
  if (cfd::launch_status() != CF_OK) return CF_ERR_CUDA;
  size_t scan_bytes = L.scan_bytes;
  if (hipcub::DeviceScan::ExclusiveSum(ws + L.scan, scan_bytes, units, offs, static_cast<int>(ngroups + 1), st) !=
      hipSuccess)
    return CF_ERR_CUDA;
  pack_kernel<<<static_cast<unsigned>(ngroups), 256, 0, st>>>(ws + L.stage, L.cap, offs, ngroups, pool,
                                                               pool_capacity, pool_at, offsets_out, pool_end, status);
  return cfd::launch_status();
}
