// kv_encode.hip — device-side sealing: quantise and entropy-code KV page groups on the GPU.
//
// The device twin of the host encoder cf_kv_encode_groups (kv_codec.cpp): same group blob format
// (kv_codec_ext.h), same pool packing and offsets, byte for byte. It replaces the host quantise + encode step of
// the append path (reference src/runtime/compressed_kv_cache.cu:89-109 seals pages on the host), so K/V that the
// model produced in HBM never leave the device. Three launches on the caller's stream, nothing allocated:
//   1. table_prep_kernel: one workgroup per table blob derives the compact (freq, cum) pairs of its 256 joint
//      symbols (last slot with offset 0 wins, exactly the host loader's rule) and whether the table is usable;
//      workgroup 0 also clears the status word.
//   2. encode_kernel: one 4-wavefront workgroup per group. Phase 1: wavefront G quantises page G (absmax over the
//      page's present tokens, IEEE division, round half to even) into LDS symbol tiles laid out for phase 2's
//      reads (K token-major, V dim-major, both padded to odd word strides). Phase 2: each wavefront rANS-codes one
//      of the four chains (K A, K B, V A, V B; 64 interleaved states each); the renormalisation words of one step
//      are placed with a ballot prefix count, written from the top of an LDS buffer down so that the reversed
//      stream needs no second pass. Phase 3 bit-slices the low parts and writes the blob (or the INT8 fallback when
//      the words exceed CF_KV_RANS_MAX_GROUP_WORDS) into a fixed-capacity staging slot, and its size in 16-byte
//      units.
//   3. an exclusive scan of the sizes (hipcub), then pack_kernel copies every blob to pool[pool_at + offset],
//      writes offsets_out and *pool_end — or nothing at all when any group or the pool capacity failed, in which
//      case the status word holds CF_ERR_INVALID_ARGUMENT.
#include <hipcub/hipcub.hpp>

#include <cstdint>

#include "cf_device.hpp"
#include "chromofold/kv_codec_ext.h"

namespace {

constexpr int kThreads = 256;
constexpr uint32_t kHeader = 64;
constexpr uint32_t kMaxDim = CF_KV_MAX_HEAD_DIM;
constexpr uint32_t kChainCap = CF_KV_RANS_MAX_GROUP_WORDS / 2;  // per chain: D/8 quads x 64 lanes <= 1024 words
constexpr int kKStride = kMaxDim / 4 + 1;              // words per K token row (odd: conflict-free lane reads)
constexpr int kVStride = 5;                            // words per V dim row (4 token quads + 1)
constexpr uint32_t kTableBytes = CF_KV_RANS_TABLE_BYTES;

__host__ __device__ inline uint64_t align16(uint64_t v) { return (v + 15) & ~uint64_t(15); }

bool dim_ok(uint32_t d) { return d != 0 && d % 16 == 0 && d <= kMaxDim; }

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
  const uint32_t *ctab, *tvalid;
  uint32_t table_count;
  uint32_t codec, head_dim;
  uint8_t *stage;
  uint64_t cap;
  uint32_t *units, *status;
};

// Symbol word (4 symbols, symbol i in byte i) of lane (G, t), quad q, in the lane order of kv_codec_ext.h.
__device__ __forceinline__ uint32_t k_word(const uint32_t *kS, int G, int t, int q) {
  return kS[(G * 16 + t) * kKStride + q];
}
__device__ __forceinline__ uint32_t v_word(const uint32_t *vT, int G, int t, int q, int ng) {
  return vT[(G * kMaxDim + t + 16 * (q % ng)) * kVStride + q / ng];
}

__device__ __forceinline__ uint32_t joint_of(uint32_t w) {
  return ((w >> 6) & 3u) | ((w >> 12) & 0xCu) | ((w >> 18) & 0x30u) | ((w >> 24) & 0xC0u);
}

__global__ void __launch_bounds__(kThreads) encode_kernel(EncodeArgs a) {
  __shared__ uint32_t kS[4 * 16 * kKStride];
  __shared__ uint32_t vT[4 * kMaxDim * kVStride];
  __shared__ uint16_t s_words[4][kChainCap];
  __shared__ uint32_t s_tab[2][256];
  __shared__ float s_scale[2][4];
  __shared__ uint32_t s_tc[4], s_count[4], s_bad;

  const uint64_t g = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t D = a.head_dim, nq = D / 4, ng = D / 16;
  const uint32_t pc = a.page_counts[g];
  const uint64_t p0 = a.first_page[g];
  const uint32_t head = a.heads ? a.heads[g] : 0u;
  const bool rans = a.codec == CF_KV_CODEC_RANS_HYBRID;
  if (tid == 0) {
    uint32_t bad = (pc == 0 || pc > 4) ? 1u : 0u;
    for (int G = 0; G < 4; ++G) {
      const uint32_t tc = static_cast<uint32_t>(G) < pc ? (a.token_counts ? a.token_counts[p0 + G] : 16u) : 0u;
      if (static_cast<uint32_t>(G) < pc && (tc == 0 || tc > 16)) bad = 1;
      s_tc[G] = bad ? 0u : tc;
    }
    if (rans && (2ull * head + 1 >= a.table_count || !a.tvalid[2 * head] || !a.tvalid[2 * head + 1])) bad = 1;
    s_bad = bad;
  }
  __syncthreads();
  if (s_bad) {
    if (tid == 0) {
      *a.status = CF_ERR_INVALID_ARGUMENT;
      a.units[g] = 0;
    }
    return;
  }
  if (rans) {  // head validated above: tables 2 head and 2 head + 1 exist
    for (int i = tid; i < 512; i += kThreads)
      s_tab[i >> 8][i & 255] = a.ctab[(2ull * head + (i >> 8)) * 256 + (i & 255)];
  }

  // ---- phase 1: wavefront G quantises page G of K and V
  {
    const int G = wave;
    const uint32_t tc = s_tc[G];
    const uint64_t page_vals = 16ull * D;
    const float *kp = a.keys + (p0 + G) * page_vals;
    const float *vp = a.values + (p0 + G) * page_vals;
    // K: float4 index i = r * 64 + lane -> token i / nq, quad i % nq (4 * D float4 per page, <= 8 per lane)
    float4 kx[8];
    float m = 0.0f;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const uint32_t i = r * 64 + lane;
      kx[r] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (i < 4 * D && i / nq < tc) {
        kx[r] = *reinterpret_cast<const float4 *>(kp + 4ull * i);
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
        if (t < tc)
          w = quant8(kx[r].x, ks) | quant8(kx[r].y, ks) << 8 | quant8(kx[r].z, ks) << 16 | quant8(kx[r].w, ks) << 24;
        kS[(G * 16 + t) * kKStride + q] = w;
      }
    }
    // V: lane owns dims d = lane, lane + 64; 16 tokens each, packed as 4 token quads
    float vx[2][16];
    m = 0.0f;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const uint32_t d = r * 64 + lane;
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        vx[r][t] = 0.0f;
        if (d < D && static_cast<uint32_t>(t) < tc) {
          vx[r][t] = vp[static_cast<uint64_t>(t) * D + d];
          m = __builtin_fmaxf(m, __builtin_fabsf(vx[r][t]));
        }
      }
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
            w |= (t < tc ? quant8(vx[r][t], vs) : 128u) << (8 * i);
          }
          vT[(G * kMaxDim + d) * kVStride + tq] = w;
        }
      }
    }
    if (lane == 0) {
      s_scale[0][G] = tc ? ks : 1.0f;
      s_scale[1][G] = tc ? vs : 1.0f;
    }
  }
  __syncthreads();

  uint8_t *blob = a.stage + g * a.cap;
  const int G = lane >> 4, t = lane & 15;
  // ---- phase 2: rANS, one chain per wavefront: wave w codes stream w / 2 (K, V), chain w % 2 (its quads
  // q = chain, chain + 2, ..., encoded in reverse)
  if (rans) {
    const int s = wave >> 1, ch = wave & 1;
    uint32_t x = 1u << 16;
    uint32_t base = 0;
    for (int q = static_cast<int>(nq) - 2 + ch; q >= 0; q -= 2) {
      const uint32_t w = s == 0 ? k_word(kS, G, t, q) : v_word(vT, G, t, q, ng);
      const uint32_t e = s_tab[s][joint_of(w)];
      const uint32_t f = e & 0xFFFFu, cum = e >> 16;
      const bool emit = static_cast<uint64_t>(x) >= (static_cast<uint64_t>(f) << 21);  // (2^16 >> 11) << 16 = 2^21
      const uint64_t mask = __ballot(emit);
      if (emit) {
        const uint32_t above = __popcll(mask & ~((2ull << lane) - 1ull));  // emitters at higher lanes go first
        s_words[wave][kChainCap - 1 - (base + above)] = static_cast<uint16_t>(x & 0xFFFFu);
        x >>= 16;
      }
      base += __popcll(mask);
      x = ((x / f) << CF_KV_RANS_PROB_BITS) + (x % f) + cum;
    }
    *reinterpret_cast<uint32_t *>(blob + kHeader + 4 * (wave * 64 + lane)) = x;
    if (lane == 0) s_count[wave] = base;
  }
  __syncthreads();

  // ---- phase 3: the blob
  uint32_t wc[4] = {0, 0, 0, 0};
  if (rans)
    for (int c = 0; c < 4; ++c) wc[c] = s_count[c];
  const uint32_t total = wc[0] + wc[1] + wc[2] + wc[3];
  const uint32_t nlow = 3 * ng * 64;
  const uint64_t wat = kHeader + 4 * 64 * 4 + 2ull * nlow * 4;  // first rANS word of the blob
  // (the second bound never binds: the first one caps the words and the capacity covers it; it keeps the staging
  // slot safe by construction)
  const bool raw = !rans || total > CF_KV_RANS_MAX_GROUP_WORDS || wat + 2ull * total > a.cap;
  uint64_t size;
  if (raw) {
    // INT8: word (q * 64 + L) of stream s = the 4 symbols of quad q of lane L
    uint32_t *out = reinterpret_cast<uint32_t *>(blob + kHeader);
    for (uint32_t i = tid; i < 2 * nq * 64; i += kThreads) {
      const uint32_t s = i / (nq * 64), r = i % (nq * 64), q = r / 64, L = r % 64;
      out[i] = s == 0 ? k_word(kS, L >> 4, L & 15, q) : v_word(vT, L >> 4, L & 15, q, ng);
    }
    size = kHeader + 2ull * nq * 64 * 4;
  } else {
    if (wave < 2) {  // bit-sliced low parts of stream `wave`
      const int s = wave;
      uint32_t *lo = reinterpret_cast<uint32_t *>(blob + kHeader + 4 * 64 * 4) + s * nlow;
      for (uint32_t gi = 0; gi < ng; ++gi) {
        uint32_t n0 = 0, n1 = 0, c = 0;
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
          const int q = 4 * gi + qd;
          const uint32_t w = s == 0 ? k_word(kS, G, t, q) : v_word(vT, G, t, q, ng);
          const uint32_t nib = (w & 0x0F0F0F0Fu) << (4 * (qd & 1));
          if (qd < 2) n0 |= nib; else n1 |= nib;
          c |= ((w >> 4) & 0x03030303u) << (2 * qd);
        }
        lo[(gi * 3 + 0) * 64 + lane] = n0;
        lo[(gi * 3 + 1) * 64 + lane] = n1;
        lo[(gi * 3 + 2) * 64 + lane] = c;
      }
    }
    uint16_t *wo = reinterpret_cast<uint16_t *>(blob + wat);  // streams K A, K B, V A, V B back to back
    const uint32_t o1 = wc[0], o2 = o1 + wc[1], o3 = o2 + wc[2];
    for (uint32_t i = tid; i < total; i += kThreads) {
      const uint32_t c = i < o1 ? 0u : i < o2 ? 1u : i < o3 ? 2u : 3u;
      const uint32_t at = i - (c == 0 ? 0u : c == 1 ? o1 : c == 2 ? o2 : o3);
      wo[i] = s_words[c][kChainCap - wc[c] + at];
    }
    const uint64_t end = wat + 2ull * total;
    size = align16(end);
    for (uint64_t b = end + tid; b < size; b += kThreads) blob[b] = 0;
  }
  if (tid == 0) {
    cf_kv_group_header h{};
    h.codec = raw ? CF_KV_CODEC_INT8 : CF_KV_CODEC_RANS_HYBRID;
    for (int c = 0; c < 4; ++c) h.word_count[c] = static_cast<uint16_t>(raw ? 0 : wc[c]);
    for (int i = 0; i < 4; ++i) {
      h.token_count[i] = static_cast<uint16_t>(s_tc[i]);
      h.k_scale[i] = s_scale[0][i];
      h.v_scale[i] = s_scale[1][i];
    }
    h.head_dim = static_cast<uint16_t>(D);
    h.page_count = static_cast<uint16_t>(pc);
    h.k_table = 2 * head;
    h.v_table = 2 * head + 1;
    const uint32_t *src = reinterpret_cast<const uint32_t *>(&h);
    uint32_t *dst = reinterpret_cast<uint32_t *>(blob);
#pragma unroll
    for (int i = 0; i < 16; ++i) dst[i] = src[i];
    a.units[g] = static_cast<uint32_t>(size / 16);
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
  if (!dim_ok(head_dim) || ngroups == 0 || ngroups >= (1ull << 31)) return 0;
  if (codec != CF_KV_CODEC_INT8 && codec != CF_KV_CODEC_RANS_HYBRID) return 0;
  return layout_of(codec, head_dim, ngroups, codec == CF_KV_CODEC_RANS_HYBRID ? table_count : 0).total;
}

extern "C" cf_status cf_kv_encode_groups_async(uint32_t codec, const float *keys, const float *values,
                                               uint64_t ngroups, const uint64_t *first_page,
                                               const uint32_t *page_counts, const uint32_t *token_counts,
                                               uint32_t head_dim, const uint8_t *tables, uint32_t table_count,
                                               const uint32_t *heads, uint8_t *pool, uint64_t pool_capacity,
                                               uint64_t pool_at, uint32_t *offsets_out, uint64_t *pool_end,
                                               uint32_t *status, void *workspace, uint64_t workspace_bytes,
                                               void *stream) {
  if (!keys || !values || !first_page || !page_counts || !pool || !offsets_out || !pool_end || !status ||
      !workspace || pool_at % 16 != 0 || ngroups == 0 || ngroups >= (1ull << 31) ||
      reinterpret_cast<uintptr_t>(keys) % 16 != 0 || reinterpret_cast<uintptr_t>(values) % 16 != 0 ||
      reinterpret_cast<uintptr_t>(pool) % 16 != 0)
    return CF_ERR_INVALID_ARGUMENT;
  if (codec != CF_KV_CODEC_INT8 && codec != CF_KV_CODEC_RANS_HYBRID) return CF_ERR_UNSUPPORTED;
  if (!dim_ok(head_dim)) return CF_ERR_UNSUPPORTED;
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
  EncodeArgs a{keys, values, first_page, page_counts, token_counts, heads, ctab, tvalid, table_count, codec,
               head_dim, ws + L.stage, L.cap, units, status};
  encode_kernel<<<static_cast<unsigned>(ngroups), kThreads, 0, st>>>(a);
  if (cfd::launch_status() != CF_OK) return CF_ERR_CUDA;
  size_t scan_bytes = L.scan_bytes;
  if (hipcub::DeviceScan::ExclusiveSum(ws + L.scan, scan_bytes, units, offs, static_cast<int>(ngroups + 1), st) !=
      hipSuccess)
    return CF_ERR_CUDA;
  pack_kernel<<<static_cast<unsigned>(ngroups), 256, 0, st>>>(ws + L.stage, L.cap, offs, ngroups, pool,
                                                               pool_capacity, pool_at, offsets_out, pool_end, status);
  return cfd::launch_status();
}
