// nibble_kv.hip — int4 nibble pages on gfx950: sealing kernels and batched split-context attention.
//
//   block_scale_kernel  finite scan + per-block absmax scale of a page's K and V   reference
//                       src/cuda/device_kv_seal_attention.cu:72-78 (finite_scan), :80-104 (the scale half)
//   pack_kernel         quantise + nibble-pack both streams, 8 values per lane     reference :80-113
//   convert_kernel      strided f16/bf16/f32 view -> fp32 active rows              reference
//                       src/cuda/device_kv_dataplane.cu:48-69
//   nib_attn_kernel     split-context attention of a batch of requests over sealed pages + an fp32 active page
//   nib_merge_kernel    merges the splits of every (request, query token, query head) row and stores the output
//                       in the caller's dtype and strides
//   The attention replaces the reference's one-block-per-(head, token) kernels (device_kv_seal_attention.cu:
//   126-194, multisequence_cuda_resolver.cu:136-195) with the same arithmetic contract: key position p is used by
//   query position P when p <= P and, with window w > 0, p + w > P; softmax with a running maximum; empty rows
//   produce 0. Requests flagged for the batched-items contract (reference src/cuda/production_attention.cu:59-139)
//   instead read two's-complement nibbles (each loaded word xor 0x88888888 gives the offset-8 form), count scale
//   blocks per (token, KV head) row, skip pages with a NULL pointer, and use p unless w > 0 and p + w < P.
//
// Attention layout: a workgroup takes `hw` KV heads x LG lanes; each lane owns 8 consecutive dims (one 32-bit word
// of nibbles) of one KV head for G query heads of that head's group, and walks the split's tokens. A token's
// score is the lane's 8-term partial dot reduced over the LG lanes of the row with DPP (quad_perm, half-row and
// row mirrors, then one xor-16 swizzle for 32-lane rows). The block scale and the -8 symbol offset are applied to
// the partial dot (sum q (s - 8) = sum q s - 8 sum q, with sum q per lane precomputed), so decoding a word is two
// masks and eight byte-to-float conversions. The softmax runs in the log2 domain; the running maximum is raised
// only when some lane of the wave sees a larger score (a wave-uniform branch).
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>

#include "nibble_kv.hpp"
#include "nibble_page.hpp"

namespace cfnib {

size_t scalar_bytes(uint32_t type) {
  if (type == CF_DEVICE_F16 || type == CF_DEVICE_BF16) return 2;
  if (type == CF_DEVICE_F32) return 4;
  return 0;
}

namespace {

constexpr float kNegInf = -__builtin_huge_valf();

__device__ inline float load_scalar(const void *base, uint32_t type, uint64_t off) {
  const char *p = static_cast<const char *>(base) + off;
  if (type == CF_DEVICE_F16) return __half2float(*reinterpret_cast<const __half *>(p));
  if (type == CF_DEVICE_BF16) return __uint_as_float(uint32_t(*reinterpret_cast<const uint16_t *>(p)) << 16);
  return *reinterpret_cast<const float *>(p);
}

__device__ inline void store_scalar(void *base, uint32_t type, uint64_t off, float x) {
  char *p = static_cast<char *>(base) + off;
  if (type == CF_DEVICE_F16) {
    *reinterpret_cast<__half *>(p) = __float2half(x);
  } else if (type == CF_DEVICE_BF16) {
    uint32_t u = __float_as_uint(x);
    // round to nearest even; NaN stays a quiet NaN
    u = (x != x) ? 0x7fc00000u : u + 0x7fffu + ((u >> 16) & 1u);
    *reinterpret_cast<uint16_t *>(p) = static_cast<uint16_t>(u >> 16);
  } else {
    *reinterpret_cast<float *>(p) = x;
  }
}

// ------------------------------------------------------------------------------------------------ sealing
// One wave per block: K blocks first, then V blocks. Non-finite values are counted; the scale of a block holding
// NaN/Inf is irrelevant because such a page is rejected before packing.
__global__ __launch_bounds__(256) void block_scale_kernel(const float *__restrict__ k, const float *__restrict__ v,
                                                          uint32_t values, uint32_t bs, uint32_t nblocks,
                                                          float *__restrict__ ks, float *__restrict__ vs,
                                                          SealStatus *__restrict__ status) {
  const uint32_t wave = blockIdx.x * 4u + (threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63u;
  if (wave >= 2u * nblocks) return;  // uniform per wave
  const bool is_v = wave >= nblocks;
  const uint32_t b = is_v ? wave - nblocks : wave;
  const float *src = is_v ? v : k;
  const uint32_t begin = b * bs;
  const uint32_t end = min(begin + bs, values);
  float amax = 0.0f;
  uint32_t nan = 0, inf = 0;
  for (uint32_t i = begin + lane; i < end; i += 64u) {
    const float x = src[i];
    nan += (x != x);
    inf += (fabsf(x) == __builtin_huge_valf());
    amax = fmaxf(amax, fabsf(x));
  }
  for (int off = 32; off > 0; off >>= 1) {
    amax = fmaxf(amax, __shfl_xor(amax, off));
    nan += __shfl_xor(nan, off);
    inf += __shfl_xor(inf, off);
  }
  if (lane == 0) {
    (is_v ? vs : ks)[b] = amax > 0.0f ? amax / 7.0f : 1.0f;
    if (nan) atomicAdd(&status->nan_values, static_cast<unsigned long long>(nan));
    if (inf) atomicAdd(&status->inf_values, static_cast<unsigned long long>(inf));
  }
}

// One lane per 8 values (one 32-bit word of each payload).
__global__ __launch_bounds__(256) void pack_kernel(const float *__restrict__ k, const float *__restrict__ v,
                                                   uint32_t values, uint32_t bs, const float *__restrict__ ks,
                                                   const float *__restrict__ vs, uint32_t *__restrict__ kp,
                                                   uint32_t *__restrict__ vp, SealStatus *__restrict__ status) {
  const uint32_t w = blockIdx.x * 256u + threadIdx.x;
  uint32_t sat = 0;
  if (w < values / 8u) {
    const uint32_t first = w * 8u;
    uint32_t blk0 = first / bs;
    uint32_t rem0 = first - blk0 * bs;
#pragma unroll
    for (int stream = 0; stream < 2; ++stream) {
      const float *src = stream ? v : k;
      const float *sc = stream ? vs : ks;
      const float4 a = reinterpret_cast<const float4 *>(src)[2u * w];
      const float4 c = reinterpret_cast<const float4 *>(src)[2u * w + 1u];
      const float x[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
      uint32_t blk = blk0, rem = rem0;
      float scale = sc[blk];
      uint32_t word = 0;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (rem == bs) {  // next block starts inside this word (block_size not a multiple of 8)
          ++blk;
          rem = 0;
          scale = sc[blk];
        }
        int q = static_cast<int>(rintf(x[e] / scale));
        if (q < -8) { q = -8; ++sat; }
        if (q > 7) { q = 7; ++sat; }
        word |= static_cast<uint32_t>(q + 8) << (4 * e);
        ++rem;
      }
      (stream ? vp : kp)[w] = word;
    }
  }
  for (int off = 32; off > 0; off >>= 1) sat += __shfl_xor(sat, off);
  if ((threadIdx.x & 63u) == 0 && sat) atomicAdd(&status->saturated, static_cast<unsigned long long>(sat));
}

__global__ __launch_bounds__(256) void clear_status_kernel(SealStatus *status, uint32_t count) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i < count) status[i] = SealStatus{0, 0, 0};
}

__global__ __launch_bounds__(256) void convert_kernel(cf_device_tensor_view view, float *__restrict__ dst,
                                                      uint32_t dst_token) {
  const uint64_t n = uint64_t(view.token_count) * view.head_count * view.head_dim;
  const uint64_t i = uint64_t(blockIdx.x) * 256u + threadIdx.x;
  if (i >= n) return;
  const uint32_t d = static_cast<uint32_t>(i % view.head_dim);
  const uint64_t r = i / view.head_dim;
  const uint32_t h = static_cast<uint32_t>(r % view.head_count);
  const uint32_t t = static_cast<uint32_t>(r / view.head_count);
  const float x = load_scalar(view.data, view.scalar_type,
                              t * view.token_stride_bytes + h * view.head_stride_bytes + d * view.element_stride_bytes);
  dst[(uint64_t(dst_token + t) * view.head_count + h) * view.head_dim + d] = x;
}

// ------------------------------------------------------------------------------------------------ attention
template <int CTRL>
__device__ inline float dpp_mov(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xf, 0xf, false));
}

// Sum over the LG aligned lanes of a row; every lane of the row receives the total.
template <int LG>
__device__ inline float row_sum(float x) {
  if constexpr (LG >= 2) x += dpp_mov<0xb1>(x);   // quad_perm [1,0,3,2]
  if constexpr (LG >= 4) x += dpp_mov<0x4e>(x);   // quad_perm [2,3,0,1]
  if constexpr (LG >= 8) x += dpp_mov<0x141>(x);  // row_half_mirror
  if constexpr (LG >= 16) x += dpp_mov<0x140>(x); // row_mirror
  if constexpr (LG >= 32) x += __shfl_xor(x, 16);
  return x;
}

// Position of dim e (0..7) of a lane's word in the decode order: even dims (low nibbles) first.
__device__ constexpr int nib_pos(int e) { return (e & 1) ? 4 + (e >> 1) : (e >> 1); }

// Nibble word -> 8 symbols as floats in decode order (low nibbles of bytes 0..3, then high nibbles).
__device__ inline void unpack_word(uint32_t w, float out[8]) {
  const uint32_t lo = w & 0x0f0f0f0fu;
  const uint32_t hi = (w >> 4) & 0x0f0f0f0fu;
  out[0] = float(lo & 0xffu);
  out[1] = float((lo >> 8) & 0xffu);
  out[2] = float((lo >> 16) & 0xffu);
  out[3] = float(lo >> 24);
  out[4] = float(hi & 0xffu);
  out[5] = float((hi >> 8) & 0xffu);
  out[6] = float((hi >> 16) & 0xffu);
  out[7] = float(hi >> 24);
}

template <int G>
struct RowState {
  float m[G], l[G], acc[G][8];
};

// One token: kf/vf in decode order. score_j = kscale * (q_j . kf - koff * qsum_j); value = vscale * (vf - voff).
template <int LG, int G>
__device__ inline void consume(RowState<G> &st, const float (&qv)[G][8], const float (&qsum)[G], const float (&kf)[8],
                               float kscale, float koff, const float (&vf)[8], float vscale, float voff, bool valid,
                               float scale_log2) {
  float s[G];
#pragma unroll
  for (int j = 0; j < G; ++j) {
    float d = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) d = fmaf(qv[j][e], kf[e], d);
    s[j] = row_sum<LG>((d - koff * qsum[j]) * kscale) * scale_log2;
    s[j] = valid ? s[j] : kNegInf;
  }
  bool grow = false;
#pragma unroll
  for (int j = 0; j < G; ++j) grow |= s[j] > st.m[j];
  if (__ballot(grow) != 0) {  // wave-uniform: raise the running maxima
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const float mn = fmaxf(st.m[j], s[j]);
      const float corr = (mn == kNegInf) ? 1.0f : __builtin_amdgcn_exp2f(st.m[j] - mn);
      st.l[j] *= corr;
#pragma unroll
      for (int e = 0; e < 8; ++e) st.acc[j][e] *= corr;
      st.m[j] = mn;
    }
  }
  float vv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) vv[e] = vf[e] - voff;
#pragma unroll
  for (int j = 0; j < G; ++j) {
    const float p = (s[j] == kNegInf) ? 0.0f : __builtin_amdgcn_exp2f(s[j] - st.m[j]);
    st.l[j] += p;
    const float pv = p * vscale;
#pragma unroll
    for (int e = 0; e < 8; ++e) st.acc[j][e] = fmaf(pv, vv[e], st.acc[j][e]);
  }
}

// Visible positions [lo, hi] of query position qpos: p <= q and, with a window, p + window > q; with kOpenWindow
// every p except those with window > 0 and p + window < q.
struct Visible {
  uint32_t lo, hi;
  __device__ bool operator()(uint32_t pos) const { return pos >= lo && pos <= hi; }
};
__device__ inline Visible visible_range(uint32_t qpos, uint32_t window, uint32_t flags) {
  if (flags & kOpenWindow) return {window != 0u && qpos >= window ? qpos - window : 0u, 0xFFFFFFFFu};
  return {window != 0u && qpos >= window ? qpos - window + 1u : 0u, qpos};
}

template <int LG, int G>
__global__ __launch_bounds__(256) void nib_attn_kernel(const AttnItem *__restrict__ items, AttnShape sh, uint32_t hw,
                                                       uint32_t hgroups, uint32_t qchunks, float *__restrict__ ws) {
  const AttnItem &it = items[blockIdx.z];
  const uint32_t split = blockIdx.x;
  if (split >= it.nsplit) return;
  // splits [0, vbase) are the MFMA kernel's, then vsplits page splits of this kernel, then the active page
  const uint32_t vbase = it.mfma_nb ? it.page_splits : 0u;
  if (split < vbase) return;  // the MFMA kernel reads these pages
  const uint32_t per_tok = hgroups * qchunks;
  const uint32_t qt = blockIdx.y / per_tok;
  if (qt >= it.q_tokens) return;
  const uint32_t rest = blockIdx.y - qt * per_tok;
  const uint32_t hg = rest / qchunks;
  const uint32_t qc = rest - hg * qchunks;
  const uint32_t unit = threadIdx.x / LG;
  const uint32_t c = threadIdx.x % LG;
  const uint32_t D = sh.head_dim, kvh = sh.kv_heads, gqa = sh.gqa;
  const uint32_t h = hg * hw + unit;
  const bool lane_ok = h < kvh && 8u * c < D;
  const uint32_t j0 = qc * G;
  const uint32_t qpos = it.q_begin + qt;
  const float scale_log2 = it.scale_log2;
  const uint32_t flags = it.flags;
  const Visible key_visible = visible_range(qpos, it.window, flags);
  const uint32_t sx = (flags & kSignedNibbles) ? 0x88888888u : 0u;  // n ^ 8 - 8 is the two's-complement value

  float qv[G][8], qsum[G];
#pragma unroll
  for (int j = 0; j < G; ++j) {
    const bool ok = lane_ok && j0 + j < gqa;
    const uint64_t qoff = uint64_t(qt) * it.q_token_stride + uint64_t(h * gqa + j0 + j) * it.q_head_stride;
    qsum[j] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = ok ? load_scalar(it.q, it.q_type, qoff + uint64_t(8u * c + e) * it.q_elem_stride) : 0.0f;
      qv[j][nib_pos(e)] = x;
      qsum[j] += x;
    }
  }
  RowState<G> st;
#pragma unroll
  for (int j = 0; j < G; ++j) {
    st.m[j] = kNegInf;
    st.l[j] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) st.acc[j][e] = 0.0f;
  }

  const uint32_t words_per_token = kvh * (D / 8u);
  const uint32_t lane_word = h * (D / 8u) + c;
  if (split < vbase + it.vsplits) {
    const uint32_t p0 = (split - vbase) * it.vunits;
    const uint32_t p_end = min(it.page_count, p0 + it.vunits);
    // with the MFMA kernel on the request, only the pages it refuses: each lane of wave 0 tests one page of the
    // split (vunits is the lane count of wave 0, at most 64). The workgroup is hw * LG threads, which need not be
    // whole waves (5 KV heads of 16 lanes make 80), so a later wave may have fewer lanes than the split has pages:
    // wave 0's ballot reaches every wave through LDS.
    uint64_t mine = ~0ull;
    if (it.mfma_nb) {
      __shared__ uint64_t s_refused;
      if (threadIdx.x < 64u) {
        const uint32_t pl = p0 + threadIdx.x;
        bool refused = false;
        if (pl < p_end) {
          const cf_device_page_descriptor &q = it.pages[pl];
          refused = !mfma_page_ok(q.key_payload, q.value_payload, q.key_scales, q.value_scales, q.block_size,
                                  q.head_dim, q.token_count, it.mfma_cap);
        }
        const uint64_t b = __ballot(refused);
        if (threadIdx.x == 0u) s_refused = b;
      }
      __syncthreads();  // the branches above are uniform over the workgroup (blockIdx and the item only)
      mine = s_refused;
    }
    for (uint32_t p = p0; p < p_end; ++p) {
      if (!((mine >> (p - p0)) & 1ull)) continue;  // wave-uniform
      const cf_device_page_descriptor &pg = it.pages[p];
      const uint32_t tcount = pg.token_count, tbegin = pg.token_begin, bs = pg.block_size;
      const uint32_t *kw = reinterpret_cast<const uint32_t *>(pg.key_payload);
      const uint32_t *vw = reinterpret_cast<const uint32_t *>(pg.value_payload);
      const float *ksc = pg.key_scales;
      const float *vsc = pg.value_scales;
      if (!kw || !vw || !ksc || !vsc || bs == 0u) continue;
      const bool row_blocks = (flags & kRowBlocks) != 0u;
      const uint32_t bpr = row_blocks ? (pg.head_dim + bs - 1u) / bs : 0u;  // blocks per (token, KV head) row
      if ((bs & 7u) == 0u && (!row_blocks || (pg.head_dim == D && D % bs == 0u))) {  // flat index / bs is the block
        const uint32_t bw = bs / 8u;  // words per block
        for (uint32_t t0 = 0; t0 < tcount; t0 += 4u) {
          uint32_t kwv[4], vwv[4];
          float kss[4], vss[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const uint32_t tok = t0 + u;
            const bool ok = lane_ok && tok < tcount;
            const uint32_t wi = tok * words_per_token + lane_word;
            const uint32_t blk = wi / bw;
            kwv[u] = ok ? kw[wi] ^ sx : 0x88888888u;
            vwv[u] = ok ? vw[wi] ^ sx : 0x88888888u;
            kss[u] = ok ? ksc[blk] : 0.0f;
            vss[u] = ok ? vsc[blk] : 0.0f;
          }
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const uint32_t tok = t0 + u;
            if (tok >= tcount) break;  // uniform across the workgroup
            float kf[8], vf[8];
            unpack_word(kwv[u], kf);
            unpack_word(vwv[u], vf);
            consume<LG, G>(st, qv, qsum, kf, kss[u], 8.0f, vf, vss[u], 8.0f, key_visible(tbegin + tok), scale_log2);
          }
        }
      } else {  // block boundaries inside a word, or per-row blocks: dequantise value by value
        for (uint32_t tok = 0; tok < tcount; ++tok) {
          const uint32_t wi = tok * words_per_token + lane_word;
          float kf[8], vf[8], kraw[8], vraw[8];
          unpack_word(lane_ok ? kw[wi] ^ sx : 0x88888888u, kraw);
          unpack_word(lane_ok ? vw[wi] ^ sx : 0x88888888u, vraw);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const uint32_t blk = row_blocks ? (tok * kvh + h) * bpr + (8u * c + e) / bs : (wi * 8u + e) / bs;
            const int pos = nib_pos(e);
            kf[pos] = (kraw[pos] - 8.0f) * (lane_ok ? ksc[blk] : 0.0f);
            vf[pos] = (vraw[pos] - 8.0f) * (lane_ok ? vsc[blk] : 0.0f);
          }
          consume<LG, G>(st, qv, qsum, kf, 1.0f, 0.0f, vf, 1.0f, 0.0f, key_visible(tbegin + tok), scale_log2);
        }
      }
    }
  } else {  // the active fp32 page
    const uint32_t n = it.active_count;
    for (uint32_t tok = 0; tok < n; ++tok) {
      float kf[8], vf[8];
      if (lane_ok) {
        const uint64_t base = (uint64_t(tok) * kvh + h) * D + 8u * c;
        const float4 a = *reinterpret_cast<const float4 *>(it.active_k + base);
        const float4 b = *reinterpret_cast<const float4 *>(it.active_k + base + 4);
        const float4 x = *reinterpret_cast<const float4 *>(it.active_v + base);
        const float4 y = *reinterpret_cast<const float4 *>(it.active_v + base + 4);
        kf[0] = a.x; kf[1] = a.z; kf[2] = b.x; kf[3] = b.z; kf[4] = a.y; kf[5] = a.w; kf[6] = b.y; kf[7] = b.w;
        vf[0] = x.x; vf[1] = x.z; vf[2] = y.x; vf[3] = y.z; vf[4] = x.y; vf[5] = x.w; vf[6] = y.y; vf[7] = y.w;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) kf[e] = vf[e] = 0.0f;
      }
      consume<LG, G>(st, qv, qsum, kf, 1.0f, 0.0f, vf, 1.0f, 0.0f, key_visible(it.active_begin + tok), scale_log2);
    }
  }

  // partial row: acc[0..D) in dim order, m at [D], l at [D + 1]
  const uint32_t stride = D + 4u;
  float *base = ws + it.ws_offset + (uint64_t(split) * it.q_tokens + qt) * sh.q_heads * stride;
#pragma unroll
  for (int j = 0; j < G; ++j) {
    if (!(h < kvh && j0 + j < gqa)) continue;
    float *row = base + uint64_t(h * gqa + j0 + j) * stride;
    if (c == 0) {
      row[D] = st.m[j];
      row[D + 1] = st.l[j];
    }
    if (8u * c < D) {
      float4 a, b;
      a.x = st.acc[j][nib_pos(0)]; a.y = st.acc[j][nib_pos(1)]; a.z = st.acc[j][nib_pos(2)]; a.w = st.acc[j][nib_pos(3)];
      b.x = st.acc[j][nib_pos(4)]; b.y = st.acc[j][nib_pos(5)]; b.z = st.acc[j][nib_pos(6)]; b.w = st.acc[j][nib_pos(7)];
      *reinterpret_cast<float4 *>(row + 8u * c) = a;
      *reinterpret_cast<float4 *>(row + 8u * c + 4u) = b;
    }
  }
}

// One wave per (query head, query token, item): combine the splits and store the normalised row.
__global__ __launch_bounds__(64) void nib_merge_kernel(const AttnItem *__restrict__ items, AttnShape sh,
                                                       const float *__restrict__ ws) {
  const AttnItem &it = items[blockIdx.z];
  const uint32_t qt = blockIdx.y, qh = blockIdx.x, lane = threadIdx.x;
  if (qt >= it.q_tokens) return;
  const uint32_t D = sh.head_dim, stride = D + 4u;
  const float *row0 = ws + it.ws_offset + (uint64_t(qt) * sh.q_heads + qh) * stride;
  const uint64_t split_stride = uint64_t(it.q_tokens) * sh.q_heads * stride;
  const uint32_t ns = it.nsplit;
  constexpr uint32_t kB = 8;  // splits whose loads are in flight together
  float M = kNegInf;
  for (uint32_t s0 = 0; s0 < ns; s0 += kB) {  // the maxima, kB loads at a time (past the end: the last split again)
    float mv[kB];
#pragma unroll
    for (uint32_t u = 0; u < kB; ++u) mv[u] = row0[min(s0 + u, ns - 1u) * split_stride + D];
#pragma unroll
    for (uint32_t u = 0; u < kB; ++u) M = fmaxf(M, mv[u]);
  }
  float L = 0.0f, o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  // splits in ascending order (the same sums in the same order for any grouping); kB splits' loads are issued
  // together so that their latencies overlap, and a split with nothing attended (m = -inf) changes nothing
  auto add = [&](float ms, float ls, const float (&v)[4]) {
    if (ms == kNegInf) return;
    const float w = __builtin_amdgcn_exp2f(ms - M);
    L = fmaf(w, ls, L);
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = fmaf(w, v[k], o[k]);
  };
  auto load = [&](uint32_t s, float &ms, float &ls, float (&v)[4]) {
    const float *row = row0 + s * split_stride;
    ms = row[D];
    ls = row[D + 1];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t d = lane + 64u * k;
      v[k] = d < D ? row[d] : 0.0f;
    }
  };
  if (M != kNegInf) {
    for (uint32_t s0 = 0; s0 < ns; s0 += kB) {
      float ms[kB], ls[kB], v[kB][4];
#pragma unroll
      for (uint32_t u = 0; u < kB; ++u) load(min(s0 + u, ns - 1u), ms[u], ls[u], v[u]);
#pragma unroll
      for (uint32_t u = 0; u < kB; ++u)
        if (s0 + u < ns) add(ms[u], ls[u], v[u]);
    }
  }
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  const uint64_t obase = uint64_t(qt) * it.o_token_stride + uint64_t(qh) * it.o_head_stride;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t d = lane + 64u * k;
    if (d < D) store_scalar(it.out, it.o_type, obase + uint64_t(d) * it.o_elem_stride, o[k] * inv);
  }
}

template <int LG, int G>
hipError_t launch_attn_lg_g(dim3 grid, dim3 block, hipStream_t s, const AttnItem *items, const AttnShape &sh,
                            uint32_t hw, uint32_t hgroups, uint32_t qchunks, float *ws) {
  nib_attn_kernel<LG, G><<<grid, block, 0, s>>>(items, sh, hw, hgroups, qchunks, ws);
  return hipPeekAtLastError();
}

template <int LG>
hipError_t launch_attn_lg(uint32_t G, dim3 grid, dim3 block, hipStream_t s, const AttnItem *items,
                          const AttnShape &sh, uint32_t hw, uint32_t hgroups, uint32_t qchunks, float *ws) {
  switch (G) {
    case 1: return launch_attn_lg_g<LG, 1>(grid, block, s, items, sh, hw, hgroups, qchunks, ws);
    case 2: return launch_attn_lg_g<LG, 2>(grid, block, s, items, sh, hw, hgroups, qchunks, ws);
    default: return launch_attn_lg_g<LG, 4>(grid, block, s, items, sh, hw, hgroups, qchunks, ws);
  }
}

}  // namespace

hipError_t launch_block_scales(const float *k, const float *v, uint32_t values, uint32_t block_size, float *k_scales,
                               float *v_scales, SealStatus *status, hipStream_t stream) {
  const uint32_t nblocks = (values + block_size - 1u) / block_size;
  const uint32_t waves = 2u * nblocks;
  block_scale_kernel<<<(waves + 3u) / 4u, 256, 0, stream>>>(k, v, values, block_size, nblocks, k_scales, v_scales,
                                                            status);
  return hipPeekAtLastError();
}

hipError_t launch_pack(const float *k, const float *v, uint32_t values, uint32_t block_size, const float *k_scales,
                       const float *v_scales, uint8_t *k_payload, uint8_t *v_payload, SealStatus *status,
                       hipStream_t stream) {
  const uint32_t words = values / 8u;
  pack_kernel<<<(words + 255u) / 256u, 256, 0, stream>>>(k, v, values, block_size, k_scales, v_scales,
                                                         reinterpret_cast<uint32_t *>(k_payload),
                                                         reinterpret_cast<uint32_t *>(v_payload), status);
  return hipPeekAtLastError();
}

hipError_t launch_convert(const cf_device_tensor_view &src, float *dst, uint32_t dst_token, hipStream_t stream) {
  const uint64_t n = uint64_t(src.token_count) * src.head_count * src.head_dim;
  if (n == 0) return hipSuccess;
  convert_kernel<<<static_cast<unsigned>((n + 255u) / 256u), 256, 0, stream>>>(src, dst, dst_token);
  return hipPeekAtLastError();
}

hipError_t launch_clear_status(SealStatus *status, uint32_t count, hipStream_t stream) {
  clear_status_kernel<<<(count + 255u) / 256u, 256, 0, stream>>>(status, count);
  return hipPeekAtLastError();
}

AttnRunner::~AttnRunner() {
  if (ws_) (void)hipFree(ws_);
}

hipError_t AttnRunner::run(const std::vector<AttnRequest> &reqs, const AttnShape &sh, hipStream_t stream,
                           std::string &error) {
  launches_ = 0;
  if (reqs.empty()) return hipSuccess;
  const uint32_t D = sh.head_dim;
  uint32_t lg = 4;
  while (lg * 8u < D) lg *= 2u;
  // at most 4 query heads per lane: 8 would need every VGPR and AGPR of the SIMD lane (one wave per SIMD)
  const uint32_t G = sh.gqa <= 1u ? 1u : sh.gqa <= 2u ? 2u : 4u;
  const uint32_t qchunks = (sh.gqa + G - 1u) / G;
  const uint32_t hw = std::min(sh.kv_heads, 256u / lg);
  const uint32_t hgroups = (sh.kv_heads + hw - 1u) / hw;

  // context splits: aim at about 2048 workgroups over the whole batch
  uint64_t page_work = 0, tile_work = 0;
  const uint32_t cpp = (sh.page_size + 15u) / 16u;  // 16-token chunks per page (MFMA kernel)
  std::vector<uint32_t> nb(reqs.size());
  for (size_t i = 0; i < reqs.size(); ++i) {
    const auto &r = reqs[i];
    // batched-items requests (the contract's three flags) run on the MFMA kernel in its per-page mode when
    // head_dim is 128 and pages have a planned size; other flagged requests stay on the VALU kernel
    nb[i] = r.flags == kContractFlags ? (D == 128u && cpp > 0u ? kMfmaContract : 0u)
                                      : r.flags ? 0u : mfma_sets(D, r.block_size);
    if (nb[i]) tile_work += uint64_t((r.page_count * cpp + 3u) / 4u) * r.query.token_count * ((sh.gqa + 3u) / 4u);
    else page_work += uint64_t(r.page_count) * r.query.token_count * hgroups * qchunks;
  }
  const uint32_t pps = static_cast<uint32_t>(std::clamp<uint64_t>((page_work + 2047u) / 2048u, 1u, 64u));
  // the MFMA kernel's workgroups take four 64-slot tiles per round (one per wave), KV head by KV head
  const uint32_t tps = static_cast<uint32_t>(
      std::clamp<uint64_t>((tile_work * sh.kv_heads + 2047u) / 2048u, 4u, 256u));

  std::vector<AttnItem> items(reqs.size());
  uint64_t floats = 0;
  uint32_t max_split = 1, max_qtok = 1, max_mfma_split = 0;
  bool any_nb[5] = {false, false, false, false, false};
  const uint32_t wave_lanes = std::min(64u, hw * lg);  // lanes of the VALU kernel's first wave
  for (size_t i = 0; i < reqs.size(); ++i) {
    const AttnRequest &r = reqs[i];
    AttnItem &it = items[i];
    it.q = r.query.data;
    it.q_token_stride = r.query.token_stride_bytes;
    it.q_head_stride = r.query.head_stride_bytes;
    it.q_elem_stride = r.query.element_stride_bytes;
    it.q_type = r.query.scalar_type;
    it.q_tokens = r.query.token_count;
    it.out = r.output;
    it.o_token_stride = r.o_token_stride;
    it.o_head_stride = r.o_head_stride;
    it.o_elem_stride = r.o_elem_stride;
    it.o_type = r.output_type;
    it.pages = r.pages;
    it.page_count = r.page_count;
    it.mfma_nb = nb[i];
    if (nb[i]) {
      const uint32_t tiles = (r.page_count * cpp + 3u) / 4u;
      it.units_per_split = tps;
      it.page_splits = (tiles + tps - 1u) / tps;
      max_mfma_split = std::max(max_mfma_split, it.page_splits);
      any_nb[nb[i]] = true;
      it.vunits = nb[i] == kMfmaContract ? wave_lanes : 0u;  // one lane per page tests it
      it.vsplits = it.vunits ? (r.page_count + it.vunits - 1u) / it.vunits : 0u;
      it.mfma_cap = 16u * cpp;
    } else {
      it.units_per_split = pps;
      it.page_splits = (r.page_count + pps - 1u) / pps;
      it.vunits = pps;
      it.vsplits = it.page_splits;
      it.mfma_cap = 0u;
    }
    it.active_k = r.active_k;
    it.active_v = r.active_v;
    it.active_begin = r.active_begin;
    it.active_count = r.active_k ? r.active_count : 0u;
    it.q_begin = r.query_begin;
    it.window = r.window;
    it.scale_log2 = r.softmax_scale * 1.4426950408889634f;
    it.flags = r.flags;
    it.nsplit = (it.mfma_nb ? it.page_splits : 0u) + it.vsplits + (it.active_count > 0u ? 1u : 0u);
    if (it.nsplit == 0u) it.nsplit = 1u;  // nothing visible: one empty split, the row comes out 0
    it.ws_offset = floats;
    floats += uint64_t(it.nsplit) * it.q_tokens * sh.q_heads * (D + 4u);
    max_split = std::max(max_split, it.nsplit);
    max_qtok = std::max(max_qtok, it.q_tokens);
  }
  const uint64_t ydim = uint64_t(max_qtok) * hgroups * qchunks;
  if (ydim > 65535u || reqs.size() > 65535u || max_split > 0x7fffffffu) {
    error = "attention batch exceeds the launch grid (too many query tokens or items in one call)";
    return hipErrorInvalidValue;
  }
  const uint64_t table_bytes = (items.size() * sizeof(AttnItem) + 255u) & ~uint64_t(255);
  const uint64_t need = table_bytes + floats * sizeof(float);
  if (need > bytes_) {
    if (ws_) {
      hipError_t e = hipStreamSynchronize(stream);  // earlier launches on this stream may still read the old buffer
      if (e != hipSuccess) return e;
      (void)hipFree(ws_);
      ws_ = nullptr;
      bytes_ = 0;
    }
    const uint64_t grow = std::max<uint64_t>(need, 1u << 20);
    hipError_t e = hipMalloc(&ws_, grow);
    if (e != hipSuccess) {
      ws_ = nullptr;
      error = "attention workspace allocation failed";
      return e;
    }
    bytes_ = grow;
  }
  hipError_t e = hipMemcpyAsync(ws_, items.data(), items.size() * sizeof(AttnItem), hipMemcpyHostToDevice, stream);
  if (e != hipSuccess) return e;
  const AttnItem *d_items = static_cast<const AttnItem *>(ws_);
  float *partials = reinterpret_cast<float *>(static_cast<char *>(ws_) + table_bytes);
  const dim3 grid(max_split, static_cast<uint32_t>(ydim), static_cast<uint32_t>(items.size()));
  const dim3 block(hw * lg);
  // the VALU kernel serves items without the MFMA path, every active page and every item with nothing visible
  bool valu_work = false;
  for (const AttnItem &it : items) valu_work = valu_work || !it.mfma_nb || it.nsplit > it.page_splits;
  if (valu_work) switch (lg) {
    case 4: e = launch_attn_lg<4>(G, grid, block, stream, d_items, sh, hw, hgroups, qchunks, partials); break;
    case 8: e = launch_attn_lg<8>(G, grid, block, stream, d_items, sh, hw, hgroups, qchunks, partials); break;
    case 16: e = launch_attn_lg<16>(G, grid, block, stream, d_items, sh, hw, hgroups, qchunks, partials); break;
    default: e = launch_attn_lg<32>(G, grid, block, stream, d_items, sh, hw, hgroups, qchunks, partials); break;
  }
  if (e != hipSuccess) return e;
  for (uint32_t n : {1u, 2u, kMfmaContract, 4u}) {
    if (!any_nb[n]) continue;
    e = launch_nib_mfma(n, d_items, static_cast<uint32_t>(items.size()), max_mfma_split, max_qtok, sh, partials,
                        stream);
    if (e != hipSuccess) return e;
  }
  nib_merge_kernel<<<dim3(sh.q_heads, max_qtok, static_cast<uint32_t>(items.size())), 64, 0, stream>>>(d_items, sh,
                                                                                                     partials);
  e = hipPeekAtLastError();
  if (e == hipSuccess) launches_ = 2;
  return e;
}

}  // namespace cfnib
