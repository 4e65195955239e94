// kv_legacy.hip — the reference's single-sequence paged-KV seam on gfx950 (include/chromofold/kv_cuda.h).
//
// Replaces reference src/cuda/paged_kv_attention.cu:41-327 (cf_kv_validate_paged_attention_desc,
// cf_kv_paged_attention_async) with identical validation rules and result semantics:
//   * query row r is token query_token_begin + r; it attends tokens in [window_begin, query_token] of every page
//     whose kv_head matches (query head h reads KV head h / gqa_group_size) and of the dense fp32 active tail;
//   * K value = (sym - zero_point) * k_scales[dim], V value = (sym - zero_point) * v_scales[token];
//   * online softmax in fp32 across all pages and the tail (pages are never normalised separately);
//   * a (row, head) with no visible token gets zeros.
// Codecs per page: fixed_code_length > 0 = fixed-width MSB-first codes; 0 = canonical-Huffman LUT codes
// (lut[look] = sym | len << 8 over max_code_length lookahead bits, reference
// include/chromofold/detail/block_huffman_device.cuh:12-19) with block_offsets every block_size symbols. The
// reference routes any head_dim % 32 == 0 page to a fixed-width-only kernel even when it is Huffman coded (its
// warp kernel shifts by 32 - 0); here every page is decoded by its own codec.
// rANS pages (fixed_code_length == 0 and k_max_code_length == 0, an additive tag of this build): k_words points at
// one kv_codec_ext.h group blob coded on its own (a chain start: it holds its lane states) of up to 64 tokens, k_lut
// and v_lut at the K and V decode tables (CF_KV_RANS_TABLE_BYTES each); the scales come from the blob header (per
// 16-token page) and the other page fields are not read. The wavefront decodes the group into the same LDS symbol
// tiles as the other codecs (offset binary, zero point 128) and applies the K scale per token to the scores. A blob
// that continues a chain, whose header disagrees with the page (head_dim, token counts, page gaps) or whose rANS
// chain does not end where the encoder started makes that (query row, KV head) NaN.
//
// Layout on gfx950: one wavefront per (query row, KV head) serves all gqa query heads of that KV head, so each
// page is decoded once per row instead of once per query head. The wavefront decodes a chunk of the page's K and V
// symbols into LDS (fixed-width: lane-strided random access; Huffman: one lane per code block, skip-decoding to
// the chunk start, with the page's LUTs staged in LDS), then lane = token computes the scores of the chunk for every query head, the wavefront
// folds them into the running (max, sum), and lane = dims accumulates the V rows. Nothing decoded leaves the CU.
#include <cmath>
#include <utility>

#include "cf_device.hpp"
#include "chromofold/kv_codec_ext.h"
#include "chromofold/kv_cuda.h"
#include "kv_group_decode.hpp"

namespace {

constexpr int kLanes = 64;
constexpr int kChunkSyms = 8192;  // symbols of K (and of V) staged per chunk: 64 tokens at head_dim 128
constexpr int kRowPad = 4;        // bytes added to each staged row
constexpr int kHeadsPass = 8;     // query heads served per pass over the pages
constexpr int kLutMaxLen = 12;    // Huffman LUTs of up to 2^12 entries are staged in LDS

// canonical-Huffman LUT decode at bit `pos` (MSB-first), returns sym | len << 8
__device__ __forceinline__ int huff_at(const uint32_t *__restrict__ words, const int32_t *__restrict__ lut, int maxlen,
                                       int64_t pos) {
  const int64_t wi = pos >> 5;
  const int b = static_cast<int>(pos & 31);
  uint64_t v = static_cast<uint64_t>(words[wi]) << 32;
  if (b + maxlen > 32) v |= words[wi + 1];
  const uint32_t look = static_cast<uint32_t>((v << b) >> (64 - maxlen));
  return lut[look];
}

// fixed-width MSB-first code of symbol i (bits dividing 32, as the reference packer writes them)
__device__ __forceinline__ int fixed_at(const uint32_t *__restrict__ words, uint32_t bits, int64_t i) {
  const int64_t bit = i * bits;
  const uint32_t w = words[bit >> 5];
  return static_cast<int>((w >> ((32u - bits) - static_cast<uint32_t>(bit & 31))) & ((1u << bits) - 1u));
}

// Decode symbols [s0, s1) of one stream (rows of hd symbols) into dst, row r at dst + r * stride (a padded row
// stride keeps the lane-per-token reads of the scoring loop off a single LDS bank).
__device__ void decode_span(const uint32_t *__restrict__ words, const int32_t *__restrict__ boff,
                            const int32_t *__restrict__ lut, uint32_t maxlen, uint32_t fixed_bits, uint32_t block,
                            int64_t s0, int64_t s1, uint32_t hd, uint32_t stride, uint8_t *__restrict__ dst, int lane) {
  auto put = [&](int64_t i, int sym) {
    const uint32_t rel = static_cast<uint32_t>(i - s0), r = rel / hd;
    dst[r * stride + (rel - r * hd)] = static_cast<uint8_t>(sym);
  };
  if (fixed_bits) {
    for (int64_t i = s0 + lane; i < s1; i += kLanes) put(i, fixed_at(words, fixed_bits, i));
    return;
  }
  // Huffman: one lane per code block intersecting [s0, s1); skip-decode up to s0 inside the first block
  const int64_t b0 = s0 / block, b1 = (s1 + block - 1) / block;
  for (int64_t b = b0 + lane; b < b1; b += kLanes) {
    int64_t pos = boff[b];
    const int64_t first = b * block, last = min(first + static_cast<int64_t>(block), s1);
    for (int64_t i = first; i < last; ++i) {
      const int e = huff_at(words, lut, static_cast<int>(maxlen), pos);
      pos += e >> 8;
      if (i >= s0) put(i, e & 0xff);
    }
  }
}

// ---- rANS pages (kv_codec_ext.h format 4)
constexpr uint32_t kRansWords = CF_KV_RANS_MAX_GROUP_WORDS + 64;  // staged K+V words + slack for idle lanes' reads

// Sign-magnitude bytes (mag: |q|, signs: 0x80 per negative byte) -> offset-binary symbols q + 128, per byte.
__device__ __forceinline__ uint32_t sm_to_offset_binary(uint32_t mag, uint32_t signs) {
  const uint32_t neg = mag & ((signs >> 7) * 0xFFu);  // |q| of the negative bytes
  return 0x80808080u + mag - (neg << 1);              // 128 + |q| or 128 - |q|, no carry between bytes
}

// Decode one self-contained group blob (RANS_HYBRID chain start, or the INT8 raw fallback) of `ntok` tokens and
// head_dim hd (% 16 == 0, % 32 for RANS) into dk[token * stride + dim] / dv[token * stride + dim] as offset-binary
// symbols, with the per-token K and V scales in kt / vt. A RANS group's K and V tables (ktab, vtab in HBM; not read
// for an INT8 group) are staged in `tab` (LDS), its word streams in `s_w`.
// Returns false (wave-uniform) when the blob is not a valid self-contained group for this page.
__device__ bool rans_group_to_lds(const uint8_t *__restrict__ blob, const uint2 *__restrict__ ktab,
                                  const uint2 *__restrict__ vtab, uint2 (*tab)[cfkv::kSlots], uint16_t *s_w,
                                  uint32_t hd, uint32_t ntok, uint8_t *dk, uint8_t *dv, uint32_t stride, float *kt,
                                  float *vt, int lane) {
  const uint32_t codec = *reinterpret_cast<const uint32_t *>(blob);
  const uint32_t cnt = *reinterpret_cast<const uint32_t *>(blob + 4);
  const uint32_t chain = *reinterpret_cast<const uint16_t *>(blob + 8);
  const uint16_t *tc = reinterpret_cast<const uint16_t *>(blob + 12);
  const uint32_t D = *reinterpret_cast<const uint16_t *>(blob + 20);
  if (D != hd || hd % 16 != 0 || hd > 128) return false;
  if (codec != CF_KV_CODEC_INT8 && (codec != CF_KV_CODEC_RANS_HYBRID || hd % 32 != 0 || chain != 1)) return false;
  // tokens must be contiguous: full 16-token pages, then at most one partial page, then empty pages
  uint32_t total = 0;
  bool open = true;
  for (int G = 0; G < 4; ++G) {
    const uint32_t n = tc[G];
    if (n > 16 || (n && !open)) return false;
    if (n < 16) open = false;
    total += n;
  }
  if (total != ntok || total == 0) return false;
  const float *ks = reinterpret_cast<const float *>(blob + 32), *vs = reinterpret_cast<const float *>(blob + 48);
  kt[lane] = ks[lane >> 4];
  vt[lane] = vs[lane >> 4];
  const uint32_t NQ = hd / 4, G = static_cast<uint32_t>(lane) >> 4, t = static_cast<uint32_t>(lane) & 15;
  // V quad q of a lane = tokens 4 tq .. 4 tq + 3 of its page at dim t + 16 i (tq = q / (hd / 16), i = q % (hd / 16))
  auto put_v = [&](uint32_t q, uint32_t w) {
    const uint32_t tq = q / (hd / 16), i = q % (hd / 16);
    uint8_t *col = dv + (16 * G + 4 * tq) * stride + t + 16 * i;
#pragma unroll
    for (int j = 0; j < 4; ++j) col[j * stride] = static_cast<uint8_t>(w >> (8 * j));
  };
  if (codec == CF_KV_CODEC_INT8) {
    const uint32_t *raw = reinterpret_cast<const uint32_t *>(blob + cfkv::kHdr);
    for (uint32_t q = 0; q < NQ; ++q) {
      *reinterpret_cast<uint32_t *>(dk + lane * stride + 4 * q) = raw[q * 64 + lane];
      put_v(q, raw[(NQ + q) * 64 + lane]);
    }
    return true;
  }
  const uint32_t nk = cnt & 0xFFFFu, nv = cnt >> 16;
  if (nk + nv > CF_KV_RANS_MAX_GROUP_WORDS) return false;
  for (uint32_t i = lane; i < cfkv::kSlots; i += kLanes) {  // {f | c << 16, spread} as the decoder reads it
    const uint2 a = ktab[i], b = vtab[i];
    tab[0][i] = uint2{(a.x & 2047u) | (((a.x >> 11) & 2047u) << 16), a.y};
    tab[1][i] = uint2{(b.x & 2047u) | (((b.x >> 11) & 2047u) << 16), b.y};
  }
  const int RAW = cfkv::raw_words_of(static_cast<int>(hd));
  const uint32_t *st = reinterpret_cast<const uint32_t *>(blob + cfkv::kHdr);
  uint32_t xk = st[lane], xv = st[64 + lane];
  const uint32_t *raw = st + 2 * 64;
  // stage both word streams (u16, K then V) in LDS; whole u32 pairs (blobs are padded to 16 bytes)
  const uint32_t *wsrc = raw + 2 * RAW;
  for (uint32_t i = lane; i < (nk + nv + 1) / 2; i += kLanes) reinterpret_cast<uint32_t *>(s_w)[i] = wsrc[i];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const uint16_t *wk = s_w, *wv = s_w + nk;
  for (uint32_t sg = 0; sg < hd / 32; ++sg) {
    uint32_t wK[7], wV[7];
#pragma unroll
    for (int w = 0; w < 7; ++w) {
      wK[w] = raw[(7 * sg + w) * 64 + lane];
      wV[w] = raw[RAW + (7 * sg + w) * 64 + lane];
    }
    [&]<int... M>(std::integer_sequence<int, M...>) {
      (
          [&] {
            constexpr int m = M;
            constexpr uint32_t rA = cfkv::kFrame[2 * m], rB = cfkv::kFrame[2 * m + 1];
            constexpr int nw = cfkv::kNWord[m], cwi = m < 2 ? 2 : 5;
            const uint2 ek = cfkv::rans_lookup(tab[0], xk), ev = cfkv::rans_lookup(tab[1], xv);
            uint32_t selk, selv;
            const uint32_t wdk = cfkv::rans_advance(ek.x, xk, wk, selk);
            const uint32_t wdv = cfkv::rans_advance(ev.x, xv, wv, selv);
            xk = __builtin_amdgcn_perm(xk, wdk, selk);
            xv = __builtin_amdgcn_perm(xv, wdv, selv);
            const uint32_t spk = rA ? __builtin_amdgcn_alignbit(ek.y, ek.y, 32 - rA) : ek.y;
            const uint32_t spv = rA ? __builtin_amdgcn_alignbit(ev.y, ev.y, 32 - rA) : ev.y;
            const uint32_t q0 = 8 * sg + 2 * m;
            *reinterpret_cast<uint32_t *>(dk + lane * stride + 4 * q0) =
                sm_to_offset_binary(cfkv::quad_mag<rA>(wK[nw], wK[cwi], spk), cfkv::quad_signs<rA>(wK[6]));
            *reinterpret_cast<uint32_t *>(dk + lane * stride + 4 * (q0 + 1)) =
                sm_to_offset_binary(cfkv::quad_mag<rB>(wK[nw], wK[cwi], spk), cfkv::quad_signs<rB>(wK[6]));
            put_v(q0, sm_to_offset_binary(cfkv::quad_mag<rA>(wV[nw], wV[cwi], spv), cfkv::quad_signs<rA>(wV[6])));
            put_v(q0 + 1, sm_to_offset_binary(cfkv::quad_mag<rB>(wV[nw], wV[cwi], spv), cfkv::quad_signs<rB>(wV[6])));
          }(),
          ...);
    }(std::make_integer_sequence<int, 4>{});
  }
  // a group coded on its own ends where the encoder started (2^16 in every lane of both streams) and has consumed
  // exactly its words
  const bool ok = xk == 65536u && xv == 65536u && wk == s_w + nk && wv == s_w + nk + nv;
  return __builtin_amdgcn_ballot_w64(!ok) == 0;
}

template <int DPL>  // dims per lane: head_dim <= 64 * DPL
__global__ __launch_bounds__(kLanes) void legacy_kernel(cf_kv_paged_attention_desc d) {
  __shared__ uint8_t s_k[kChunkSyms + kLanes * kRowPad], s_v[kChunkSyms + kLanes * kRowPad];
  __shared__ float s_q[kHeadsPass][64 * DPL];
  __shared__ float s_p[kHeadsPass][kLanes];
  __shared__ float s_ks[64 * DPL];
  __shared__ __align__(16) int32_t s_lut[2][1 << kLutMaxLen];  // Huffman LUTs, or the rANS K and V tables
  __shared__ __align__(16) uint16_t s_w[kRansWords];
  __shared__ float s_kt[kLanes], s_vt[kLanes];  // rANS pages: per-token K and V scales
  static_assert(sizeof(s_lut) >= 2 * cfkv::kSlots * sizeof(uint2), "the rANS tables share the LUT area");

  const int lane = threadIdx.x;
  const uint32_t row = blockIdx.x, kvh = blockIdx.y;
  const uint32_t D = d.head_dim;
  const uint32_t gqa = d.gqa_group_size;
  const uint32_t qtok = d.query_token_begin + row;
  const uint32_t wbegin = (d.causal_window == 0 || qtok + 1 <= d.causal_window) ? 0u : qtok + 1 - d.causal_window;

  bool bad = false;  // a rANS page that is not a valid self-contained group for its descriptor (see the file header)
  for (uint32_t h0 = 0; h0 < gqa; h0 += kHeadsPass) {
    const int nh = static_cast<int>(min<uint32_t>(kHeadsPass, gqa - h0));
    // queries of this pass (softmax scale applied to the dot product, as the reference does)
    for (int i = lane; i < kHeadsPass * 64 * DPL; i += kLanes) {
      const int h = i / (64 * DPL), dd = i % (64 * DPL);
      float q = 0.0f;
      if (h < nh && static_cast<uint32_t>(dd) < D)
        q = d.queries[(static_cast<size_t>(row) * d.query_head_count + kvh * gqa + h0 + h) * D + dd];
      s_q[h][dd] = q;
    }
    float m[kHeadsPass], l[kHeadsPass], acc[kHeadsPass][DPL];
#pragma unroll
    for (int h = 0; h < kHeadsPass; ++h) {
      m[h] = -INFINITY;
      l[h] = 0.0f;
#pragma unroll
      for (int j = 0; j < DPL; ++j) acc[h][j] = 0.0f;
    }

    // fold a chunk of up to 64 tokens: lane = token scores, then lane = dims V accumulation
    auto fold = [&](int ntok, bool dense, const float *kd, const float *vd, const float *vsc, int zp,
                    uint32_t tok0, uint32_t hd, uint32_t stride, const float *kt = nullptr) {
      float sc[kHeadsPass];
      const uint32_t token = tok0 + lane;
      const bool vis = lane < ntok && token >= wbegin && token <= qtok;
#pragma unroll
      for (int h = 0; h < kHeadsPass; ++h) sc[h] = 0.0f;
      if (lane < ntok) {
        for (uint32_t dd = 0; dd < D; ++dd) {
          float kv;
          if (dense) kv = kd[(static_cast<size_t>(lane) * d.kv_head_count + kvh) * D + dd];
          else if (dd < hd) kv = static_cast<float>(static_cast<int>(s_k[lane * stride + dd]) - zp) * s_ks[dd];
          else kv = 0.0f;
#pragma unroll
          for (int h = 0; h < kHeadsPass; ++h) sc[h] += s_q[h][dd] * kv;
        }
      }
      if (kt && lane < ntok) {
#pragma unroll
        for (int h = 0; h < kHeadsPass; ++h) sc[h] *= kt[lane];
      }
#pragma unroll
      for (int h = 0; h < kHeadsPass; ++h) {
        float s = vis ? sc[h] * d.softmax_scale : -INFINITY;
        float mx = s;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        const float mn = fmaxf(m[h], mx);
        const float alpha = (m[h] == -INFINITY) ? 0.0f : expf(m[h] - mn);
        const float p = vis ? expf(s - mn) : 0.0f;
        float ps = p;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) ps += __shfl_xor(ps, o);
        if (mn != -INFINITY) {
          l[h] = l[h] * alpha + ps;
#pragma unroll
          for (int j = 0; j < DPL; ++j) acc[h][j] *= alpha;
          m[h] = mn;
        }
        s_p[h][lane] = p * (dense ? 1.0f : vsc[lane < ntok ? lane : 0]);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      for (int t = 0; t < ntok; ++t) {
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          const uint32_t dd = lane + 64 * j;
          if (dd >= D) continue;
          float vv;
          if (dense) vv = vd[(static_cast<size_t>(t) * d.kv_head_count + kvh) * D + dd];
          else if (dd < hd) vv = static_cast<float>(static_cast<int>(s_v[t * stride + dd]) - zp);
          else vv = 0.0f;
#pragma unroll
          for (int h = 0; h < kHeadsPass; ++h) acc[h][j] += s_p[h][t] * vv;
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };

    for (uint32_t p = 0; p < d.page_count; ++p) {
      if (d.pages[p].kv_head != kvh) continue;  // wave-uniform
      const cf_kv_device_page pg = d.pages[p];
      if (pg.token_count == 0) continue;
      // skip pages entirely outside the visible window
      if (pg.token_begin > qtok || pg.token_begin + pg.token_count <= wbegin) continue;
      if (pg.fixed_code_length == 0 && pg.k_max_code_length == 0) {  // rANS page (kv_codec_ext.h group blob)
        if (pg.token_count > static_cast<uint32_t>(kLanes) || pg.head_dim > D) {
          bad = true;
          continue;
        }
        for (uint32_t dd = lane; dd < D; dd += kLanes) s_ks[dd] = 1.0f;
        uint2(*tab)[cfkv::kSlots] = reinterpret_cast<uint2(*)[cfkv::kSlots]>(&s_lut[0][0]);
        const uint32_t stride = pg.head_dim + kRowPad;
        if (!rans_group_to_lds(reinterpret_cast<const uint8_t *>(pg.k_words),
                               reinterpret_cast<const uint2 *>(pg.k_lut), reinterpret_cast<const uint2 *>(pg.v_lut),
                               tab, s_w, pg.head_dim, pg.token_count, s_k, s_v, stride, s_kt, s_vt, lane)) {
          bad = true;
          continue;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        fold(static_cast<int>(pg.token_count), false, nullptr, nullptr, s_vt, 128, pg.token_begin, pg.head_dim,
             stride, s_kt);
        continue;
      }
      for (uint32_t dd = lane; dd < min(D, pg.head_dim); dd += kLanes) s_ks[dd] = pg.k_scales[dd];
      if (pg.head_dim == 0 || pg.head_dim > CF_KV_MAX_HEAD_DIM) continue;
      // Huffman pages: stage both LUTs in LDS when they fit (the lookups are the decoder's hot loop)
      const int32_t *klut = pg.k_lut, *vlut = pg.v_lut;
      if (!pg.fixed_code_length && pg.k_max_code_length <= kLutMaxLen && pg.v_max_code_length <= kLutMaxLen) {
        for (uint32_t i = lane; i < (1u << pg.k_max_code_length); i += kLanes) s_lut[0][i] = pg.k_lut[i];
        for (uint32_t i = lane; i < (1u << pg.v_max_code_length); i += kLanes) s_lut[1][i] = pg.v_lut[i];
        klut = s_lut[0];
        vlut = s_lut[1];
      }
      const uint32_t chunk = max(1u, min<uint32_t>(kLanes, kChunkSyms / pg.head_dim));
      for (uint32_t t0 = 0; t0 < pg.token_count; t0 += chunk) {
        const uint32_t nt = min(chunk, pg.token_count - t0);
        // chunk symbols [t0*hd, (t0+nt)*hd) of each stream; lane-token t reads row t at t*hd (page row stride)
        const int64_t s0 = static_cast<int64_t>(t0) * pg.head_dim, s1 = s0 + static_cast<int64_t>(nt) * pg.head_dim;
        const uint32_t stride = pg.head_dim + kRowPad;
        decode_span(pg.k_words, pg.k_block_offsets, klut, pg.k_max_code_length, pg.fixed_code_length,
                    pg.block_size, s0, s1, pg.head_dim, stride, s_k, lane);
        decode_span(pg.v_words, pg.v_block_offsets, vlut, pg.v_max_code_length, pg.fixed_code_length,
                    pg.block_size, s0, s1, pg.head_dim, stride, s_v, lane);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        fold(static_cast<int>(nt), false, nullptr, nullptr, pg.v_scales + t0, static_cast<int>(pg.zero_point),
             pg.token_begin + t0, pg.head_dim, stride);
      }
    }
    // dense fp32 active tail [active_token_count, kv_head_count, head_dim]
    for (uint32_t t0 = 0; t0 < d.active_token_count; t0 += kLanes) {
      const uint32_t nt = min<uint32_t>(kLanes, d.active_token_count - t0);
      fold(static_cast<int>(nt), true, d.active_k + static_cast<size_t>(t0) * d.kv_head_count * D,
           d.active_v + static_cast<size_t>(t0) * d.kv_head_count * D, nullptr, 0, d.active_token_begin + t0, D, D);
    }
    // finalize: w / sum, zeros when nothing was visible
    for (int h = 0; h < nh; ++h) {
      const float inv = (l[h] > 0.0f) ? 1.0f / l[h] : 0.0f;
      float *out = d.output + (static_cast<size_t>(row) * d.query_head_count + kvh * gqa + h0 + h) * D;
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        const uint32_t dd = lane + 64 * j;
        if (dd < D) out[dd] = bad ? __builtin_nanf("") : acc[h][j] * inv;
      }
    }
  }
}

}  // namespace

// reference src/cuda/paged_kv_attention.cu:280-299 (same rules, same order)
extern "C" cf_status cf_kv_validate_paged_attention_desc(const cf_kv_paged_attention_desc *desc) {
  if (desc == nullptr || desc->struct_size != sizeof(cf_kv_paged_attention_desc) ||
      desc->abi_version != CF_KV_CUDA_ABI_VERSION || desc->queries == nullptr || desc->output == nullptr ||
      desc->query_count == 0 || desc->query_head_count == 0 || desc->kv_head_count == 0 ||
      desc->gqa_group_size == 0 || desc->head_dim == 0 || desc->head_dim > CF_KV_MAX_HEAD_DIM ||
      !std::isfinite(desc->softmax_scale)) {
    return CF_ERR_INVALID_ARGUMENT;
  }
  if (desc->query_head_count != desc->kv_head_count * desc->gqa_group_size ||
      desc->page_count > CF_KV_CUDA_MAX_PAGES_PER_LAUNCH || (desc->page_count != 0 && desc->pages == nullptr) ||
      (desc->active_token_count != 0 && (desc->active_k == nullptr || desc->active_v == nullptr))) {
    return CF_ERR_INVALID_ARGUMENT;
  }
  if (desc->query_token_begin > UINT32_MAX - desc->query_count ||
      desc->active_token_begin > UINT32_MAX - desc->active_token_count) {
    return CF_ERR_INVALID_ARGUMENT;
  }
  return CF_OK;
}

// reference src/cuda/paged_kv_attention.cu:301-327
extern "C" cf_status cf_kv_paged_attention_async(const cf_kv_paged_attention_desc *desc, void *stream) {
  const cf_status valid = cf_kv_validate_paged_attention_desc(desc);
  if (valid != CF_OK) return valid;
  if (desc->kv_head_count > 65535) return CF_ERR_UNSUPPORTED;
  const hipStream_t s = cfd::as_stream(stream);
  const dim3 grid(desc->query_count, desc->kv_head_count);
  if (desc->head_dim <= 64) legacy_kernel<1><<<grid, kLanes, 0, s>>>(*desc);
  else legacy_kernel<2><<<grid, kLanes, 0, s>>>(*desc);
  return cfd::launch_status();
}
