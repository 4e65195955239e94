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
// 16-token page) and the other page fields are not read. A blob that continues a chain, whose header disagrees with
// the page (head_dim, token counts, page gaps) or whose rANS chain does not end where the encoder started makes that
// (query row, KV head) NaN.
//
// Layout on gfx950. The query vectors of a KV head are its (query row, query head) pairs, vector v = row * gqa +
// head. One 4-wavefront workgroup serves 64 vectors (16 per wavefront) of one KV head over one context split (the
// head's pages taken round-robin by their order in the descriptor array; the dense tail in 64-token chunks after
// them). Wave 0 lists the workgroup's pages, up to 64 per scan, with their fields (one memory latency per list, not
// per page). Per chunk of up to 64 tokens, two halves of 32 (a page's tokens, or two consecutive fixed-width pages
// of 32 tokens or fewer), the workgroup decodes K and V once into LDS as integer symbols (K token-major, V
// dim-major; a fixed-width chunk's words and scales were loaded during the previous chunk's MFMAs), then every
// wavefront runs its 16 vectors through:
//   QK^T  v_mfma_f32_16x16x16f16: A = the queries times the page's per-channel K scale, split into f16 hi + lo
//         parts; B = K symbol - zero point, exact in f16. The scores are fp32-grade.
//   softmax online per vector in fp32 (each vector's row of the 16x16 tile lives in 16 lanes);
//   P.V   the same MFMA: A = p times the token's V scale, f16 hi + lo, through a small LDS tile; B = V symbol - zero
//         point, exact.
// The dense tail (fp32) takes the same softmax on VALU. Split partials (m, l, acc) go to a per-GPU device array and
// a second kernel merges them; with one split the workgroup writes the output itself.
#include <cmath>
#include <functional>
#include <mutex>
#include <thread>
#include <utility>

#include "cf_device.hpp"
#include "chromofold/kv_codec_ext.h"
#include "chromofold/kv_cuda.h"
#include "kv_group_decode.hpp"
#include "kv_seam_route.hpp"

namespace {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kVecs = 16 * kWaves;                      // query vectors per workgroup
constexpr int kChunk = 64;                              // tokens staged per chunk
constexpr int kMaxD = CF_KV_MAX_HEAD_DIM;
constexpr int kKStride = kMaxD + 4;                     // bytes per staged K row (token-major)
constexpr int kVStride = kChunk + 4;                    // bytes per staged V row (dim-major)
constexpr int kPStride = kChunk + 4;                    // halves per P row
constexpr int kLutMaxLen = 12;                          // Huffman LUTs of up to 2^12 entries are staged in LDS
constexpr uint32_t kRansWords = CF_KV_RANS_MAX_GROUP_WORDS + 64;  // staged rANS words + slack for idle lanes' reads
constexpr int kList = 64;                               // pages listed per round (one lane of wave 0 each)
// 16-byte units per thread that stage an rANS page's body (at most the INT8 group: 2 streams x hd / 4 quads x 64
// lanes x 4 bytes) into the P tile's bytes
constexpr int kStageA = (2 * (kMaxD / 4) * 64 * 4 / 16 + kThreads - 1) / kThreads;

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

// Decode symbols [s0, s1) of one Huffman stream (rows of hd symbols) with the workgroup's threads; put(token, dim,
// sym) with the token relative to s0 / hd.
template <typename Put>
__device__ void decode_span(const uint32_t *__restrict__ words, const int32_t *__restrict__ boff,
                            const int32_t *__restrict__ lut, uint32_t maxlen, uint32_t block, int64_t s0, int64_t s1,
                            uint32_t hd, int tid, const Put &put) {
  auto at = [&](int64_t i, int sym) {
    const uint32_t rel = static_cast<uint32_t>(i - s0), r = rel / hd;
    put(r, rel - r * hd, static_cast<uint32_t>(sym));
  };
  // Huffman (fixed-width pages go through decode_fixed_pair): one thread per code block intersecting [s0, s1); skip-decode up to s0 inside the first block
  const int64_t b0 = s0 / block, b1 = (s1 + block - 1) / block;
  for (int64_t b = b0 + tid; b < b1; b += kThreads) {
    int64_t pos = boff[b];
    const int64_t first = b * block, last = min(first + static_cast<int64_t>(block), s1);
    for (int64_t i = first; i < last; ++i) {
      const int e = huff_at(words, lut, static_cast<int>(maxlen), pos);
      pos += e >> 8;
      if (i >= s0) at(i, e & 0xff);
    }
  }
}

// ---- rANS pages (kv_codec_ext.h format 4)

// Sign-magnitude bytes (mag: |q|, signs: 0x80 per negative byte) -> offset-binary symbols q + 128, per byte.
__device__ __forceinline__ uint32_t sm_to_offset_binary(uint32_t mag, uint32_t signs) {
  const uint32_t neg = mag & ((signs >> 7) * 0xFFu);  // |q| of the negative bytes
  return 0x80808080u + mag - (neg << 1);              // 128 + |q| or 128 - |q|, no carry between bytes
}

// Stream `stm` (0 = K, 1 = V) of a self-contained group blob (RANS_HYBRID chain start, or the INT8 raw fallback) of
// `ntok` tokens and head_dim hd (% 16 == 0, % 32 for RANS), decoded by one wavefront: K into sk[token * kKStride +
// dim], V into svt[dim * kVStride + token], as offset-binary symbols, with the stream's per-token scales in `sc`.
// The blob's body is already in LDS: `sa` holds the bytes after the header (RANS: lane states, then raw words;
// INT8: the symbol words), `s_w` the RANS word streams (K from s_w[0], V after them), `tab` the stream's table.
// Returns false (wave-uniform) when the blob is not a valid self-contained group for this page. Two wavefronts
// decode K and V at once.
__device__ bool rans_stream_to_lds(const uint8_t *__restrict__ blob_in, const uint32_t *sa, const uint2 *__restrict__ tab,
                                   const uint16_t *s_w, uint32_t hd, uint32_t ntok, uint8_t *sk, uint8_t *svt,
                                   float *sc, int lane, uint32_t stm) {
  const CF_GLOBAL uint8_t *blob = cfd::global_ptr(blob_in);  // global loads: no wait shared with the LDS traffic
  const uint32_t codec = *reinterpret_cast<const CF_GLOBAL uint32_t *>(blob);
  const uint32_t cnt = *reinterpret_cast<const CF_GLOBAL uint32_t *>(blob + 4);
  const uint32_t chain = *reinterpret_cast<const CF_GLOBAL uint16_t *>(blob + 8);
  const CF_GLOBAL uint16_t *tc = reinterpret_cast<const CF_GLOBAL uint16_t *>(blob + 12);
  const uint32_t D = *reinterpret_cast<const CF_GLOBAL uint16_t *>(blob + 20);
  const float scale = reinterpret_cast<const CF_GLOBAL float *>(blob + 32 + 16 * stm)[lane >> 4];
  if (D != hd || hd % 16 != 0 || hd > kMaxD) return false;
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
  sc[lane] = scale;
  const uint32_t NQ = hd / 4, G = static_cast<uint32_t>(lane) >> 4, t = static_cast<uint32_t>(lane) & 15;
  // V quad q of a lane = tokens 4 tq .. 4 tq + 3 of its page at dim t + 16 i (tq = q / (hd / 16), i = q % (hd / 16)):
  // four consecutive bytes of a dim-major row; K quad q = dims 4q .. 4q + 3 of the lane's token
  auto put = [&](uint32_t q, uint32_t w) {
    if (stm == 0) {
      *reinterpret_cast<uint32_t *>(sk + lane * kKStride + 4 * q) = w;
    } else {
      const uint32_t tq = q / (hd / 16), i = q % (hd / 16);
      *reinterpret_cast<uint32_t *>(svt + (t + 16 * i) * kVStride + 16 * G + 4 * tq) = w;
    }
  };
  if (codec == CF_KV_CODEC_INT8) {
    const uint32_t *raw = sa + stm * NQ * 64;
    for (uint32_t q = 0; q < NQ; ++q) put(q, raw[q * 64 + lane]);
    return true;
  }
  const uint32_t nk = cnt & 0xFFFFu, nv = cnt >> 16;
  if (nk + nv > CF_KV_RANS_MAX_GROUP_WORDS) return false;
  const int RAW = cfkv::raw_words_of(static_cast<int>(hd));
  uint32_t x = sa[stm * 64 + lane];
  const uint32_t *raw = sa + 2 * 64 + stm * RAW;
  const uint16_t *w0 = s_w + (stm ? nk : 0u), *wend = w0 + (stm ? nv : nk);
  const uint16_t *wp = w0;
  for (uint32_t sg = 0; sg < hd / 32; ++sg) {
    uint32_t wr[7];
#pragma unroll
    for (int w = 0; w < 7; ++w) wr[w] = raw[(7 * sg + w) * 64 + lane];
    [&]<int... M>(std::integer_sequence<int, M...>) {
      (
          [&] {
            constexpr int m = M;
            constexpr uint32_t rA = cfkv::kFrame[2 * m], rB = cfkv::kFrame[2 * m + 1];
            constexpr int nw = cfkv::kNWord[m], cwi = m < 2 ? 2 : 5;
            const uint2 e = cfkv::rans_lookup(tab, x);
            uint32_t sel;
            const uint32_t wd = cfkv::rans_advance(e.x, x, wp, sel);
            x = __builtin_amdgcn_perm(x, wd, sel);
            const uint32_t sp = rA ? __builtin_amdgcn_alignbit(e.y, e.y, 32 - rA) : e.y;
            const uint32_t q0 = 8 * sg + 2 * m;
            put(q0, sm_to_offset_binary(cfkv::quad_mag<rA>(wr[nw], wr[cwi], sp), cfkv::quad_signs<rA>(wr[6])));
            put(q0 + 1, sm_to_offset_binary(cfkv::quad_mag<rB>(wr[nw], wr[cwi], sp), cfkv::quad_signs<rB>(wr[6])));
          }(),
          ...);
    }(std::make_integer_sequence<int, 4>{});
  }
  // a group coded on its own ends where the encoder started (2^16 in every lane) and has consumed exactly its words
  const bool ok = x == 65536u && wp == wend;
  return __builtin_amdgcn_ballot_w64(!ok) == 0;
}

// ---- the attention kernel

// Four symbol bytes b (offset binary around zp) as exact f16 values b - zp: 1024 + b from the 0x64 exponent byte,
// minus 1024 + zp (integers below 2048 are exact in f16).
__device__ __forceinline__ half4_t sym4_to_half4(uint32_t b, _Float16 base) {
  half4_t h;
  uint32_t *w = reinterpret_cast<uint32_t *>(&h);
  w[0] = __builtin_amdgcn_perm(0x64646464u, b, 0x04010400u);
  w[1] = __builtin_amdgcn_perm(0x64646464u, b, 0x04030402u);
  const half4_t off = {base, base, base, base};
  return h - off;
}

__device__ __forceinline__ float4_t mfma16(half4_t a, half4_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Split s of the (vectors, KV head) unit writes slot slot0 + s of `partial`: [slot][kv head][vector][head_dim + 2] =
// acc, m, l; with no `partial` (one split) the workgroup writes the output itself. `route_taken` (the decode-shape
// route's per-head flags, kv_seam_route.hpp, or NULL): a head the route took is left to it.
template <int D>  // staged query dims: desc head_dim <= D (64 or 128)
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void seam_kernel(
    cf_kv_paged_attention_desc d, uint32_t splits, float *__restrict__ partial, const uint32_t *__restrict__ route_taken,
    uint32_t slot0) {
  constexpr int KS = D / 16;  // 16-dim k-steps of QK^T, 16-dim tiles of the output
  __shared__ __align__(16) uint8_t s_k[kChunk * kKStride];
  __shared__ __align__(16) uint8_t s_vt[kMaxD * kVStride];
  __shared__ __align__(16) _Float16 s_p[kWaves][2][16][kPStride];  // per wavefront: P hi and lo [vector][token]
  __shared__ __align__(16) int32_t s_lut[2][1 << kLutMaxLen];      // Huffman LUTs, rANS tables, or tail queries
  __shared__ __align__(16) uint16_t s_w[kRansWords];
  __shared__ float s_ks[2][kMaxD];               // K scale per channel of the staged page(s) (rANS pages: 1)
  __shared__ float s_kt[kChunk], s_vs[kChunk];   // per token: K scale (legacy pages: 1) and V scale
  __shared__ int s_bad;
  // this workgroup's current list of pages: fields {token_begin, token_count, head_dim, fixed bits | zero point << 8 |
  // kind << 16}, word and scale pointers, descriptor index; count, more-to-come flag, pages of the head seen
  __shared__ uint4 s_pmeta[kList];
  __shared__ uint64_t s_pptr[kList][4];
  __shared__ uint32_t s_pidx[kList];
  __shared__ uint32_t s_pn, s_pmore, s_ord;
  static_assert(sizeof(s_lut) >= 2 * cfkv::kSlots * sizeof(uint2), "the rANS tables share the LUT area");
  static_assert(sizeof(s_lut) >= kVecs * kMaxD * sizeof(float), "the tail's queries share the LUT area");

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t kvh = blockIdx.y, split = blockIdx.z;
  const uint32_t gqa = d.gqa_group_size, HD = d.head_dim;
  const uint32_t M = d.query_count * gqa;                    // query vectors of this KV head
  const uint32_t wv0 = blockIdx.x * kVecs + wave * 16;       // this wavefront's first vector
  const bool wave_active = wv0 < M;
  const float scale = d.softmax_scale;
  if (route_taken && route_taken[kvh]) return;  // the decode-shape route covers this head (the merge knows)

  auto row_of = [&](uint32_t v) { return v / gqa; };
  auto qtok_of = [&](uint32_t r) { return d.query_token_begin + r; };
  auto wbegin_of = [&](uint32_t r) {
    const uint32_t qt = qtok_of(r);
    return (d.causal_window == 0 || qt + 1 <= d.causal_window) ? 0u : qt + 1 - d.causal_window;
  };
  // visible token range of the workgroup's rows (pages wholly outside it are skipped)
  const uint32_t wg_v1 = min(M, (blockIdx.x + 1) * kVecs) - 1;
  const uint32_t vis_lo = wbegin_of(row_of(blockIdx.x * kVecs)), vis_hi = qtok_of(row_of(wg_v1));

  // A-operand vector of this lane (row lane % 16 of the wavefront's 16) and its raw query values: k-step kk holds
  // dims 16 kk + 4 (lane / 16) .. + 3
  const uint32_t av = wv0 + (lane & 15);
  float qraw[KS][4];
  {
    const bool ok = av < M;
    const uint32_t r = ok ? row_of(av) : 0, g = ok ? av % gqa : 0;
    const float *qp = d.queries + (static_cast<size_t>(r) * d.query_head_count + kvh * gqa + g) * HD;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t dd = 16 * kk + 4 * (lane >> 4) + j;
        qraw[kk][j] = (ok && dd < HD) ? qp[dd] : 0.0f;
      }
  }
  // A operands of one page: the queries times its per-channel K scales (s_ks[p]; 1 for rANS pages), f16 hi + lo
  auto build_q = [&](half4_t (&qhi)[KS], half4_t (&qlo)[KS], uint32_t p) {
#pragma unroll
    for (int kk = 0; kk < KS; ++kk)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        _Float16 h, l;
        cfd::split_mul_f16(qraw[kk][j], s_ks[p][16 * kk + 4 * (lane >> 4) + j], h, l);
        qhi[kk][j] = h;
        qlo[kk][j] = l;
      }
  };

  // C-layout vectors of this lane: wv0 + 4 (lane / 16) + i, i < 4; their rows' visible token ranges
  uint32_t c_lo[4], c_hi[4];
  bool c_ok[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t v = wv0 + 4 * (lane >> 4) + i;
    c_ok[i] = v < M;
    const uint32_t r = c_ok[i] ? row_of(v) : 0;
    c_lo[i] = wbegin_of(r);
    c_hi[i] = qtok_of(r);
  }
  float m_run[4], l_run[4];
  float4_t acc[KS];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m_run[i] = -INFINITY;
    l_run[i] = 0.0f;
  }
#pragma unroll
  for (int t = 0; t < KS; ++t) acc[t] = float4_t{0, 0, 0, 0};
  if (tid == 0) s_bad = 0;

  // Online softmax over one chunk: s[i][j] = score of vector i (C layout) with token 16 j + lane % 16 (-inf when
  // not visible); rescales acc, updates (m, l), returns p in s.
  auto softmax_chunk = [&](float (&s)[4][4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float mx = cfd::row16_max(fmaxf(fmaxf(s[i][0], s[i][1]), fmaxf(s[i][2], s[i][3])));
      const float mn = fmaxf(m_run[i], mx);
      const float alpha = (m_run[i] == -INFINITY) ? 0.0f : __expf(m_run[i] - mn);
      float ps = 0.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        s[i][j] = (s[i][j] == -INFINITY) ? 0.0f : __expf(s[i][j] - mn);
        ps += s[i][j];
      }
      ps = cfd::row16_sum(ps);
      if (mn != -INFINITY) {
        l_run[i] = l_run[i] * alpha + ps;
#pragma unroll
        for (int t = 0; t < KS; ++t) acc[t][i] *= alpha;
        m_run[i] = mn;
      }
    }
  };

  // Scores, online softmax and P.V of the staged chunk. Rows 0-31 (half 0) and 32-63 (half 1) of s_k / s_vt hold
  // nh[h] tokens from position tok[h] (a half is one page's tokens, or the continuation of half 0's page);
  // half h's K scales are s_ks[h ? kp1 : 0], its symbols sit around zb[h] (1024 + the page's zero point); per-token
  // scales in s_kt / s_vs.
  auto compute_chunk = [&](const uint32_t (&tok)[2], const uint32_t (&nh)[2], const _Float16 (&zb)[2], uint32_t kp1) {
    float s[4][4];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      half4_t qhi[KS], qlo[KS];
      if (h == 0 || nh[1] != 0) build_q(qhi, qlo, h ? kp1 : 0u);
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int j = 2 * h + jj;
        float4_t c = {0, 0, 0, 0};
        if (16u * jj < nh[h]) {
          const uint8_t *krow = s_k + (16 * j + (lane & 15)) * kKStride + 4 * (lane >> 4);
#pragma unroll
          for (int kk = 0; kk < KS; ++kk) {
            const half4_t b = sym4_to_half4(*reinterpret_cast<const uint32_t *>(krow + 16 * kk), zb[h]);
            c = mfma16(qhi[kk], b, c);
            c = mfma16(qlo[kk], b, c);
          }
        }
        const uint32_t r = 16 * jj + (lane & 15), tk = tok[h] + r;
        const float kts = s_kt[16 * j + (lane & 15)];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bool vis = r < nh[h] && c_ok[i] && tk >= c_lo[i] && tk <= c_hi[i];
          s[i][j] = vis ? c[i] * kts * scale : -INFINITY;
        }
      }
    }
    softmax_chunk(s);
    // P (times the token's V scale) -> this wavefront's LDS tile as f16 hi + lo [vector][token]
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t tt = 16 * j + (lane & 15);
      const float vsc = s_vs[tt];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        cfd::split_mul_f16(s[i][j], vsc, s_p[wave][0][4 * (lane >> 4) + i][tt], s_p[wave][1][4 * (lane >> 4) + i][tt]);
      }
    }
    wave_sync();
    // P.V: acc[t] (vector rows, dims 16 t + lane % 16) += P[16 x tokens] V[tokens x 16]
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      if (16u * (ks & 1) >= nh[ks >> 1]) continue;
      const half4_t ph = *reinterpret_cast<const half4_t *>(&s_p[wave][0][lane & 15][16 * ks + 4 * (lane >> 4)]);
      const half4_t pl = *reinterpret_cast<const half4_t *>(&s_p[wave][1][lane & 15][16 * ks + 4 * (lane >> 4)]);
#pragma unroll
      for (int t = 0; t < KS; ++t) {
        const uint32_t w = *reinterpret_cast<const uint32_t *>(s_vt + (16 * t + (lane & 15)) * kVStride + 16 * ks +
                                                               4 * (lane >> 4));
        const half4_t b = sym4_to_half4(w, zb[ks >> 1]);
        acc[t] = mfma16(ph, b, acc[t]);
        acc[t] = mfma16(pl, b, acc[t]);
      }
    }
    wave_sync();
  };

  // ---- pages of this KV head, round-robin over the splits by their order in the descriptor array.
  // Wave 0 lists this workgroup's pages, up to kList at a time, with the fields the fixed-width path needs (one
  // lane per listed page: one memory latency per list instead of one per page). The listed pages' chunks then run
  // in order; for fixed-width pages the next chunk's words and scales load while the current chunk computes, so a
  // chunk waits for memory only when the previous one was not fixed-width.
  uint32_t scan_pb = 0, scan_ord = 0;  // wave 0: next descriptor to examine, ordinal of the head's next page there
  const int32_t *tab_k = nullptr, *tab_v = nullptr;  // the rANS tables staged in s_lut (uniform)
  for (;;) {
    if (wave == 0) {
      // pass 1: which descriptors are this workgroup's (kv head, ordinal % splits), 256 descriptors per step with
      // their loads in flight together, selection and compaction lane-parallel
      uint32_t cnt = 0;
      bool full = false;
      while (!full && scan_pb < d.page_count) {
        uint32_t hv[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t pi = scan_pb + 64 * q + lane;
          hv[q] = pi < d.page_count ? cfd::global_ptr(d.pages)[pi].kv_head : 0xFFFFFFFFu;
        }
        uint32_t ord_run = scan_ord;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (full) break;
          const uint32_t pi = scan_pb + 64 * q + lane;
          const bool match = hv[q] == kvh && pi < d.page_count;
          const uint64_t m = __builtin_amdgcn_ballot_w64(match);
          const uint32_t ordl = ord_run + __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u));
          const bool sel = match && ordl % splits == split;
          const uint64_t ms = __builtin_amdgcn_ballot_w64(sel);
          const uint32_t rk = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(ms >> 32),
                                                        __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(ms), 0u));
          const uint32_t nsel = static_cast<uint32_t>(__builtin_popcountll(ms));
          if (cnt + nsel > static_cast<uint32_t>(kList)) {
            // the list is full inside this batch: take the first pages, resume at the first one not taken
            const uint32_t take = static_cast<uint32_t>(kList) - cnt;
            if (sel && rk < take) s_pidx[cnt + rk] = pi;
            const uint64_t mr = __builtin_amdgcn_ballot_w64(sel && rk == take);
            const int lr = __builtin_ctzll(mr);
            scan_pb = __builtin_amdgcn_readlane(pi, lr);
            scan_ord = __builtin_amdgcn_readlane(ordl, lr);
            cnt = kList;
            full = true;
            break;
          }
          if (sel) s_pidx[cnt + rk] = pi;
          cnt += nsel;
          ord_run += static_cast<uint32_t>(__builtin_popcountll(m));
        }
        if (!full) {
          scan_pb += 256;
          scan_ord = ord_run;
        }
      }
      wave_sync();
      const uint32_t my_p = static_cast<uint32_t>(lane) < cnt ? s_pidx[lane] : 0u;
      wave_sync();
      // the listed pages' fields, one lane each; empty pages and pages wholly outside the workgroup's visible
      // range are dropped, the others compacted in order
      bool keep = false;
      uint4 meta = make_uint4(0, 0, 0, 0);
      const CF_GLOBAL cf_kv_device_page *pg = cfd::global_ptr(d.pages) + my_p;
      if (static_cast<uint32_t>(lane) < cnt) {
        const uint32_t tb = pg->token_begin, tc = pg->token_count, fixed = pg->fixed_code_length;
        keep = tc != 0 && !(tb > vis_hi || tb + tc <= vis_lo);
        const uint32_t kind = fixed ? 0u : (pg->k_max_code_length == 0 ? 2u : 1u);  // fixed / Huffman / rANS
        meta = make_uint4(tb, tc, pg->head_dim, (fixed & 0xFFu) | ((pg->zero_point & 0xFFu) << 8) | (kind << 16));
      }
      const uint64_t km = __builtin_amdgcn_ballot_w64(keep);
      const uint32_t at = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(km >> 32),
                                                    __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(km), 0u));
      if (keep) {
        s_pmeta[at] = meta;
        s_pptr[at][0] = reinterpret_cast<uintptr_t>(pg->k_words);
        s_pptr[at][1] = reinterpret_cast<uintptr_t>(pg->v_words);
        s_pptr[at][2] = reinterpret_cast<uintptr_t>(pg->k_scales);
        s_pptr[at][3] = reinterpret_cast<uintptr_t>(pg->v_scales);
        s_pidx[at] = my_p;
      }
      if (lane == 0) {
        s_pn = static_cast<uint32_t>(__builtin_popcountll(km));
        s_pmore = full ? 1u : 0u;
        s_ord = scan_ord;
      }
    }
    __syncthreads();
    const uint32_t n = __builtin_amdgcn_readfirstlane(s_pn);
    const bool more = __builtin_amdgcn_readfirstlane(s_pmore) != 0;

    // Fixed-width chunks: two halves of up to 32 tokens (rows 0-31 and 32-63 of the staged tiles). Half 0 takes
    // page li from token t0; half 1 the page's next 32 tokens, or, when the page has none left, page li + 1 if it is
    // a fixed-width page of the same head_dim and code width with at most 32 tokens (two 32-token pages per
    // chunk: one staging, one softmax and one barrier pair per 64 tokens).
    struct Plan {
      uint32_t li[2], t0[2], nt[2];
      uint32_t nli, nt0;  // the chunk after this one
    };
    auto plan_at = [&](uint32_t li, uint32_t t0) {
      Plan p{};
      const uint4 mt = s_pmeta[li];
      const uint32_t tc = __builtin_amdgcn_readfirstlane(mt.y), mw = __builtin_amdgcn_readfirstlane(mt.w);
      const uint32_t rem = tc - t0;
      p.li[0] = li;
      p.t0[0] = t0;
      p.nt[0] = min(rem, 32u);
      p.li[1] = li;
      p.t0[1] = t0 + 32u;
      p.nt[1] = rem > 32u ? min(rem - 32u, 32u) : 0u;
      p.nli = rem > 64u ? li : li + 1u;
      p.nt0 = rem > 64u ? t0 + 64u : 0u;
      if (rem <= 32u && li + 1u < n) {
        const uint4 mb = s_pmeta[li + 1u];
        const uint32_t bw = __builtin_amdgcn_readfirstlane(mb.w), bc = __builtin_amdgcn_readfirstlane(mb.y);
        const uint32_t bd = __builtin_amdgcn_readfirstlane(mb.z), ad = __builtin_amdgcn_readfirstlane(mt.z);
        if ((bw >> 16) == 0u && (bw & 0xFFu) == (mw & 0xFFu) && bd == ad && bc <= 32u) {
          p.li[1] = li + 1u;
          p.t0[1] = 0u;
          p.nt[1] = bc;
          p.nli = li + 2u;
        }
      }
      return p;
    };
    // what a thread loads for a chunk ahead of its turn: per half the first 2 * kThreads words of K and of V, the
    // K scale of channel tid; the V scale of token tid of the chunk
    struct Pre {
      uint32_t k[2][2], v[2][2];
      float ks[2], vs;
    };
    auto fixed_ok = [&](uint32_t li) {  // a fixed-width page this kernel stages
      if (li >= n) return false;
      const uint4 mt = s_pmeta[li];
      const uint32_t mw = __builtin_amdgcn_readfirstlane(mt.w), phd = __builtin_amdgcn_readfirstlane(mt.z);
      return (mw >> 16) == 0u && (mw & 0xFFu) != 0u && phd != 0u && phd <= static_cast<uint32_t>(kMaxD);
    };
    auto prefetch = [&](uint32_t li, uint32_t t0) {
      Pre r{};
      if (!fixed_ok(li)) return r;
      const Plan p = plan_at(li, t0);
      const uint4 mt = s_pmeta[li];
      const uint32_t bits = __builtin_amdgcn_readfirstlane(mt.w) & 0xFFu, phd = __builtin_amdgcn_readfirstlane(mt.z);
      const uint32_t spw = 32u / bits;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t ph = p.nt[h] ? p.li[h] : p.li[0];  // an empty half loads half 0's page (never used)
        const CF_GLOBAL uint32_t *kw = cfd::global_ptr(reinterpret_cast<const uint32_t *>(s_pptr[ph][0]));
        const CF_GLOBAL uint32_t *vw = cfd::global_ptr(reinterpret_cast<const uint32_t *>(s_pptr[ph][1]));
        const CF_GLOBAL float *ksc = cfd::global_ptr(reinterpret_cast<const float *>(s_pptr[ph][2]));
        const uint32_t nt = p.nt[h] ? p.nt[h] : p.nt[0], t0h = p.nt[h] ? p.t0[h] : p.t0[0];
        const int64_t s0 = static_cast<int64_t>(t0h) * phd, s1 = s0 + static_cast<int64_t>(nt) * phd;
        const int64_t w0 = s0 / spw, w1 = (s1 + spw - 1) / spw;
        const int64_t wa = min<int64_t>(w0 + tid, w1 - 1), wc = min<int64_t>(w0 + tid + kThreads, w1 - 1);
        r.k[h][0] = kw[wa];
        r.k[h][1] = kw[wc];
        r.v[h][0] = vw[wa];
        r.v[h][1] = vw[wc];
        r.ks[h] = ksc[min<uint32_t>(static_cast<uint32_t>(tid), phd - 1)];
      }
      const bool h1 = ((static_cast<uint32_t>(tid) >> 5) & 1u) && p.nt[1];  // the thread's token is in half 1
      const uint32_t pv = h1 ? p.li[1] : p.li[0], tv = h1 ? p.t0[1] : p.t0[0], nv = h1 ? p.nt[1] : p.nt[0];
      const CF_GLOBAL float *vsc = cfd::global_ptr(reinterpret_cast<const float *>(s_pptr[pv][3]));
      r.vs = vsc[tv + min<uint32_t>(static_cast<uint32_t>(tid) & 31u, nv - 1u)];
      return r;
    };
    // 16-byte units of a self-contained group blob of head_dim hd after its header: part 0 = lane states and raw
    // words (RANS) or the symbol words (INT8), part 1 = the RANS word streams; 0 when the header does not describe
    // such a group (the decode refuses the blob), so that staging never reads past a blob
    auto blob_units = [&](const uint8_t *b, uint32_t hd, int part) -> uint32_t {
      const CF_GLOBAL uint8_t *g = cfd::global_ptr(b);
      const uint32_t codec = *reinterpret_cast<const CF_GLOBAL uint32_t *>(g);
      const uint32_t cnt = *reinterpret_cast<const CF_GLOBAL uint32_t *>(g + 4);
      const uint32_t chain = *reinterpret_cast<const CF_GLOBAL uint16_t *>(g + 8);
      const uint32_t bd = *reinterpret_cast<const CF_GLOBAL uint16_t *>(g + 20);
      if (bd != hd || hd == 0 || hd > static_cast<uint32_t>(kMaxD) || hd % 16 != 0) return 0u;
      if (codec == CF_KV_CODEC_INT8) return part ? 0u : 2u * (hd / 4) * 64u * 4u / 16u;
      const uint32_t words = (cnt & 0xFFFFu) + (cnt >> 16);
      if (codec != CF_KV_CODEC_RANS_HYBRID || chain != 1 || hd % 32 != 0 || words > CF_KV_RANS_MAX_GROUP_WORDS)
        return 0u;
      if (part) return (2u * words + 15u) / 16u;
      return (cfkv::kStateBytes + 8u * static_cast<uint32_t>(cfkv::raw_words_of(static_cast<int>(hd)))) / 16u;
    };

    uint32_t li = 0, t0 = 0;
    Pre cur = prefetch(0, 0);
    while (li < n) {
      const uint4 mt = s_pmeta[li];
      const uint32_t phd = __builtin_amdgcn_readfirstlane(mt.z), mw = __builtin_amdgcn_readfirstlane(mt.w);
      const uint32_t kind = mw >> 16;
      if (kind != 0) {
        // Huffman and rANS pages: staged at their turn (no prefetch), every chunk of the page; a page this kernel
        // cannot stage leaves the do-while early
        do {
        const cf_kv_device_page pg = d.pages[__builtin_amdgcn_readfirstlane(s_pidx[li])];
        const bool rans = pg.fixed_code_length == 0 && pg.k_max_code_length == 0;
        if (rans && (pg.token_count > static_cast<uint32_t>(kChunk) || pg.head_dim == 0 || pg.head_dim > kMaxD)) {
          if (tid == 0) s_bad = 1;
          continue;
        }
        if (!rans && (pg.head_dim == 0 || pg.head_dim > kMaxD)) continue;
        const uint32_t phd = pg.head_dim;
        const uint32_t zp = rans ? 128u : pg.zero_point;
        const _Float16 zbase = static_cast<_Float16>(1024.0f + static_cast<float>(zp));
        // Huffman pages: both LUTs in LDS when they fit (the lookups are the decoder's hot loop)
        const int32_t *klut = pg.k_lut, *vlut = pg.v_lut;
        if (!rans && !pg.fixed_code_length && pg.k_max_code_length <= kLutMaxLen && pg.v_max_code_length <= kLutMaxLen) {
          __syncthreads();  // the previous chunk's readers of s_lut are done
          for (uint32_t i = tid; i < (1u << pg.k_max_code_length); i += kThreads) s_lut[0][i] = pg.k_lut[i];
          for (uint32_t i = tid; i < (1u << pg.v_max_code_length); i += kThreads) s_lut[1][i] = pg.v_lut[i];
          tab_k = tab_v = nullptr;  // the rANS tables staged there are gone
          klut = s_lut[0];
          vlut = s_lut[1];
        }
        for (uint32_t t0 = 0; t0 < pg.token_count; t0 += kChunk) {
          const uint32_t nt = min<uint32_t>(kChunk, pg.token_count - t0);
          const uint32_t tok0 = pg.token_begin + t0;
          __syncthreads();  // the previous chunk's compute no longer reads the staged tiles
          for (uint32_t dd = tid; dd < kMaxD; dd += kThreads) s_ks[0][dd] = rans ? 1.0f : (dd < phd ? pg.k_scales[dd] : 0.0f);
          if (rans) {
            uint2(*tab)[cfkv::kSlots] = reinterpret_cast<uint2(*)[cfkv::kSlots]>(&s_lut[0][0]);
            const uint8_t *blob = reinterpret_cast<const uint8_t *>(pg.k_words);
            const uint32_t codec = __builtin_amdgcn_readfirstlane(*reinterpret_cast<const uint32_t *>(blob));
            if (codec == CF_KV_CODEC_RANS_HYBRID && (pg.k_lut != tab_k || pg.v_lut != tab_v)) {
              // the K and V tables as the decoder reads them ({f | c << 16, spread}), staged by every thread; kept
              // for the next rANS page with the same tables
              const uint2 *kt = reinterpret_cast<const uint2 *>(pg.k_lut), *vt = reinterpret_cast<const uint2 *>(pg.v_lut);
              for (uint32_t i = tid; i < cfkv::kSlots; i += kThreads) {
                const uint2 a = kt[i], b = vt[i];
                tab[0][i] = uint2{(a.x & 2047u) | (((a.x >> 11) & 2047u) << 16), a.y};
                tab[1][i] = uint2{(b.x & 2047u) | (((b.x >> 11) & 2047u) << 16), b.y};
              }
              tab_k = pg.k_lut;
              tab_v = pg.v_lut;
              __syncthreads();
            }
            // the blob's body after the header into LDS with every thread's 16-byte loads in flight together:
            // states and raw words (or INT8 symbol words) into the P tile's bytes (free until this chunk's compute),
            // the word streams into s_w; a header that does not describe a group of this head_dim stages nothing
            // (the decode refuses it), so no byte past a blob is read
            static_assert(sizeof(s_p) >= kStageA * kThreads * 16, "an rANS page body fits the P tile");
            static_assert(sizeof(s_w) >= 2 * CF_KV_RANS_MAX_GROUP_WORDS && kThreads * 16 >= 2 * CF_KV_RANS_MAX_GROUP_WORDS,
                          "one 16-byte unit per thread stages the word streams");
            uint32_t *sa = reinterpret_cast<uint32_t *>(&s_p[0][0][0][0]);
            {
              const uint32_t ua = blob_units(blob, phd, 0), uw = blob_units(blob, phd, 1);
              typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
              const CF_GLOBAL u32x4 *g16 = cfd::global_ptr(reinterpret_cast<const u32x4 *>(blob + cfkv::kHdr));
              if (ua) {  // uniform
                u32x4 v[kStageA];
#pragma unroll
                for (int k = 0; k < kStageA; ++k) v[k] = g16[min<uint32_t>(tid + kThreads * k, ua - 1)];
                u32x4 vw = v[0];
                if (uw) vw = g16[ua + min<uint32_t>(tid, uw - 1)];  // uniform
#pragma unroll
                for (int k = 0; k < kStageA; ++k)
                  if (tid + kThreads * k < ua) reinterpret_cast<u32x4 *>(sa)[tid + kThreads * k] = v[k];
                if (static_cast<uint32_t>(tid) < uw) reinterpret_cast<u32x4 *>(s_w)[tid] = vw;
              }
            }
            __syncthreads();
            if (wave < 2) {  // wave 0 decodes K, wave 1 V
              const bool ok = rans_stream_to_lds(blob, sa, tab[wave], s_w, phd, nt, s_k, s_vt, wave ? s_vs : s_kt, lane,
                                                 static_cast<uint32_t>(wave));
              if (!ok && lane == 0) s_bad = 1;
            }
          } else {
            for (int t = tid; t < kChunk; t += kThreads) {
              s_kt[t] = 1.0f;
              s_vs[t] = t < static_cast<int>(nt) ? pg.v_scales[t0 + t] : 0.0f;
            }
            const int64_t s0 = static_cast<int64_t>(t0) * phd, s1 = s0 + static_cast<int64_t>(nt) * phd;
            decode_span(pg.k_words, pg.k_block_offsets, klut, pg.k_max_code_length, pg.block_size, s0, s1, phd, tid,
                        [&](uint32_t r, uint32_t c, uint32_t sym) { s_k[r * kKStride + c] = static_cast<uint8_t>(sym); });
            decode_span(pg.v_words, pg.v_block_offsets, vlut, pg.v_max_code_length, pg.block_size, s0, s1, phd, tid,
                        [&](uint32_t r, uint32_t c, uint32_t sym) { s_vt[c * kVStride + r] = static_cast<uint8_t>(sym); });
          }
          // dims the page does not have read as V = 0 (the query side zeroes K through s_ks)
          for (uint32_t i = tid; i < (HD > phd ? HD - phd : 0u) * kChunk; i += kThreads)
            s_vt[(phd + i / kChunk) * kVStride + i % kChunk] = static_cast<uint8_t>(zp);
          __syncthreads();
          if (!s_bad && wave_active) {
            const uint32_t tk[2] = {tok0, tok0 + 32u}, nh[2] = {min(nt, 32u), nt > 32u ? nt - 32u : 0u};
            const _Float16 zb[2] = {zbase, zbase};
            compute_chunk(tk, nh, zb, 0u);
          }
        }
        } while (false);
        ++li;
        t0 = 0;
        cur = prefetch(li, 0);
        continue;
      }
      // fixed-width chunk at (li, t0)
      if (!fixed_ok(li)) {  // not a page this kernel can stage: skipped
        ++li;
        t0 = 0;
        cur = prefetch(li, 0);
        continue;
      }
      const Plan p = plan_at(li, t0);
      const uint32_t bits = mw & 0xFFu, spw = 32u / bits, mask = (1u << bits) - 1u;
      uint32_t zp[2], tk[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint4 mh = s_pmeta[p.li[h]];
        zp[h] = (__builtin_amdgcn_readfirstlane(mh.w) >> 8) & 0xFFu;
        tk[h] = __builtin_amdgcn_readfirstlane(mh.x) + p.t0[h];
      }
      const uint32_t kp1 = p.li[1] != p.li[0] ? 1u : 0u;  // half 1's K scales: its own page's, or half 0's
      __syncthreads();  // the previous chunk's compute no longer reads the staged tiles
      if (static_cast<uint32_t>(tid) < kMaxD) {
        s_ks[0][tid] = static_cast<uint32_t>(tid) < phd ? cur.ks[0] : 0.0f;
        s_ks[1][tid] = static_cast<uint32_t>(tid) < phd ? cur.ks[1] : 0.0f;
      }
      if (tid < kChunk) {
        s_kt[tid] = 1.0f;
        s_vs[tid] = (static_cast<uint32_t>(tid) & 31u) < (tid < 32 ? p.nt[0] : p.nt[1]) ? cur.vs : 0.0f;
      }
      // int4 / int8 codes with head_dim a multiple of the codes per word (every shape the adapter seals): each word
      // lies inside one token row, its row from one multiply-high (rel < 2^13 and the reciprocal's error below
      // head_dim keep it exact) and its codes reordered by byte permutes into one piece of a K row
      const bool whole = (bits == 4u || bits == 8u) && phd % spw == 0u;
      const uint32_t inv = 0xFFFFFFFFu / phd + 1u;  // ceil(2^32 / phd) for phd >= 2
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if (p.nt[h] == 0u) continue;  // uniform
        const int64_t s0 = static_cast<int64_t>(p.t0[h]) * phd, s1 = s0 + static_cast<int64_t>(p.nt[h]) * phd;
        const int64_t w0 = s0 / spw, w1 = (s1 + spw - 1) / spw;
        const uint32_t rbase = 32u * h;
        auto put = [&](int64_t w, uint32_t kword, uint32_t vword) {
          if (whole) {
            const uint32_t rel = static_cast<uint32_t>(w * spw - s0), r = __umulhi(rel, inv), c = rel - r * phd;
            uint8_t *kd = s_k + (rbase + r) * kKStride + c;
            uint8_t *vd = s_vt + c * kVStride + rbase + r;
            const uint32_t yk = __builtin_bswap32(kword), yv = __builtin_bswap32(vword);  // first code in byte 0
            if (bits == 8u) {
              *reinterpret_cast<uint32_t *>(kd) = yk;
#pragma unroll
              for (int k = 0; k < 4; ++k) vd[k * kVStride] = static_cast<uint8_t>(yv >> (8 * k));
            } else {
              // byte b of y holds codes 2b (high nibble) and 2b + 1: codes 0..3 = {h0, l0, h1, l1}, 4..7 = {h2, ...}
              const uint32_t hk = (yk >> 4) & 0x0F0F0F0Fu, lk = yk & 0x0F0F0F0Fu;
              const uint32_t hv = (yv >> 4) & 0x0F0F0F0Fu, lv = yv & 0x0F0F0F0Fu;
              reinterpret_cast<uint32_t *>(kd)[0] = __builtin_amdgcn_perm(hk, lk, 0x01050004u);
              reinterpret_cast<uint32_t *>(kd)[1] = __builtin_amdgcn_perm(hk, lk, 0x03070206u);
              const uint32_t v0 = __builtin_amdgcn_perm(hv, lv, 0x01050004u), v1 = __builtin_amdgcn_perm(hv, lv, 0x03070206u);
#pragma unroll
              for (int k = 0; k < 4; ++k) {
                vd[k * kVStride] = static_cast<uint8_t>(v0 >> (8 * k));
                vd[(k + 4) * kVStride] = static_cast<uint8_t>(v1 >> (8 * k));
              }
            }
            return;
          }
          for (uint32_t k = 0; k < spw; ++k) {
            const int64_t i = w * spw + k;
            if (i < s0 || i >= s1) continue;
            const uint32_t sh = 32u - bits * (k + 1), rel = static_cast<uint32_t>(i - s0), r = rel / phd, c = rel - r * phd;
            s_k[(rbase + r) * kKStride + c] = static_cast<uint8_t>((kword >> sh) & mask);
            s_vt[c * kVStride + rbase + r] = static_cast<uint8_t>((vword >> sh) & mask);
          }
        };
        if (w0 + tid < w1) put(w0 + tid, cur.k[h][0], cur.v[h][0]);
        if (w0 + tid + kThreads < w1) put(w0 + tid + kThreads, cur.k[h][1], cur.v[h][1]);
        // words past the prefetched 2 * kThreads (halves of more than 1 KiB per stream) are loaded here
        const CF_GLOBAL uint32_t *kw = cfd::global_ptr(reinterpret_cast<const uint32_t *>(s_pptr[p.li[h]][0]));
        const CF_GLOBAL uint32_t *vw = cfd::global_ptr(reinterpret_cast<const uint32_t *>(s_pptr[p.li[h]][1]));
        for (int64_t w = w0 + 2 * kThreads + tid; w < w1; w += kThreads) put(w, kw[w], vw[w]);
      }
      // dims the page does not have read as V = 0 (the query side zeroes K through s_ks)
      for (uint32_t i = tid; i < (HD > phd ? HD - phd : 0u) * kChunk; i += kThreads)
        s_vt[(phd + i / kChunk) * kVStride + i % kChunk] = static_cast<uint8_t>(i % kChunk < 32u ? zp[0] : zp[1]);
      const Pre nxt = prefetch(p.nli, p.nt0);  // in flight during this chunk's compute
      __syncthreads();
      if (!s_bad && wave_active) {
        const _Float16 zb[2] = {static_cast<_Float16>(1024.0f + static_cast<float>(zp[0])),
                                static_cast<_Float16>(1024.0f + static_cast<float>(zp[1]))};
        const uint32_t nh[2] = {p.nt[0], p.nt[1]};
        compute_chunk(tk, nh, zb, kp1);
      }
      cur = nxt;
      li = p.nli;
      t0 = p.nt0;
    }
    if (!more) break;
    __syncthreads();  // the list is rewritten by the next round
  }
  const uint32_t ord = __builtin_amdgcn_readfirstlane(s_ord);

  // ---- dense fp32 tail [active_token_count, kv_head_count, head_dim], 64-token chunks continuing the round-robin
  if (d.active_token_count) {
    __syncthreads();
    float *s_qf = reinterpret_cast<float *>(&s_lut[0][0]) + wave * 16 * kMaxD;  // this wavefront's 16 queries
    for (uint32_t i = lane; i < 16u * HD; i += 64) {
      const uint32_t v = wv0 + i / HD, dd = i % HD;
      float q = 0.0f;
      if (v < M) q = d.queries[(static_cast<size_t>(row_of(v)) * d.query_head_count + kvh * gqa + v % gqa) * HD + dd];
      s_qf[(i / HD) * kMaxD + dd] = q;
    }
    wave_sync();
    float *s_pf = reinterpret_cast<float *>(&s_p[wave][0][0][0]);  // p [vector][token] in fp32 (same bytes)
    static_assert(sizeof(s_p[0]) >= 16 * kChunk * sizeof(float), "fp32 tail weights share the P tile");
    uint32_t tord = ord;
    for (uint32_t t0 = 0; t0 < d.active_token_count; t0 += kChunk) {
      if (tord++ % splits != split) continue;
      if (!wave_active) continue;
      const uint32_t nt = min<uint32_t>(kChunk, d.active_token_count - t0);
      const uint32_t tok0 = d.active_token_begin + t0;
      float s[4][4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t tt = 16 * j + (lane & 15), tok = tok0 + tt;
        float dot[4] = {0, 0, 0, 0};
        if (tt < nt) {
          const float *kr = d.active_k + (static_cast<size_t>(t0 + tt) * d.kv_head_count + kvh) * HD;
          for (uint32_t dd = 0; dd < HD; ++dd) {
            const float kv = kr[dd];
#pragma unroll
            for (int i = 0; i < 4; ++i) dot[i] += s_qf[(4 * (lane >> 4) + i) * kMaxD + dd] * kv;
          }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bool vis = tt < nt && c_ok[i] && tok >= c_lo[i] && tok <= c_hi[i];
          s[i][j] = vis ? dot[i] * scale : -INFINITY;
        }
      }
      softmax_chunk(s);
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) s_pf[(4 * (lane >> 4) + i) * kChunk + 16 * j + (lane & 15)] = s[i][j];
      wave_sync();
      for (uint32_t tt = 0; tt < nt; ++tt) {
        const float *vr = d.active_v + (static_cast<size_t>(t0 + tt) * d.kv_head_count + kvh) * HD;
#pragma unroll
        for (int t = 0; t < KS; ++t) {
          const uint32_t dd = 16 * t + (lane & 15);
          const float vv = dd < HD ? vr[dd] : 0.0f;
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[t][i] += s_pf[(4 * (lane >> 4) + i) * kChunk + tt] * vv;
        }
      }
      wave_sync();
    }
  }

  // ---- output (one split) or this split's partial
  __syncthreads();
  const bool bad = s_bad != 0;
  if (!wave_active) return;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t v = wv0 + 4 * (lane >> 4) + i;
    if (v >= M) continue;
    if (!partial) {
      const float inv = l_run[i] > 0.0f ? 1.0f / l_run[i] : 0.0f;
      float *out = d.output + (static_cast<size_t>(row_of(v)) * d.query_head_count + kvh * gqa + v % gqa) * HD;
#pragma unroll
      for (int t = 0; t < KS; ++t) {
        const uint32_t dd = 16 * t + (lane & 15);
        if (dd < HD) out[dd] = bad ? __builtin_nanf("") : acc[t][i] * inv;
      }
    } else {
      float *pp = partial + ((static_cast<size_t>(slot0 + split) * d.kv_head_count + kvh) * M + v) * (HD + 2);
#pragma unroll
      for (int t = 0; t < KS; ++t) {
        const uint32_t dd = 16 * t + (lane & 15);
        if (dd < HD) pp[dd] = acc[t][i];
      }
      if ((lane & 15) == 0) {
        pp[HD] = bad ? __builtin_nanf("") : m_run[i];
        pp[HD + 1] = l_run[i];
      }
    }
  }
}

// Merge the split partials of one (vector, KV head) per workgroup: out = sum_s acc_s e^(m_s - m) / sum_s l_s
// e^(m_s - m); zeros when nothing was visible; NaN when a split saw a refused page. The splits' (m, l) pairs are read
// once into LDS; each thread then streams its dim of every split with 8 loads in flight.
// With the decode-shape route (`taken` not NULL), a head it took has its slots at [0, route_slots), the others at
// [route_slots, splits).
__global__ __launch_bounds__(kMaxD) void seam_merge_kernel(cf_kv_paged_attention_desc d, uint32_t splits,
                                                           const float *__restrict__ partial,
                                                           const uint32_t *__restrict__ taken, uint32_t route_slots) {
  __shared__ float s_sc[cfkv::kSeamMergeMaxSlots];  // e^(m_s - m) per split (0 for splits that saw nothing)
  __shared__ float s_l, s_m;
  __shared__ int s_nan;
  const uint32_t v = blockIdx.x, kvh = blockIdx.y, dd = threadIdx.x;
  const uint32_t gqa = d.gqa_group_size, HD = d.head_dim, M = d.query_count * gqa;
  const size_t stride = static_cast<size_t>(d.kv_head_count) * M * (HD + 2);
  const float *base = partial + (static_cast<size_t>(kvh) * M + v) * (HD + 2);
  if (taken) {
    if (taken[kvh]) {
      splits = route_slots;
    } else {
      base += route_slots * stride;
      splits -= route_slots;
    }
  }
  if (dd < 64) {  // one wavefront: the splits' maxima (two per lane), their merge, the scales and l
    float ms[2], ls[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const uint32_t sp = dd + 64u * k;
      ms[k] = sp < splits ? base[sp * stride + HD] : -INFINITY;
      ls[k] = sp < splits ? base[sp * stride + HD + 1] : 0.0f;
    }
    const bool nan = __builtin_amdgcn_ballot_w64(ms[0] != ms[0] || ms[1] != ms[1]) != 0;
    float m = fmaxf((ms[0] != ms[0]) ? -INFINITY : ms[0], (ms[1] != ms[1]) ? -INFINITY : ms[1]);
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    float l = 0.0f;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const float sc = (m == -INFINITY || ms[k] == -INFINITY || ms[k] != ms[k]) ? 0.0f : __expf(ms[k] - m);
      s_sc[dd + 64 * k] = sc;
      l += ls[k] * sc;
    }
    for (int o = 32; o > 0; o >>= 1) l += __shfl_xor(l, o);
    if (dd == 0) {
      s_l = l;
      s_m = m;
      s_nan = nan;
    }
  }
  __syncthreads();
  if (dd >= HD) return;
  // the splits' rows in batches of 32, then 8, then one at a time: each batch's loads are in flight together (one
  // L2 round trip per batch, not per 8 splits), and the sum keeps the ascending split order
  float o = 0.0f;
  uint32_t s = 0;
  for (; s + 32 <= splits; s += 32) {
    float x[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) x[j] = base[(s + j) * stride + dd];
#pragma unroll
    for (int j = 0; j < 32; ++j) o += x[j] * s_sc[s + j];
  }
  for (; s + 8 <= splits; s += 8) {
    float x[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = base[(s + j) * stride + dd];
#pragma unroll
    for (int j = 0; j < 8; ++j) o += x[j] * s_sc[s + j];
  }
  for (; s < splits; ++s) o += base[s * stride + dd] * s_sc[s];
  const float l = s_l;
  d.output[(static_cast<size_t>(v / gqa) * d.query_head_count + kvh * gqa + v % gqa) * HD + dd] =
      s_nan ? __builtin_nanf("") : (l > 0.0f ? o / l : 0.0f);
  (void)s_m;
}

}  // namespace

// Split partials of the seam. Its signature has no workspace and it allocates nothing, so the partial softmax
// states of split contexts go to kSeamRegions regions of one file-scope device array per GPU (its address looked up
// once per device with hipGetSymbolAddress). Each region belongs to one stream at a time, so calls on different
// streams or threads never share partials in flight. A stream is known by its handle: the legacy default stream
// under either of its names (NULL, hipStreamLegacy) is one stream, and the per-thread default stream
// (hipStreamPerThread) is a different stream in each host thread. A handle the runtime reuses for a new stream after
// hipStreamDestroy counts as the same stream, so a stream is destroyed only after its seam calls completed, as any
// buffer its pending work reads:
//   * a stream that owns a region uses it; calls on one stream are ordered by the stream itself;
//   * a stream without one takes a free region;
//   * with every region owned by other streams, the device switches to handover mode for the rest of the process:
//     from then on each split call records an event on its stream after its merge launch, and a stream without a
//     region takes the least recently used region whose owner has recorded one, after making its own stream wait
//     for that event (hipStreamWaitEvent). Until such a region exists the call runs unsplit and uses none.
// Programs that run the seam on at most kSeamRegions streams never record an event (an event record costs ~4.5 us
// of stream time per call, 10-15 % of a short seam call). The host mutex is held from choosing the region to the
// last launch, so two threads on one stream cannot interleave their kernel and merge launches. A stream under graph
// capture cannot wait for an event recorded outside it, so there the call runs unsplit and touches no region.
constexpr uint32_t kSeamRegions = 4;
constexpr uint64_t kSeamRegionBytes = 16ull << 20;
static __device__ __align__(256) uint8_t seam_scratch[kSeamRegions * kSeamRegionBytes];

namespace {

constexpr int kMaxDevices = 64;

struct StreamKey {
  uintptr_t handle = 0;
  size_t thread = 0;  // the host thread, for the per-thread default stream only
  bool operator==(const StreamKey &o) const { return handle == o.handle && thread == o.thread; }
};

StreamKey stream_key(hipStream_t s) {
  if (s == nullptr || s == hipStreamLegacy) return {};
  if (s == hipStreamPerThread)
    return {reinterpret_cast<uintptr_t>(s), std::hash<std::thread::id>{}(std::this_thread::get_id()) | 1u};
  return {reinterpret_cast<uintptr_t>(s), 0};
}

struct SeamRegion {
  StreamKey owner;  // the owning stream
  bool owned = false;
  hipEvent_t done = nullptr;  // handover mode: recorded on the owner's stream after its last call
  bool done_valid = false;    // `done` was recorded after the owner's most recent call
  uint64_t stamp = 0;         // call counter when last used
};

struct SeamDevice {
  uint8_t *base = nullptr;
  bool handover = false;  // some stream once found every region owned by others
  uint64_t calls = 0;
  SeamRegion r[kSeamRegions];
};

std::mutex g_seam_mu;
SeamDevice g_seam[kMaxDevices];

// Region for a call on the stream `sid` (g_seam_mu held); `wait` is set when the caller must order its
// stream after the region's previous owner first. nullptr: run unsplit.
SeamRegion *seam_pick(SeamDevice &d, const StreamKey &sid, bool &wait) {
  wait = false;
  SeamRegion *fresh = nullptr, *lru = nullptr;
  for (SeamRegion &r : d.r) {
    if (r.owned && r.owner == sid) return &r;
    if (!r.owned && !fresh) fresh = &r;
    if (r.owned && r.done_valid && (!lru || r.stamp < lru->stamp)) lru = &r;
  }
  if (fresh) return fresh;
  d.handover = true;
  if (lru) wait = true;
  return lru;
}

bool stream_capturing(hipStream_t s) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &st) != hipSuccess) {
    (void)hipGetLastError();
    return true;  // unknown: take the path that needs no ordering
  }
  return st != hipStreamCaptureStatusNone;
}

uint32_t seam_cus() {
  static thread_local int cached_dev = -1;
  static thread_local uint32_t cached = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (dev != cached_dev) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cached = static_cast<uint32_t>(cus);
    cached_dev = dev;
  }
  return cached;
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
// Context splits: about two workgroups per CU over the (64-vector tile, KV head) units, at least four page chunks
// per split, at most 64 splits, and no more partials than one scratch region holds (one split writes the output
// directly and uses no region).
extern "C" cf_status cf_kv_paged_attention_async(const cf_kv_paged_attention_desc *desc, void *stream) {
  return cfkv::seam_paged_attention(desc, stream, true);
}

cf_status cfkv::seam_paged_attention(const cf_kv_paged_attention_desc *desc, void *stream, bool allow_route) {
  const cf_status valid = cf_kv_validate_paged_attention_desc(desc);
  if (valid != CF_OK) return valid;
  if (desc->kv_head_count > 65535) return CF_ERR_UNSUPPORTED;
  const uint64_t M = static_cast<uint64_t>(desc->query_count) * desc->gqa_group_size;
  const uint64_t tiles = (M + kVecs - 1) / kVecs;
  if (tiles > 0x7FFFFFFFu || M > 0x7FFFFFFFu) return CF_ERR_UNSUPPORTED;
  const uint64_t units = tiles * desc->kv_head_count;
  const uint64_t chunks_per_head = (desc->page_count + desc->kv_head_count - 1) / desc->kv_head_count +
                                   (desc->active_token_count + kChunk - 1) / kChunk;
  uint64_t splits = units >= 2ull * seam_cus() ? 1 : (2ull * seam_cus()) / units;
  splits = std::min<uint64_t>(splits, std::max<uint64_t>(1, chunks_per_head / 4));
  splits = std::min<uint64_t>(splits, 64);
  const uint64_t part_bytes = M * desc->kv_head_count * (desc->head_dim + 2) * sizeof(float);
  if (splits > 1 && part_bytes * splits > kSeamRegionBytes)
    splits = std::max<uint64_t>(1, kSeamRegionBytes / part_bytes);
  const hipStream_t s = cfd::as_stream(stream);
  const bool capturing = stream_capturing(s);
  if (splits > 1 && capturing) splits = 1;
  // the decode-shape route (kv_seam_route.hpp) when a region can hold its page lists and both sets of slots
  uint64_t route_splits = 0, route_words = 0;
  if (allow_route && !capturing && cfkv::seam_route_applies(*desc)) {
    route_splits = cfkv::seam_route_splits(*desc);
    route_words = cfkv::seam_route_scratch_words(*desc);
    splits = std::min<uint64_t>(splits, cfkv::kSeamMergeMaxSlots - route_splits);
    const uint64_t list_bytes = (route_words * 4 + 255) & ~uint64_t(255);
    if (list_bytes + part_bytes * (route_splits + splits) > kSeamRegionBytes) route_splits = 0;
  }
  const auto launch = [&](uint8_t *region) -> cf_status {
    float *partial = reinterpret_cast<float *>(region);
    const uint32_t *taken = nullptr;
    if (route_splits) {
      uint32_t *lists =
          reinterpret_cast<uint32_t *>(region + kSeamRegionBytes - ((route_words * 4 + 255) & ~uint64_t(255)));
      const cf_status rs = cfkv::seam_route_launch(*desc, static_cast<uint32_t>(route_splits), partial, lists, s);
      if (rs != CF_OK) return rs;
      taken = cfkv::seam_route_taken(*desc, lists);
    }
    const dim3 grid(static_cast<uint32_t>(tiles), desc->kv_head_count, static_cast<uint32_t>(splits));
    const uint32_t slot0 = static_cast<uint32_t>(route_splits);
    if (desc->head_dim <= 64)
      seam_kernel<64><<<grid, kThreads, 0, s>>>(*desc, static_cast<uint32_t>(splits), partial, taken, slot0);
    else
      seam_kernel<128><<<grid, kThreads, 0, s>>>(*desc, static_cast<uint32_t>(splits), partial, taken, slot0);
    if (partial)
      seam_merge_kernel<<<dim3(static_cast<uint32_t>(M), desc->kv_head_count), kMaxD, 0, s>>>(
          *desc, static_cast<uint32_t>(route_splits + splits), partial, taken, slot0);
    return cfd::launch_status();
  };
  if (splits == 1 && !route_splits) return launch(nullptr);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return CF_ERR_CUDA;
  const StreamKey sid = stream_key(s);
  std::lock_guard<std::mutex> lock(g_seam_mu);  // held from choosing the region to the last launch
  SeamDevice &sd = g_seam[dev];
  if (!sd.base) {
    void *addr = nullptr;
    if (hipGetSymbolAddress(&addr, HIP_SYMBOL(seam_scratch)) != hipSuccess) return CF_ERR_CUDA;
    sd.base = static_cast<uint8_t *>(addr);
  }
  bool wait = false;
  SeamRegion *r = seam_pick(sd, sid, wait);
  if (!r) {  // every region is owned by another stream that has not recorded an event yet
    splits = 1;
    route_splits = 0;
    return launch(nullptr);
  }
  if (wait && hipStreamWaitEvent(s, r->done, 0) != hipSuccess) return CF_ERR_CUDA;
  r->owner = sid;
  r->owned = true;
  r->done_valid = false;
  r->stamp = ++sd.calls;
  const cf_status st = launch(sd.base + static_cast<uint64_t>(r - sd.r) * kSeamRegionBytes);
  if (sd.handover) {
    if (!r->done && hipEventCreateWithFlags(&r->done, hipEventDisableTiming) != hipSuccess) {
      r->done = nullptr;
      return CF_ERR_CUDA;
    }
    if (hipEventRecord(r->done, s) != hipSuccess) return CF_ERR_CUDA;
    r->done_valid = true;
  }
  return st;
}
