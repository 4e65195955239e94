// kv_batched.hip — batched compressed paged-KV attention decode on gfx950 (kv_codec_ext.h entry point).
//
// One workgroup serves one (sequence, KV head, context split): 12 wavefronts (one workgroup per CU) for long
// contexts, 4 (three workgroups per CU) for short ones. In a 12-wavefront workgroup each wavefront takes a contiguous
// block of the split's chain pairs sized by its issue priority (arbitration favours the oldest wavefront of a SIMD),
// so that all finish together. Each wavefront walks "page quads": four consecutive 16-token pages, one per 16-lane
// group. Lane (G, t) = lane 16G + t:
//   K phase: lane decodes token t of page G (its 16 interleaved rANS states are the 16 lanes of the group);
//            every decoded quad of 4 dims goes straight into v_mfma_f32_4x4x4f16 as the B operand, with the
//            GQA group's 4 query heads (split into f16 hi + lo parts for fp32-grade scores) as the A operand, so
//            the lane ends up holding its token's 4 head scores. Nothing decoded is written anywhere.
//   softmax: one running max per head for the whole wavefront (so the 4 page groups can be summed at the end),
//            probabilities times the page's V scale (in units of a power of two per wavefront, so that the f16 value
//            neither underflows nor overflows), split into f16 hi + lo parts, go to two 512-byte LDS tiles.
//   V phase: lane decodes dims {t + 16i} of page G, 4 tokens per quad; two quads (8 tokens) of each of the 4 pages
//            are the k = 32 of one v_mfma_f32_16x16x32_f16 whose rows are 4 heads x {hi, lo} weight parts and whose
//            16 columns are dims 16i .. 16i + 15 (B = the decoded values as exact signed f16): 16 MFMAs per group
//            where 4x4x4 MFMAs would take 64. With one f16 per weight (11
//            significant bits) an output made of near-cancelling terms (weights of different pages, whose V scales
//            differ) would carry an error of ~2^-12 of the terms themselves; hi + lo leaves ~2^-22.
// Codec decode (format 4): one rANS step per 8 values of a stream (LDS slot table, 64-bit entry = freq/offset +
// the symbol's 8 big bits spread to their frame positions; SDWA reads the 16-bit freq/offset halves in place); the
// raw nibble, crumb and sign words of the lane merged with two bit-field inserts and a rotation per quad; two
// v_perm build the exact f16 operand (sign-magnitude bytes read as f16 denormals = q * 2^-24). INT8 groups (the
// raw fallback) use 1024 + symbol operands with the 1152 offset folded out of the scores and subtracted from V.
// Memory: a wavefront's next group is in flight while it works on the current one (header in registers, word
// streams copied straight into LDS by global_load_lds after the current decode loop, first low-part words in
// registers), so a group starts without a memory round trip.
// Split-context partial states (m, l, acc) are merged by a second small kernel (online-softmax merge,
// reference src/runtime/kv_runtime.cpp:219-243 semantics).
#include <hip/hip_fp16.h>

#include <cmath>
#include <cstring>
#include <mutex>
#include <utility>

#include "cf_device.hpp"
#include "chromofold/kv_codec_ext.h"
#include "kv_group_decode.hpp"
#include "kv_seam_route.hpp"

namespace {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));

// Occupancy floor for the compiler (3 wavefronts per SIMD: <= 168 VGPRs); the LDS footprint below allows one
// 12-wavefront or three 4-wavefront workgroups per CU.
#ifndef CF_KV_WPE
#define CF_KV_WPE 3
#endif
constexpr int kWavesWide = 12;   // one workgroup per CU
constexpr int kWavesNarrow = 4;  // three workgroups per CU
constexpr int kGqa = 4;            // MFMA rows: query heads of one KV head (gqa < 4 pads with zero queries)
using cfkv::bfi;
using cfkv::kFrame;
using cfkv::kHdr;
using cfkv::kNWord;
using cfkv::kSlots;
using cfkv::kStateBytes;
using cfkv::quad_mag;
using cfkv::quad_signs;
using cfkv::rans_advance;
using cfkv::rans_lookup;
constexpr float kOffset = 1152.0f;  // f16 operand = 1024 + symbol, symbol = q + 128

__device__ __forceinline__ half4_t bytes_to_half4(uint32_t b) {
  const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, b, 0x04010400u);  // [s0,0x64,s1,0x64]
  const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, b, 0x04030402u);  // [s2,0x64,s3,0x64]
  half4_t h;
  uint32_t *w = reinterpret_cast<uint32_t *>(&h);
  w[0] = lo;
  w[1] = hi;
  return h;
}

// The same bytes as exact signed values (symbol - 128) in f16: the 1024 + 128 offset removed by a packed f16
// subtract (exact: integers in [-128, 127]). The V operand uses this form: with the offset left in, a row whose
// heaviest tokens have V = 0 would carry 1152 x (sum of their weights) in an fp32 accumulator whose true value
// is many orders of magnitude smaller.
__device__ __forceinline__ half4_t bytes_to_half4_signed(uint32_t b) {
  const half4_t off = {static_cast<_Float16>(-1152.0f), static_cast<_Float16>(-1152.0f),
                       static_cast<_Float16>(-1152.0f), static_cast<_Float16>(-1152.0f)};
  return bytes_to_half4(b) + off;
}

__device__ __forceinline__ float4_t mfma4(half4_t a, half4_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_4x4x4f16(a, b, c, 0, 0, 0);
}

// Exact f16 operand of four sign-magnitude values: the f16 denormals (sign << 15) | |q| = q * 2^-24.
__device__ __forceinline__ half4_t sm_to_half4(uint32_t mag, uint32_t signs) {
  half4_t h;
  uint32_t *w = reinterpret_cast<uint32_t *>(&h);
  w[0] = __builtin_amdgcn_perm(signs, mag, 0x05010400u);  // [|q0|, s0, |q1|, s1]
  w[1] = __builtin_amdgcn_perm(signs, mag, 0x07030602u);
  return h;
}

constexpr uint32_t kCapWords = CF_KV_RANS_MAX_GROUP_WORDS;  // K+V words staged in LDS per wavefront
constexpr uint32_t kSlackWords = 64;     // reads past the last word by non-renormalising lanes stay in the buffer

template <int D>
constexpr int raw_words() {  // u32 raw words of one stream of a RANS group
  return cfkv::raw_words_of(D);
}

template <int D>
constexpr int buf_u32() {
  constexpr int words = (kCapWords + kSlackWords) / 2;
  constexpr int red = kGqa * (D + 2);
  return words > red ? words : red;
}

// Max over the 64 lanes of four values at once, as wave-uniform values: v_max_f32_dpp within each row (quad_perm
// [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror), then row_bcast:15 (rows 1, 3) and row_bcast:31 (rows 2, 3)
// fold the rows into lane 63, which is read. One asm statement, so that nothing the compiler emits lands between
// the steps: the four chains are interleaved, so each DPP source was written three VALU instructions earlier, and
// the leading s_nop 1 gives the two wait states a DPP read needs after the write of its source before the block.
// Replaces six rounds of ds_bpermute (an LDS round trip each) on the softmax's dependency chain: -2 to -3 % per
// launch at C4.
__device__ __forceinline__ void wave64_max4(float (&x)[4]) {
#define CF_DPP4(CTL)                                                                                                \
  "v_max_f32_dpp %0, %0, %0 " CTL "\n\tv_max_f32_dpp %1, %1, %1 " CTL "\n\tv_max_f32_dpp %2, %2, %2 " CTL        \
  "\n\tv_max_f32_dpp %3, %3, %3 " CTL "\n\t"
  asm volatile("s_nop 1\n\t"
               CF_DPP4("quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf")
               CF_DPP4("quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf")
               CF_DPP4("row_half_mirror row_mask:0xf bank_mask:0xf")
               CF_DPP4("row_mirror row_mask:0xf bank_mask:0xf")
               CF_DPP4("row_bcast:15 row_mask:0xa bank_mask:0xf")
               CF_DPP4("row_bcast:31 row_mask:0xc bank_mask:0xf")
               : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]));
#undef CF_DPP4
#pragma unroll
  for (int h = 0; h < 4; ++h) x[h] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x[h]), 63));
}

// Decode one page group (K scores, softmax, V accumulation).
// RANS groups: `st` holds the chain's lane states on entry (K, V) and the states the group ends with on return;
// the word streams are read through `wk` (the wave's LDS staging buffer, K stream then V); `raw` points at the
// group's raw words. `pre` holds 14 raw words (7 K + 7 V): on entry the group's first sign group, on return the
// first sign group of the next RANS group at `nlw` (NULL if none); in between, each word of sign group s + 1 is
// loaded into its slot as soon as sign group s no longer needs that slot.
// INT8 groups: `raw` points at the symbol words (offset binary).
// `after_decode` runs as soon as the decode loop no longer needs the word buffer (the caller stages the next group
// there).
// V quads 0..KL-1 do not wait for the V phase in registers: the decode parks them in the wave's LDS area `vl`
// ([KL][64] words) (RANS), or the V phase loads them again from `raw` (INT8 groups, rare in the launches that use
// KL > 0). The registers this frees keep the 12-wave kernel free of spills.
// With kEnds (RANS groups), `ends` receives where the K and V word cursors stopped (words from the K stream's start),
// so that a caller can check that a self-contained group consumed exactly its words. With kPageVis, `page_vis`
// tells whether any token of the lane's 16-token page is visible (for callers whose visible tokens are not a prefix
// of each page, e.g. behind a causal window); otherwise tok_ok of the page's first lane says it. kStreamRaw: INT8
// groups' words are read with non-temporal loads (for launches whose groups are each read once).
template <int D, int CODEC, int KL, typename WordPtr, typename Hook, bool kEnds = false, bool kPageVis = false,
          bool kStreamRaw = false>
__device__ __forceinline__ void group_body(const Hook &after_decode, uint32_t (&pre)[14], const uint32_t *nlw,
                                           uint32_t (&st)[2], const uint32_t *__restrict__ raw, WordPtr wk,
                                           uint32_t cnt_kv, const uint2 (*__restrict__ s_tab)[kSlots],
                                           const half4_t *qhi, const half4_t *qlo, const float *qsum,
                                           _Float16 (*s_pw)[4][kGqa][16], uint32_t *__restrict__ vl, int lane,
                                           bool tok_ok, float ks, float vs, int &e_run, float *m_run, float *l_run,
                                           float4_t *acc_v, uint32_t *ends = nullptr, bool page_vis = false) {
  constexpr int NQ = D / 4, RAW = raw_words<D>();
  constexpr bool RANS = CODEC == CF_KV_CODEC_RANS_HYBRID;
  const int G = lane >> 4, t = lane & 15;
  float4_t sa = {0, 0, 0, 0}, sb = {0, 0, 0, 0};
  uint32_t vb[NQ];                         // V: magnitude bytes (RANS) or offset-binary symbols (INT8) per quad
  auto put_v = [&](auto qc, uint32_t v) {
    constexpr int q = decltype(qc)::value;
    if constexpr (q < KL) vl[q * 64 + lane] = v;
    else vb[q] = v;
  };
  uint32_t vsg[RANS ? D / 32 : 1];         // V sign words per sign group (RANS)
  // K MFMAs of quad q (A = the 4 query heads broadcast from block q % 16, hi and lo parts)
  auto k_mfma = [&](auto qc, half4_t bk) {
    constexpr int q = decltype(qc)::value;
    sa = __builtin_amdgcn_mfma_f32_4x4x4f16(qhi[q / 16], bk, sa, 4, q % 16, 0);
    sb = __builtin_amdgcn_mfma_f32_4x4x4f16(qlo[q / 16], bk, sb, 4, q % 16, 0);
  };
  if constexpr (RANS) {
    uint32_t xk = st[0], xv = st[1];
    // word cursors of the two streams (wave-uniform: scalar registers; their advance is scalar work)
    const uint32_t ckv = __builtin_amdgcn_readfirstlane(cnt_kv);
    WordPtr wkk = wk, wvv = wk + (ckv & 0xFFFFu);
    // pre[] holds this sign group's raw words (K N0 N1 C0 N2 N3 C1 S, then V the same); each slot is refilled with
    // the next sign group's word right after its last use here (at least three steps before that word is needed),
    // and the next sign words go to snx at the sign group's first step.
    uint32_t snx[2] = {0, 0};
    auto refill = [&](auto sgc, auto wc) {  // slots w (K) and 7 + w (V) <- word w of sign group sgc + 1
      constexpr int sn = decltype(sgc)::value + 1, w = decltype(wc)::value;
      if constexpr (sn < D / 32) {
        pre[w] = raw[(7 * sn + w) * 64 + lane];
        pre[7 + w] = raw[RAW + (7 * sn + w) * 64 + lane];
      } else if (nlw) {
        pre[w] = nlw[w * 64 + lane];
        pre[7 + w] = nlw[RAW + w * 64 + lane];
      }
    };
    // step P decodes quads 2P and 2P + 1 of K and of V: two independent rANS steps
    [&]<int... P>(std::integer_sequence<int, P...>) {
      (
          [&] {
            constexpr int sg = P / 4, m = P % 4, q0 = 2 * P;
            constexpr uint32_t rA = kFrame[2 * m], rB = kFrame[2 * m + 1];
            using SG = std::integral_constant<int, sg>;
            if constexpr (m == 0) {
              vsg[sg] = pre[13];  // V signs, kept for the V phase
              if constexpr (sg + 1 < D / 32) {
                snx[0] = raw[(7 * (sg + 1) + 6) * 64 + lane];
                snx[1] = raw[RAW + (7 * (sg + 1) + 6) * 64 + lane];
              } else if (nlw) {
                snx[0] = nlw[6 * 64 + lane];
                snx[1] = nlw[RAW + 6 * 64 + lane];
              }
            }
            const uint2 ek = rans_lookup(s_tab[0], xk), ev = rans_lookup(s_tab[1], xv);
            uint32_t selk, selv;
            const uint32_t wdk = rans_advance(ek.x, xk, wkk, selk);
            const uint32_t wdv = rans_advance(ev.x, xv, wvv, selv);
            xk = __builtin_amdgcn_perm(xk, wdk, selk);
            xv = __builtin_amdgcn_perm(xv, wdv, selv);
            // the spread words hold the big bits in the frames (0, 4): rotate them into this pair's frames
            const uint32_t spk = rA ? __builtin_amdgcn_alignbit(ek.y, ek.y, 32 - rA) : ek.y;
            const uint32_t spv = rA ? __builtin_amdgcn_alignbit(ev.y, ev.y, 32 - rA) : ev.y;
            constexpr int nw = kNWord[m], cwi = m < 2 ? 2 : 5;
            k_mfma(std::integral_constant<int, q0>{},
                   sm_to_half4(quad_mag<rA>(pre[nw], pre[cwi], spk), quad_signs<rA>(pre[6])));
            k_mfma(std::integral_constant<int, q0 + 1>{},
                   sm_to_half4(quad_mag<rB>(pre[nw], pre[cwi], spk), quad_signs<rB>(pre[6])));
            put_v(std::integral_constant<int, q0>{}, quad_mag<rA>(pre[7 + nw], pre[7 + cwi], spv));
            put_v(std::integral_constant<int, q0 + 1>{}, quad_mag<rB>(pre[7 + nw], pre[7 + cwi], spv));
            // refill what this step used for the last time in this sign group
            refill(SG{}, std::integral_constant<int, nw>{});
            if constexpr (m == 1 || m == 3) refill(SG{}, std::integral_constant<int, cwi>{});
            if constexpr (m == 3) {
              pre[6] = snx[0];
              pre[13] = snx[1];
            }
          }(),
          ...);
    }(std::make_integer_sequence<int, D / 8>{});
    st[0] = xk;
    st[1] = xv;
    if constexpr (kEnds) {
      ends[0] = static_cast<uint32_t>(wkk - wk);
      ends[1] = static_cast<uint32_t>(wvv - wk);
    }
  } else {
    if (nlw) {  // a raw group: start the next RANS group's first raw words now
#pragma unroll
      for (int w = 0; w < 7; ++w) {
        pre[w] = nlw[w * 64 + lane];
        pre[7 + w] = nlw[RAW + w * 64 + lane];
      }
    }
    // with kStreamRaw the words go past the caches (non-temporal): ~12 % faster at C4's 2.2 GB of INT8 groups read
    // once each, but raw groups that many sequences share (a prefix inside a RANS pool) need the caches
    auto ld = [&](const uint32_t *p) { return kStreamRaw ? __builtin_nontemporal_load(p) : *p; };
    [&]<int... Q>(std::integer_sequence<int, Q...>) {
      ((Q < KL ? void() : void(vb[Q] = ld(&raw[NQ * 64 + Q * 64 + lane])),
        k_mfma(std::integral_constant<int, Q>{}, bytes_to_half4(ld(&raw[Q * 64 + lane])))),
       ...);
    }(std::make_integer_sequence<int, NQ>{});
  }
  after_decode();  // the word buffer is free from here on

  // ---- online softmax over the wavefront's 64 tokens (one running max per head for all four pages)
  // K operands: RANS = q * 2^-24 (f16 denormals); INT8 = 1024 + symbol, the 1152 offset folded out with the query sum
  const float ksc = RANS ? ks * 16777216.0f : ks;
  float s[kGqa], mx[kGqa];
#pragma unroll
  for (int h = 0; h < kGqa; ++h) {
    s[h] = tok_ok ? (RANS ? (sa[h] + sb[h]) : (sa[h] + sb[h] - kOffset * qsum[h])) * ksc : -INFINITY;
    mx[h] = s[h];
  }
  static_assert(kGqa == 4, "wave64_max4 reduces four heads");
  wave64_max4(mx);
  // P.V runs on v_mfma_f32_16x16x32_f16 with k = 8 tokens of each of the 4 pages (page G's from lane group G), so
  // one MFMA sums all four pages: rows 0-3 are the 4 heads' hi parts of the weights p * v_scale, rows 4-7 their lo
  // parts (rows 8-15 repeat rows 0-7 and are dropped), 16 dims per MFMA. The lane's accumulators acc_v hold rows
  // 4G..4G+3: the hi (G = 0) or lo (G = 1) sums. The wavefront keeps them in units of 2^e_run with e = (exponent of
  // the group's largest V scale among its pages with a visible token) - 15 (+ 24 for RANS groups, whose V operands
  // are q * 2^-24): every f16 weight lies in [0, 2^15) whatever the V magnitude, weights down to 2^-29 of the
  // running maximum stay normal f16 numbers (a row whose heaviest tokens have V = 0 is carried by such small
  // weights), and hi + lo keep ~22 bits for every page within 2^18 of the group's largest V scale (the lo part of a
  // page further below loses bits gradually: ~16 bits at 2^24, those of one f16 at 2^29). Moving to new units is an
  // exact power-of-two factor folded into the softmax rescale; a drop of more than 2^60 is clamped so that the
  // rescale cannot overflow.
  constexpr int kOpExp = RANS ? 24 : 0;
  constexpr int kNone = -(1 << 24);
  // tokens are visible as a prefix of each page, so a page's lane 16 G is visible iff any of its tokens is
  const int ep = (kPageVis ? page_vis : tok_ok) ? __builtin_amdgcn_frexp_expf(vs) - 15 + kOpExp : kNone;
  const int eb = max(max(__builtin_amdgcn_readlane(ep, 0), __builtin_amdgcn_readlane(ep, 16)),
                     max(__builtin_amdgcn_readlane(ep, 32), __builtin_amdgcn_readlane(ep, 48)));
  const int nb = eb != kNone ? max(eb, e_run - 60) : e_run;
  const int de = e_run - nb;
  e_run = nb;
  const float vsn = ldexpf(vs, kOpExp - nb);
  float alpha[kGqa], pr[kGqa];
#pragma unroll
  for (int h = 0; h < kGqa; ++h) {
    const float mn = fmaxf(m_run[h], mx[h]);
    const float a = (m_run[h] == -INFINITY) ? 0.0f : __expf(m_run[h] - mn);
    pr[h] = tok_ok ? __expf(s[h] - mn) : 0.0f;
    l_run[h] = l_run[h] * a + pr[h];
    alpha[h] = ldexpf(a, de);  // ldexp(0, .) = 0 before the first visible token
    m_run[h] = mn;
  }
#pragma unroll
  for (int h = 0; h < kGqa; h += 2)
    cfd::split2_mul_f16(pr[h], pr[h + 1], vsn, s_pw[0][G][h][t], s_pw[1][G][h][t], s_pw[0][G][h + 1][t],
                        s_pw[1][G][h + 1][t]);
#pragma unroll
  for (int i = 0; i < D / 16; ++i)
#pragma unroll
    for (int h = 0; h < kGqa; ++h) acc_v[i][h] *= alpha[h];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // ---- V MFMAs: rows {hi, lo} x heads, k = tokens 8 tp .. 8 tp + 7 of every page, cols = dims 16 i .. 16 i + 15.
  // A: lane (G, t) gives row t for page G (rows 8-15 read rows 0-7's weights); B: its V quads of tokens
  // 8 tp .. + 3 and 8 tp + 4 .. + 7 at dim 16 i + t.
  auto v_quad = [&](auto qc) {
    constexpr int q = decltype(qc)::value;  // quad q = tokens 4 (q / (D / 16)) .. + 3 at dim t + 16 (q % (D / 16))
    if constexpr (RANS)  // quad q is quad q % 8 of sign group q / 8
      return sm_to_half4(q < KL ? vl[q * 64 + lane] : vb[q], quad_signs<kFrame[q % 8]>(vsg[q / 8]));
    else
      return bytes_to_half4_signed(q < KL ? raw[NQ * 64 + q * 64 + lane] : vb[q]);
  };
  [&]<int... TP>(std::integer_sequence<int, TP...>) {
    (
        [&] {
          constexpr int tp = TP;
          // Read in inline asm: the compiler cannot tell this tile from the word buffer that the next group's
          // global_load_lds copies are filling, and for a plain LDS read it would first wait for those copies
          // (s_waitcnt vmcnt(0)), i.e. for the next group's whole prefetch, in the middle of every group. The
          // tile was written by this wavefront's own ds_write instructions, which the LDS executes in order.
          half8_t pa;
          asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)"
                       : "=v"(pa)
                       : "v"(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(&s_pw[(t >> 2) & 1][G][t & 3][8 * tp])))
                       : "memory");
          [&]<int... I>(std::integer_sequence<int, I...>) {
            (
                [&] {
                  constexpr int i = I;
                  const half4_t b0 = v_quad(std::integral_constant<int, (2 * tp) * (D / 16) + i>{});
                  const half4_t b1 = v_quad(std::integral_constant<int, (2 * tp + 1) * (D / 16) + i>{});
                  const half8_t bv = __builtin_shufflevector(b0, b1, 0, 1, 2, 3, 4, 5, 6, 7);
                  acc_v[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, bv, acc_v[i], 0, 0, 0);
                }(),
                ...);
          }(std::make_integer_sequence<int, D / 16>{});
        }(),
        ...);
  }(std::make_integer_sequence<int, 2>{});
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

#if CF_KV_WPE > 0
#define CF_KV_OCC __attribute__((amdgpu_waves_per_eu(CF_KV_WPE, 8)))
#else
#define CF_KV_OCC
#endif

// Partial-state slots of one (sequence, KV head) in the split workspace: this launch's splits write slots
// [slot0, slot0 + splits) of `slots`; with slots == 1 the kernel writes the output directly. The launch covers the
// sequence's groups from g0 on (a cascade launch leaves the shared prefix groups [0, g0) to the prefix kernel).
struct SplitSlots {
  uint32_t g0, slot0, slots;
};

// Narrow workgroups: a wave's groups are the pairs (2k, 2k + 1), k = k0 + wave, k0 + wave + 4, ..., clipped to the
// split's [ga, gb).
__device__ __forceinline__ uint32_t next_group_strided(uint32_t g, uint32_t gb) {
  if ((g & 1u) == 0 && g + 1 < gb) return g + 1;
  const uint32_t n = ((g >> 1) + kWavesNarrow) * 2;
  return n < gb ? n : gb;
}

// Wide workgroups: wavefront w (SIMD w % 4; the w / 4-th oldest of that SIMD's three) takes a contiguous block of the
// split's pairs in proportion to kSlotWeight[w / 4], the relative rates at which MI355X's issue arbitration lets the
// oldest, middle and youngest wavefront of a SIMD progress in this kernel (measured on the C4 shape: with the ticket
// that handed pairs out dynamically, the three took 48 : 44 : 36 groups in 359 : 368 : 372 us). Static blocks keep
// the result bitwise reproducible; equal blocks left the youngest wavefronts finishing ~15 % after the oldest.
constexpr uint32_t kSlotWeight[3] = {139, 124, 100};
constexpr uint32_t kSlotWeightSum = 4 * (kSlotWeight[0] + kSlotWeight[1] + kSlotWeight[2]);

// Pairs [lo, hi) of `np` that wavefront w of a wide workgroup takes: counts c_w that minimise the latest finish
// max_w c_w / rate_w (rate = kSlotWeight of w's age slot), in wavefront order. Every wavefront first takes
// floor(np * rate / sum of rates); the remaining d < 12 pairs go one each to the d wavefronts that would finish
// their extra pair earliest ((c_w + 1) / rate_w, ties to the lower index). With few pairs per wavefront (short
// contexts) this keeps the slowest age slot from being the one that rounds up.
__device__ __forceinline__ void wide_block(uint32_t w, uint32_t np, uint32_t &lo, uint32_t &hi) {
  auto rate = [](uint32_t v) { return kSlotWeight[(v >> 2) < 3 ? (v >> 2) : 2]; };
  auto base = [&](uint32_t v) {
    return static_cast<uint32_t>((static_cast<uint64_t>(np) * rate(v)) / kSlotWeightSum);
  };
  uint32_t given = 0;
  for (uint32_t v = 0; v < kWavesWide; ++v) given += base(v);
  const uint32_t d = np - given;  // < kWavesWide
  // wavefront v gets an extra pair iff fewer than d wavefronts precede it in the order (c + 1) / rate, index
  auto extra = [&](uint32_t v) {
    const uint64_t kv = static_cast<uint64_t>(base(v) + 1);
    uint32_t ahead = 0;
    for (uint32_t u = 0; u < kWavesWide; ++u) {
      const uint64_t ku = static_cast<uint64_t>(base(u) + 1);
      // (ku / rate(u) < kv / rate(v)) or equal with u < v
      const uint64_t l = ku * rate(v), r = kv * rate(u);
      ahead += (l < r || (l == r && u < v)) ? 1u : 0u;
    }
    return ahead < d ? 1u : 0u;
  };
  lo = 0;
  for (uint32_t v = 0; v < w; ++v) lo += base(v) + extra(v);
  hi = lo + base(w) + extra(w);
}

template <int D, int CODEC, int W>
__global__ CF_KV_OCC __launch_bounds__(64 * W) void kv_batched_kernel(cf_kv_batched_desc d, uint32_t splits,
                                                                       float *__restrict__ partial, SplitSlots ss) {
  constexpr int NQ = D / 4;
  constexpr int RAW = raw_words<D>();
  constexpr bool RANS = CODEC == CF_KV_CODEC_RANS_HYBRID;
  constexpr int BUF = buf_u32<D>();
  constexpr int kThreads = 64 * W;
  constexpr bool kWide = W == kWavesWide;           // contiguous weighted pair blocks (else strided pairs)
  constexpr int KL = kWide && RANS ? 16 : 0;        // V quads parked in LDS (see group_body)
  __shared__ __attribute__((aligned(16))) uint2 s_tab[RANS ? 2 : 1][kSlots];  // {f | c << 16, spread big bits} per
                                                                              // slot, K and V tables
  __shared__ __attribute__((aligned(16))) _Float16 s_p[W][2][4][kGqa][16];  // per wave: [hi, lo][page][head][token]
                                                                          // probability * v_scale
  __shared__ uint32_t s_buf[W][BUF];                // per wave: staged words; query staging and partials alias it
  __shared__ uint32_t s_vl[KL ? W : 1][KL ? KL : 1][64];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int G = lane >> 4, t = lane & 15;
  const uint32_t split = blockIdx.x, head = blockIdx.y, seq = blockIdx.z;
  const uint32_t gqa = d.query_head_count / d.kv_head_count;
  static_assert(2 * kGqa * D * 2 <= W * BUF * 4, "query staging must fit the word buffers");
  _Float16(*s_q)[kGqa][D] = reinterpret_cast<_Float16(*)[kGqa][D]>(&s_buf[0][0]);

  // ---- stage tables and queries
  if constexpr (RANS) {
    // K table then V table (adjacent blobs), two entries per 16-byte load; every load of a thread is issued before
    // its first LDS write (one memory latency instead of one per loop step; the tail loads repeat the last pair)
    const uint4 *tk = reinterpret_cast<const uint4 *>(d.tables + static_cast<size_t>(2 * head) * CF_KV_RANS_TABLE_BYTES);
    constexpr uint32_t kPairs = kSlots;  // 2 * kSlots entries
    constexpr int kIt = static_cast<int>((kPairs + kThreads - 1) / kThreads);
    uint4 e[kIt];
#pragma unroll
    for (int k = 0; k < kIt; ++k) e[k] = tk[min(threadIdx.x + static_cast<uint32_t>(k * kThreads), kPairs - 1)];
#pragma unroll
    for (int k = 0; k < kIt; ++k) {
      const uint32_t i = threadIdx.x + static_cast<uint32_t>(k * kThreads), j = 2 * i;
      if (i < kPairs)
        *reinterpret_cast<uint4 *>(&s_tab[j / kSlots][j % kSlots]) =
            uint4{(e[k].x & 2047u) | (((e[k].x >> 11) & 2047u) << 16), e[k].y,
                  (e[k].z & 2047u) | (((e[k].z >> 11) & 2047u) << 16), e[k].w};
    }
  }
  for (int i = threadIdx.x; i < kGqa * D; i += kThreads) {
    const int h = i / D, dd = i % D;
    const float q = static_cast<uint32_t>(h) < gqa
                        ? d.queries[(static_cast<size_t>(seq) * d.query_head_count + head * gqa + h) * D + dd]
                        : 0.0f;
    cfd::split_mul_f16(q, d.softmax_scale, s_q[0][h][dd], s_q[1][h][dd]);
  }
  __syncthreads();

  // Query operands held in registers for the whole kernel: lane (block b = lane/4, row i = lane%4) keeps head i's
  // dims of quad 16c + b; the K MFMA of quad q broadcasts block q%16's A operand to all 16 blocks (CBSZ 4).
  constexpr int NC = NQ / 16 > 0 ? NQ / 16 : 1;
  half4_t qhi[NC], qlo[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int qd = 16 * c + (lane >> 2);
    qhi[c] = (4 * qd < D) ? *reinterpret_cast<const half4_t *>(&s_q[0][lane & 3][4 * qd]) : half4_t{0, 0, 0, 0};
    qlo[c] = (4 * qd < D) ? *reinterpret_cast<const half4_t *>(&s_q[1][lane & 3][4 * qd]) : half4_t{0, 0, 0, 0};
  }
  // per-head sum of the query operand as the MFMA sees it, for the 1152 offset fold of INT8 groups (lanes 16h..
  // reduce head h)
  float qsum[kGqa];
  {
    float part = 0.0f;
    const int h = lane >> 4;
#pragma unroll
    for (int k = 0; k < D / 16; ++k) {
      const int dd = (lane & 15) * (D / 16) + k;
      part += static_cast<float>(s_q[0][h][dd]) + static_cast<float>(s_q[1][h][dd]);
    }
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) part += __shfl_xor(part, o);
#pragma unroll
    for (int hh = 0; hh < kGqa; ++hh) qsum[hh] = __shfl(part, 16 * hh);
  }
  __syncthreads();  // s_q (aliasing the word buffers) is dead from here on

  const uint32_t ntok_seq = d.seq_tokens[seq];
  const uint32_t qpos = d.query_pos[seq];
  const uint32_t visible = min(ntok_seq, qpos + 1);  // tokens [0, visible) are attended
  const uint32_t ngroups = min((visible + 63) / 64, d.max_groups);
  const uint32_t g0 = min(ss.g0, ngroups);
  // splits cover whole group pairs: pairs [p0, p1) over groups [g0, ngroups)
  const uint32_t p0 = g0 >> 1, p1 = (ngroups + 1) >> 1;
  const uint32_t per = (p1 - p0 + splits - 1) / splits;
  const uint32_t pa = min(p1, p0 + split * per), pb = min(p1, pa + per);
  const uint32_t ga = max(g0, 2 * pa), gb = min(ngroups, 2 * pb);
  const uint32_t *grow = d.group_offsets + (static_cast<size_t>(seq) * d.kv_head_count + head) * d.max_groups;

  float m_run[kGqa], l_run[kGqa];
  int e_run = -(1 << 20);  // exponent of the wavefront's P.V units (set by its first group; see group_body)
  float4_t acc_v[D / 16];
#pragma unroll
  for (int h = 0; h < kGqa; ++h) {
    m_run[h] = -INFINITY;
    l_run[h] = 0.0f;
  }
#pragma unroll
  for (int i = 0; i < D / 16; ++i) acc_v[i] = float4_t{0, 0, 0, 0};

  uint32_t *buf = s_buf[__builtin_amdgcn_readfirstlane(wave)];  // uniform base: cursor arithmetic stays scalar
  uint32_t *vl = &s_vl[KL ? __builtin_amdgcn_readfirstlane(wave) : 0][0][0];
  // A wavefront's groups: pairs (2k, 2k + 1), clipped to the split's [ga, gb); the groups of a pair are decoded back
  // to back by the same wavefront (a RANS chain may run across them). Wide workgroups: one contiguous block of pairs
  // per wavefront (wide_block), i.e. the consecutive groups [w_begin, w_end). Narrow: next_group_strided.
  uint32_t w_begin = gb, w_end = gb;
  if constexpr (kWide) {
    uint32_t lo, hi;
    wide_block(static_cast<uint32_t>(wave), pb - pa, lo, hi);
    if (lo < hi) {
      w_begin = max(ga, 2 * (pa + lo));
      w_end = min(gb, 2 * (pa + hi));
    }
  }
  auto stream_next = [&](uint32_t prev) {
    if (prev >= gb) return gb;
    if constexpr (kWide) return prev + 1 < w_end ? prev + 1 : gb;
    else return next_group_strided(prev, gb);
  };
  // Memory pipeline of a wavefront over its groups:
  //   blob offset   loaded two groups ahead;
  //   header        loaded at the start of the previous group (fields and chain-start lane states kept in
  //                 registers; the two state words are read for every group and used only by chain starts);
  //   word streams  copied into this wave's LDS buffer by global_load_lds (16 bytes per lane, 1 KiB per wave
  //                 instruction, whole 16-byte chunks: blobs are padded to 16 bytes) during the previous group's
  //                 softmax / V phase — the buffer is free once that group's decode loop has ended;
  //   raw words     rolling prefetch: the next sign group's 14 words per lane are always in flight (issued when the
  //                 previous sign group starts; across the group boundary for the last one).
  // The next group's copies are awaited with s_waitcnt vmcnt(0) at the top of the loop.
  auto blob_at = [&](uint32_t g) { return d.pool + static_cast<size_t>(grow[g]) * 16; };
  const uint32_t gfirst = kWide ? (w_begin < w_end ? w_begin : gb)
                               : ((2 * (pa + wave) < gb) ? max(ga, 2 * (pa + wave)) : gb);
  uint32_t g_next = stream_next(gfirst);
  uint32_t off_next = g_next < gb ? grow[g_next] : 0u;
  const uint8_t *blob = gfirst < gb ? blob_at(gfirst) : d.pool;
  uint32_t h_cnt = 0, h_chain = 0, h_tc = 0, h_codec = 0;
  uint32_t h_st[2] = {0, 0};  // the group's chain-start lane states (read for every group: harmless, unused)
  float h_ks = 0.f, h_vs = 0.f;
  auto load_header = [&](const uint8_t *b) {
    h_st[0] = reinterpret_cast<const uint32_t *>(b + kHdr)[lane];
    h_st[1] = reinterpret_cast<const uint32_t *>(b + kHdr)[64 + lane];
    h_cnt = *reinterpret_cast<const uint32_t *>(b + 4);
    h_chain = *reinterpret_cast<const uint16_t *>(b + 8);
    h_tc = reinterpret_cast<const uint16_t *>(b + 12)[G];
    h_ks = reinterpret_cast<const float *>(b + 32)[G];
    h_vs = reinterpret_cast<const float *>(b + 48)[G];
    h_codec = *reinterpret_cast<const uint32_t *>(b);
  };
  if (gfirst < gb) load_header(blob);
  // the raw words of a RANS group follow its header (and its states when it starts a chain); its word streams
  // follow the raw words
  auto raw_of = [&](const uint8_t *b, uint32_t chain) {
    return reinterpret_cast<const uint32_t *>(b + kHdr + (chain ? kStateBytes : 0));
  };
  constexpr int kStage16 = ((kCapWords * 2) + 1023) / 1024;  // 1 KiB copies per group
  auto stage_words = [&](const uint8_t *b, uint32_t chain, uint32_t cnt) {
    const uint32_t nbytes = ((min((cnt & 0xFFFFu) + (cnt >> 16), kCapWords) * 2u) + 15u) & ~15u;
    const uint8_t *src = reinterpret_cast<const uint8_t *>(raw_of(b, chain) + 2 * RAW) + 16u * lane;
#pragma unroll
    for (int k = 0; k < kStage16; ++k)
      if (1024u * k + 16u * lane < nbytes)
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint32_t *>(src + 1024 * k),
                                         (__attribute__((address_space(3))) void *)(buf + 256 * k), 16, 0, 0);
  };
  uint32_t pre[14];
#pragma unroll
  for (int w = 0; w < 14; ++w) pre[w] = 0;
  if (RANS && gfirst < gb && h_codec == CF_KV_CODEC_RANS_HYBRID) {
    const uint32_t *lw = raw_of(blob, h_chain);
#pragma unroll
    for (int w = 0; w < 7; ++w) {
      pre[w] = lw[w * 64 + lane];
      pre[7 + w] = lw[RAW + w * 64 + lane];
    }
    stage_words(blob, h_chain, h_cnt);
  }
  uint32_t st[2] = {0, 0};     // lane states carried along a chain
  uint32_t prev = 0xFFFFFFFFu;  // the group decoded before (a chain continues only from its own first group)
  bool broken = false;          // a group continued a chain whose first group this wave did not decode
  for (uint32_t gi = gfirst; gi < gb;) {
    const uint32_t cnt = h_cnt, chain = h_chain, tcG = h_tc, gcodec = h_codec;  // gcodec, chain wave-uniform
    const float ks = h_ks, vs = h_vs;
    const uint8_t *cur = blob;
    const bool tok_ok = static_cast<uint32_t>(t) < tcG && 64 * gi + 16 * G + t < visible;
    if constexpr (RANS) {  // this group's copies (started during the previous group) have landed
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    if (RANS && gcodec == CF_KV_CODEC_RANS_HYBRID) {
      if (chain) {
        st[0] = h_st[0];
        st[1] = h_st[1];
      } else {
        broken |= prev + 1 != gi;
      }
    }
    const uint32_t gn = g_next;
    if (gn < gb) {  // next group's header and states (its offset was loaded one group earlier)
      blob = d.pool + static_cast<size_t>(off_next) * 16;
      load_header(blob);
      g_next = stream_next(gn);
      off_next = g_next < gb ? grow[g_next] : 0u;
    }
    const bool next_rans = RANS && gn < gb && h_codec == CF_KV_CODEC_RANS_HYBRID;
    const uint32_t *nlw = next_rans ? raw_of(blob, h_chain) : nullptr;
    auto stage_next = [&]() {  // next group's word streams, straight into LDS (no VGPRs)
      if (next_rans) stage_words(blob, h_chain, h_cnt);
    };
    if (RANS && gcodec == CF_KV_CODEC_RANS_HYBRID) {
      group_body<D, CF_KV_CODEC_RANS_HYBRID, KL>(stage_next, pre, nlw, st, raw_of(cur, chain),
                                                 reinterpret_cast<const uint16_t *>(buf), cnt, s_tab, qhi, qlo, qsum,
                                                 s_p[wave], vl, lane, tok_ok, ks, vs, e_run, m_run, l_run, acc_v);
    } else {  // raw int8 group (the INT8 codec, or the raw fallback of a group holding -128)
      // an INT8-codec launch streams its groups; raw groups inside a RANS launch (e.g. a shared prefix) are cached
      group_body<D, CF_KV_CODEC_INT8, KL, const uint16_t *, decltype(stage_next), false, false, !RANS>(
          stage_next, pre, nlw, st, reinterpret_cast<const uint32_t *>(cur + kHdr), static_cast<const uint16_t *>(nullptr),
          0, s_tab, qhi, qlo, qsum, s_p[wave], vl, lane, tok_ok, ks, vs, e_run, m_run, l_run, acc_v);
    }
    prev = gi;
    gi = gn;
  }

  // ---- reduce the wavefront: sum the hi and lo parts (lanes t and t + 16; lanes 32-63 hold the repeated rows
  // 8-15) in absolute units, l over all lanes
#pragma unroll
  for (int i = 0; i < D / 16; ++i)
#pragma unroll
    for (int h = 0; h < kGqa; ++h) {
      float v = G < 2 ? ldexpf(acc_v[i][h], e_run) : 0.0f;
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      acc_v[i][h] = v;
    }
#pragma unroll
  for (int h = 0; h < kGqa; ++h)
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) l_run[h] += __shfl_xor(l_run[h], o);
  // wave partial -> the wave's LDS buffer: [h][D] acc, then m, l (m NaN for a broken chain: the output shows it)
  float *red = reinterpret_cast<float *>(buf);
  if (lane < 16) {
#pragma unroll
    for (int i = 0; i < D / 16; ++i)
#pragma unroll
      for (int h = 0; h < kGqa; ++h) red[h * (D + 2) + t + 16 * i] = acc_v[i][h];
  }
  if (lane < kGqa) {
    red[lane * (D + 2) + D] = broken ? __builtin_nanf("") : m_run[lane];
    red[lane * (D + 2) + D + 1] = l_run[lane];
  }
  __syncthreads();

  // ---- merge the wavefronts; write the split partial (or the final output when splits == 1)
  for (int i = threadIdx.x; i < kGqa * D; i += kThreads) {
    const int h = i / D, dd = i % D;
    float m = -INFINITY;
    bool nan = false;
    for (int w = 0; w < W; ++w) {
      const float mw = reinterpret_cast<const float *>(s_buf[w])[h * (D + 2) + D];
      nan |= mw != mw;
      m = fmaxf(m, mw);
    }
    float l = 0.0f, o = 0.0f;
    if (m != -INFINITY)
      for (int w = 0; w < W; ++w) {
        const float *rw = reinterpret_cast<const float *>(s_buf[w]);
        const float mw = rw[h * (D + 2) + D];
        if (mw == -INFINITY || mw != mw) continue;
        const float sc = __expf(mw - m);
        l += rw[h * (D + 2) + D + 1] * sc;
        o += rw[h * (D + 2) + dd] * sc;
      }
    if (nan) m = __builtin_nanf("");
    if (ss.slots == 1) {
      if (static_cast<uint32_t>(h) < gqa)
        d.output[(static_cast<size_t>(seq) * d.query_head_count + head * gqa + h) * D + dd] =
            nan ? m : l > 0.0f ? o / l : 0.0f;
    } else {
      float *pp = partial + ((static_cast<size_t>(seq) * d.kv_head_count + head) * ss.slots + ss.slot0 + split) *
                                (kGqa * (D + 2));
      pp[h * (D + 2) + dd] = o;
      if (dd == 0) {
        pp[h * (D + 2) + D] = m;
        pp[h * (D + 2) + D + 1] = l;
      }
    }
  }
}

// ---- shared-prefix pass of the cascade entry point (head_dim 128, INT8 prefix groups)
// Every sequence's first `shared` groups are the same blobs (sequence 0's table gives them). One wave takes 16 query
// rows = 4 sequences x 4 query heads of one KV head and streams the prefix groups of its split once for all of
// them, on v_mfma_f32_16x16x32_f16:
//   scores   S^T = K Q^T per 16-token page: A = K[token][8 dims] (two raw u32 quads, converted exactly to f16 as
//            (1024 + sym) - 1152), B = Q^T (hi and lo f16 parts held in registers), scaled by the page's K scale;
//            the lane's accumulator registers hold S^T[tokens 4kg + r][row lane & 15];
//   softmax  online per row (its values live in the 4 lanes sharing lane & 15);
//   P V      those same registers ARE the A operand of the P V product when the k index of a 32-token step is
//            ordered {4kg + r of page 2s, 4kg + r of page 2s + 1}: no transpose. B = V[those tokens][dim] is two raw
//            u32 V quads of the INT8 layout as they are; P is pre-multiplied by each page's V scale and split into
//            f16 hi + lo parts, one MFMA each (one f16 per weight loses near-cancelling outputs).
// Operands: each group is converted once per workgroup into double-buffered LDS (see the kernel body).
// A non-INT8 group in the prefix makes the prefix partials NaN, so every output is NaN (the prefix must be raw).

__device__ __forceinline__ half8_t sym8_to_f16(uint32_t w0, uint32_t w1) {
  const half2_t off = {static_cast<_Float16>(-1152.0f), static_cast<_Float16>(-1152.0f)};
  uint32_t u[4] = {__builtin_amdgcn_perm(0x64646464u, w0, 0x04010400u), __builtin_amdgcn_perm(0x64646464u, w0, 0x04030402u),
                   __builtin_amdgcn_perm(0x64646464u, w1, 0x04010400u), __builtin_amdgcn_perm(0x64646464u, w1, 0x04030402u)};
  half8_t r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    half2_t h;
    __builtin_memcpy(&h, &u[i], 4);
    h = h + off;  // exact: (1024 + sym) - 1152 = sym - 128
    r[2 * i] = h[0];
    r[2 * i + 1] = h[1];
  }
  return r;
}

constexpr int kPfxThreads = 256;  // 4 waves x 16 rows = 16 sequences per workgroup

__global__ __launch_bounds__(kPfxThreads) void kv_prefix_kernel(cf_kv_batched_desc d, uint32_t shared,
                                                                 uint32_t psplits, float *__restrict__ partial,
                                                                 SplitSlots ss) {
  constexpr int D = 128, NQ = D / 4;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 15, kg = lane >> 4;
  const uint32_t head = blockIdx.y, psplit = blockIdx.z;
  const uint32_t gqa = d.query_head_count / d.kv_head_count;
  const uint32_t rseq = blockIdx.x * 16 + wave * 4 + j / 4, rh = j % 4;  // the lane's row j
  const bool row_ok = rseq < d.seq_count && rh < gqa;

  // Q^T operand: B[dims 32ks + 8kg .. +7][row j], split into f16 hi + lo parts (fp32-grade scores)
  half8_t qh[4], ql[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float q = row_ok ? d.queries[(static_cast<size_t>(rseq) * d.query_head_count + head * gqa + rh) * D +
                                         32 * ks + 8 * kg + e]
                             : 0.0f;
      _Float16 h, l;
      cfd::split_mul_f16(q, d.softmax_scale, h, l);
      qh[ks][e] = h;
      ql[ks][e] = l;
    }
  const uint32_t vis = row_ok ? min(d.seq_tokens[rseq], d.query_pos[rseq] + 1) : 0u;
  // wave-wide: the fewest visible tokens over the valid rows (invalid rows are never written)
  uint32_t vmin = row_ok ? vis : 0xFFFFFFFFu;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) vmin = min(vmin, static_cast<uint32_t>(__shfl_xor(static_cast<int>(vmin), o)));

  const uint32_t per = (shared + psplits - 1) / psplits;
  const uint32_t ga = min(shared, psplit * per), gb = min(shared, ga + per);
  const uint32_t *grow = d.group_offsets + static_cast<size_t>(head) * d.max_groups;  // sequence 0's table

  float m = -INFINITY, l = 0.0f;  // row j's running max / sum (same in the 4 lanes of the row)
  bool coded = false;              // a prefix group that is not INT8 was met
  int e_run = -(1 << 20);          // acc is kept in units of 2^e_run (e_run: V-scale exponent of the current group)
  float4_t acc[D / 16];            // O[rows 4kg + r][dims 16 dt + j]
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt) acc[dt] = float4_t{0, 0, 0, 0};

  // Each group is converted to f16 MFMA operands once per workgroup: wave w converts operand slots 4w .. 4w + 3 of
  // K (slot = 4 * page + k-step) and of V (slot = 8 * page pair + dim tile) for every lane, into one of two LDS
  // buffers; the next group's raw words are loaded while the current group is computed from the other buffer.
  __shared__ half8_t s_op[2][2][16][64];  // [buffer][K, V][slot][lane], 64 KiB
  uint32_t w[16];
  auto codec_at = [&](uint32_t g) { return *reinterpret_cast<const uint32_t *>(d.pool + static_cast<size_t>(grow[g]) * 16); };
  // raw words of group g; a group that is not INT8 (smaller blob: reading an INT8-sized span could run past the
  // pool) is not read, its outputs become NaN anyway
  auto fetch = [&](uint32_t g, bool raw_group) {
    const uint32_t *raw = reinterpret_cast<const uint32_t *>(d.pool + static_cast<size_t>(grow[g]) * 16 + kHdr);
    if (!raw_group) {
#pragma unroll
      for (int i = 0; i < 16; ++i) w[i] = 0;
      return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ks_slot = 4 * wave + i, G = ks_slot / 4, ks = ks_slot % 4;
      w[2 * i] = raw[(8 * ks + 2 * kg) * 64 + 16 * G + j];
      w[2 * i + 1] = raw[(8 * ks + 2 * kg + 1) * 64 + 16 * G + j];
      const int v_slot = 4 * wave + i, s2 = v_slot / 8, dt = v_slot % 8;
      w[8 + 2 * i] = raw[NQ * 64 + (kg * (D / 16) + dt) * 64 + 16 * (2 * s2) + j];
      w[9 + 2 * i] = raw[NQ * 64 + (kg * (D / 16) + dt) * 64 + 16 * (2 * s2 + 1) + j];
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s_op[buf][0][4 * wave + i][lane] = sym8_to_f16(w[2 * i], w[2 * i + 1]);
      s_op[buf][1][4 * wave + i][lane] = sym8_to_f16(w[8 + 2 * i], w[9 + 2 * i]);
    }
  };
  // the codec of group g + 1 is loaded one group ahead of its fetch, so the fetch does not wait for it
  uint32_t codec_next = ga + 1 < gb ? codec_at(ga + 1) : 0u;
  if (ga < gb) {
    fetch(ga, codec_at(ga) == CF_KV_CODEC_INT8);
    store(0);
  }
  __syncthreads();
  for (uint32_t g = ga; g < gb; ++g) {
    const int buf = (g - ga) & 1;
    const uint32_t codec1 = codec_next;
    if (g + 2 < gb) codec_next = codec_at(g + 2);
    if (g + 1 < gb) fetch(g + 1, codec1 == CF_KV_CODEC_INT8);
    const uint8_t *blob = d.pool + static_cast<size_t>(grow[g]) * 16;
    const uint32_t codec = *reinterpret_cast<const uint32_t *>(blob);
    const uint32_t tc01 = *reinterpret_cast<const uint32_t *>(blob + 12), tc23 = *reinterpret_cast<const uint32_t *>(blob + 16);
    const float *kscale = reinterpret_cast<const float *>(blob + 32), *vscale = reinterpret_cast<const float *>(blob + 48);
    const bool full = tc01 == 0x00100010u && tc23 == 0x00100010u;
    coded |= codec != CF_KV_CODEC_INT8;
    const bool fast = full && vmin >= 64u * (g + 1);  // every row sees every token of the group
    float4_t st[4];
#pragma unroll
    for (int G = 0; G < 4; ++G) {
      float4_t acc_s = {0, 0, 0, 0};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const half8_t kf = s_op[buf][0][4 * G + ks][lane];
        acc_s = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qh[ks], acc_s, 0, 0, 0);
        acc_s = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, ql[ks], acc_s, 0, 0, 0);
      }
      const float ksc = kscale[G];
#pragma unroll
      for (int r = 0; r < 4; ++r) st[G][r] = acc_s[r] * ksc;
      if (!fast) {
        const uint32_t tcg = (G < 2 ? tc01 : tc23) >> (16 * (G & 1)) & 0xFFFFu;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t t = 4 * kg + r;
          if (t >= tcg || 64u * g + 16u * G + t >= vis) st[G][r] = -INFINITY;
        }
      }
    }
    // online softmax of row j over the group's 64 tokens
    float mx = -INFINITY;
#pragma unroll
    for (int G = 0; G < 4; ++G)
#pragma unroll
      for (int r = 0; r < 4; ++r) mx = fmaxf(mx, st[G][r]);
    mx = cfd::rows4_max(mx);
    const float mn = fmaxf(m, mx);
    const float alpha = m == -INFINITY ? 0.0f : __expf(m - mn);
    m = mn;
    float psum = 0.0f;
#pragma unroll
    for (int G = 0; G < 4; ++G)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = st[G][r] == -INFINITY ? 0.0f : __expf(st[G][r] - mn);
        st[G][r] = p;
        psum += p;
      }
    psum = cfd::rows4_sum(psum);
    l = l * alpha + psum;
    // P V units: O is kept in units of 2^e with e = (exponent of the group's largest present-page V scale) - 15,
    // so the f16 operand p * v_scale * 2^-e stays below 2^15 whatever the V magnitude and weights down to 2^-29
    // of the running maximum stay normal; moving to the group's units is an exact power-of-two factor folded into
    // the softmax rescale (a drop of more than 2^60 is clamped)
    float vmax = 0.0f;
#pragma unroll
    for (int G = 0; G < 4; ++G)
      if (((G < 2 ? tc01 : tc23) >> (16 * (G & 1)) & 0xFFFFu) != 0u) vmax = fmaxf(vmax, vscale[G]);
    const int ev = max(__builtin_amdgcn_frexp_expf(vmax) - 15, e_run - 60);
    const int de = e_run - ev;
    e_run = ev;
    // rescale O: its rows are 4kg + r, whose alpha lives in lane 4kg + r
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float ar = ldexpf(__shfl(alpha, 4 * kg + r), de);
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt) acc[dt][r] *= ar;
    }
    // P V over page pairs (2s, 2s + 1); the weights p * v_scale as f16 hi + lo parts
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      half8_t pa, pl;
      const float v0 = ldexpf(vscale[2 * s2], -ev), v1 = ldexpf(vscale[2 * s2 + 1], -ev);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        _Float16 h, lo;
        cfd::split_mul_f16(st[2 * s2][r], v0, h, lo);
        pa[r] = h;
        pl[r] = lo;
        cfd::split_mul_f16(st[2 * s2 + 1][r], v1, h, lo);
        pa[4 + r] = h;
        pl[4 + r] = lo;
      }
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt) {
        const half8_t vb = s_op[buf][1][8 * s2 + dt][lane];
        acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, vb, acc[dt], 0, 0, 0);
        acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl, vb, acc[dt], 0, 0, 0);
      }
    }
    if (g + 1 < gb) store(buf ^ 1);  // the other buffer: every wave finished with it before the last barrier
    __syncthreads();
  }

  // partial state of rows 4kg + r (m and l from lane 4kg + r) into slot psplit
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int row = 4 * kg + r;
    // a coded prefix group makes the partial NaN, which the merge carries into the output
    const float mr = coded ? __builtin_nanf("") : __shfl(m, row), lr = coded ? __builtin_nanf("") : __shfl(l, row);
    const uint32_t seq = blockIdx.x * 16 + wave * 4 + row / 4, h = row % 4;
    if (seq >= d.seq_count || h >= gqa) continue;
    float *pp = partial + ((static_cast<size_t>(seq) * d.kv_head_count + head) * ss.slots + ss.slot0 + psplit) *
                              (kGqa * (D + 2)) + h * (D + 2);
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) pp[16 * dt + j] = ldexpf(acc[dt][r], e_run);
    if (j == 0) {
      pp[D] = mr;
      pp[D + 1] = lr;
    }
  }
}

// merge split partials of one (sequence, kv head): grid (kv_head, seq), block = kGqa * D threads
template <int D>
__global__ __launch_bounds__(kGqa * D) void kv_merge_kernel(cf_kv_batched_desc d, uint32_t splits,
                                                             const float *__restrict__ partial) {
  const uint32_t head = blockIdx.x, seq = blockIdx.y;
  const int h = threadIdx.x / D, dd = threadIdx.x % D;
  const uint32_t gqa = d.query_head_count / d.kv_head_count;
  if (static_cast<uint32_t>(h) >= gqa) return;
  const float *pp = partial + (static_cast<size_t>(seq) * d.kv_head_count + head) * splits * (kGqa * (D + 2));
  // eight splits' values loaded at a time (indices clamped to the last split), combined in ascending split order
  constexpr uint32_t kB = 8;
  float m = -INFINITY;
  bool nan = false;  // a NaN partial (a coded prefix group, see kv_prefix_kernel) makes the row NaN
  for (uint32_t s0 = 0; s0 < splits; s0 += kB) {
    float ms[kB];
#pragma unroll
    for (uint32_t u = 0; u < kB; ++u) ms[u] = pp[min(s0 + u, splits - 1u) * (kGqa * (D + 2)) + h * (D + 2) + D];
#pragma unroll
    for (uint32_t u = 0; u < kB; ++u)
      if (s0 + u < splits) {
        nan |= ms[u] != ms[u];
        m = fmaxf(m, ms[u]);  // fmaxf drops a NaN, hence the flag
      }
  }
  float l = 0.0f, o = 0.0f;
  if (m != -INFINITY)
    for (uint32_t s0 = 0; s0 < splits; s0 += kB) {
      float mq[kB], lq[kB], oq[kB];
#pragma unroll
      for (uint32_t u = 0; u < kB; ++u) {
        const float *q = pp + min(s0 + u, splits - 1u) * (kGqa * (D + 2)) + h * (D + 2);
        mq[u] = q[D];
        lq[u] = q[D + 1];
        oq[u] = q[dd];
      }
#pragma unroll
      for (uint32_t u = 0; u < kB; ++u) {
        if (s0 + u >= splits || mq[u] == -INFINITY) continue;
        const float sc = __expf(mq[u] - m);
        l += lq[u] * sc;
        o += oq[u] * sc;
      }
    }
  // 0 when no token is visible
  d.output[(static_cast<size_t>(seq) * d.query_head_count + head * gqa + h) * D + dd] =
      nan ? __builtin_nanf("") : l == 0.0f ? 0.0f : o / l;
}

// ---- decode-shape route of the reference seam (kv_seam_route.hpp)

using cfkv::kRouteChunk;
using cfkv::kRouteInfoWords;
using cfkv::kRouteMaxHeads;
using cfkv::seam_route_chunks;
static_assert(CF_KV_CUDA_MAX_PAGES_PER_LAUNCH / kRouteChunk <= 64, "a wavefront holds a head's chunk records");

// One workgroup per chunk of 256 descriptors (thread t: descriptor 256 chunk + t). Each wavefront walks the KV
// heads present among its 64 descriptors (one ballot per head) and notes per (head, wavefront) the match count,
// whether a match is refused or names other tables than the wavefront's first match, and those tables; thread h
// then combines the four wavefronts of head h into the (head, chunk) record and the wavefronts' offsets, and every
// thread writes its page's entry to lists[kv_head][256 chunk + offset] (descriptor order within the chunk): the
// blob pointer's two halves, token_begin and token_count, so that the group kernel reads one 16-byte entry per page
// instead of an index and then the descriptor.
// Descriptors whose kv_head is not below the call's KV head count belong to no head (the seam kernel skips them).
__global__ __launch_bounds__(kRouteChunk) void seam_list_kernel(cf_kv_paged_attention_desc d,
                                                                uint4 *__restrict__ lists,
                                                                uint32_t *__restrict__ info) {
  constexpr unsigned W = kRouteChunk / 64;
  static_assert(kRouteMaxHeads * W == kRouteChunk, "one counter per thread to clear");
  __shared__ uint32_t s_cnt[kRouteMaxHeads][W];  // matches per (head, wavefront), then their offsets
  __shared__ uint32_t s_bad[kRouteMaxHeads][W];
  __shared__ uint64_t s_kl[kRouteMaxHeads][W], s_vl[kRouteMaxHeads][W];
  const uint32_t chunk = blockIdx.x, t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const uint32_t H = d.kv_head_count, p = chunk * kRouteChunk + t;
  s_cnt[t / W][t % W] = 0;
  uint32_t hp = 0xFFFFFFFFu, tbeg = 0, tcnt = 0;
  uint64_t kl = 0, vl = 0, kw = 0;
  bool badp = false;
  if (p < d.page_count) {
    const cf_kv_device_page &pg = d.pages[p];
    hp = pg.kv_head;
    tbeg = pg.token_begin;
    tcnt = pg.token_count;
    kw = reinterpret_cast<uintptr_t>(pg.k_words);
    kl = reinterpret_cast<uintptr_t>(pg.k_lut);
    vl = reinterpret_cast<uintptr_t>(pg.v_lut);
    const bool rans = pg.fixed_code_length == 0 && pg.k_max_code_length == 0;
    badp = !rans || pg.head_dim != d.head_dim || pg.token_count == 0 || pg.token_count > 64 || !pg.k_words || !kl ||
           !vl || ((kl | vl) & 15u) != 0;  // tables staged by 16-byte loads
  }
  __syncthreads();
  const bool mine_ok = hp < H;
  uint64_t mine = 0, left = __builtin_amdgcn_ballot_w64(mine_ok);
  while (left != 0) {  // wave-uniform: one head per pass
    const int f = __builtin_ctzll(left);
    const uint32_t h = __shfl(hp, f);
    const uint64_t k0 = __shfl(kl, f), v0 = __shfl(vl, f);
    const uint64_t bal = __builtin_amdgcn_ballot_w64(hp == h);
    if (hp == h) mine = bal;
    const bool wb = __builtin_amdgcn_ballot_w64(hp == h && (badp || kl != k0 || vl != v0)) != 0;
    if (lane == 0) {
      s_cnt[h][wave] = static_cast<uint32_t>(__builtin_popcountll(bal));
      s_bad[h][wave] = wb ? 1u : 0u;
      s_kl[h][wave] = k0;
      s_vl[h][wave] = v0;
    }
    left &= ~bal;
  }
  __syncthreads();
  if (t < H) {  // head t's record for this chunk
    uint32_t run = 0, bad = 0;
    bool seen = false;
    uint64_t k0 = 0, v0 = 0;
#pragma unroll
    for (unsigned w = 0; w < W; ++w) {
      const uint32_t c = s_cnt[t][w];
      if (c) {
        bad |= s_bad[t][w];
        if (!seen) {
          k0 = s_kl[t][w];
          v0 = s_vl[t][w];
          seen = true;
        } else if (s_kl[t][w] != k0 || s_vl[t][w] != v0) {
          bad = 1u;
        }
      }
      s_cnt[t][w] = run;
      run += c;
    }
    uint4 *e = reinterpret_cast<uint4 *>(info + (static_cast<size_t>(t) * gridDim.x + chunk) * kRouteInfoWords);
    e[0] = uint4{run, bad, static_cast<uint32_t>(k0), static_cast<uint32_t>(k0 >> 32)};
    e[1] = uint4{static_cast<uint32_t>(v0), static_cast<uint32_t>(v0 >> 32), 0u, 0u};
  }
  __syncthreads();
  if (mine_ok)
    lists[static_cast<size_t>(hp) * d.page_count + chunk * kRouteChunk + s_cnt[hp][wave] +
          __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mine >> 32),
                                    __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mine), 0u))] =
        uint4{static_cast<uint32_t>(kw), static_cast<uint32_t>(kw >> 32), tbeg, tcnt};
}

// One (context split, KV head) per 4-wavefront workgroup. Each wavefront reads the head's chunk records (lane c:
// chunk c) and decides whether the route takes the head: no refused page and one pair of table pointers over all
// chunks with pages; workgroup (0, head) publishes that in taken[head]. For a head it takes, wavefront w decodes
// the head's pages of ordinals split + splits * (w + 4 k) (ordinal o: chunk = number of chunks whose inclusive
// page prefix is at most o, then its list entry o - exclusive prefix), each page one self-contained group
// (RANS_HYBRID chain start or INT8 fallback) run through group_body with the page's token positions, then the
// workgroup writes slot `split` of the seam's partials ([slot][kv head][vector][head_dim + 2] = acc, m, l; m NaN
// when a page was refused). Heads the route did not take are left alone (the seam kernel serves them and the merge
// reads its slots); splits without pages get empty slots (m = -inf, l = 0).
template <int D>
__global__ CF_KV_OCC __launch_bounds__(64 * kWavesNarrow) void seam_group_kernel(cf_kv_paged_attention_desc d, uint32_t splits,
                                                                       const uint32_t *__restrict__ info,
                                                                       const uint4 *__restrict__ lists,
                                                                       uint32_t *__restrict__ taken,
                                                                       float *__restrict__ partial) {
  constexpr int W = kWavesNarrow, NQ = D / 4, RAW = raw_words<D>(), BUF = buf_u32<D>(), kThreads = 64 * W;
  __shared__ __attribute__((aligned(16))) uint2 s_tab[2][kSlots];
  __shared__ __attribute__((aligned(16))) _Float16 s_p[W][2][4][kGqa][16];
  __shared__ uint32_t s_buf[W][BUF];  // per wave: staged words; query staging and partials alias it
  // (no other shared variable: with 53,760 bytes or less three workgroups fit a CU)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int G = lane >> 4, t = lane & 15;
  const uint32_t split = blockIdx.x, head = blockIdx.y, gqa = d.gqa_group_size;
  // the head's chunk records, lane c holding chunk c
  const uint32_t chunks = seam_route_chunks(d.page_count);
  uint32_t ccount = 0, cbad = 0;
  uint64_t ckl = 0, cvl = 0;
  if (static_cast<uint32_t>(lane) < chunks) {
    const uint4 *e = reinterpret_cast<const uint4 *>(
        info + (static_cast<size_t>(head) * chunks + static_cast<uint32_t>(lane)) * kRouteInfoWords);
    const uint4 a = e[0], b = e[1];
    ccount = a.x;
    cbad = a.y;
    ckl = a.z | (static_cast<uint64_t>(a.w) << 32);
    cvl = b.x | (static_cast<uint64_t>(b.y) << 32);
  }
  const uint64_t with = __builtin_amdgcn_ballot_w64(ccount != 0);
  bool ok = __builtin_amdgcn_ballot_w64(ccount != 0 && cbad != 0) == 0;
  uint64_t tkl = 0, tvl = 0;
  if (with != 0) {
    const int f = __builtin_ctzll(with);
    tkl = __shfl(ckl, f);
    tvl = __shfl(cvl, f);
    ok &= __builtin_amdgcn_ballot_w64(ccount != 0 && (ckl != tkl || cvl != tvl)) == 0;
  }
  uint32_t cinc = ccount;  // inclusive prefix of the chunks' page counts
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(cinc, o);
    if (lane >= o) cinc += y;
  }
  const uint32_t n = __shfl(cinc, 63);
  if (split == 0 && threadIdx.x == 0) taken[head] = ok ? 1u : 0u;
  float *pp = partial + (static_cast<size_t>(split) * d.kv_head_count + head) * gqa * (D + 2);
  if (!ok) return;  // the seam kernel serves this head (the merge reads its slots instead)
  if (split >= n) {
    for (uint32_t i = threadIdx.x; i < gqa * (D + 2); i += kThreads) pp[i] = i % (D + 2) == D ? -INFINITY : 0.0f;
    return;
  }
  const uint4 *list = lists + static_cast<size_t>(head) * d.page_count;
  const uint32_t cexc = cinc - ccount;
  {  // the head's tables (every listed page has these), as the decoder reads them: two entries per 16-byte load,
     // all of a thread's loads issued before its first LDS write
    constexpr int kIt = static_cast<int>(kSlots / 2 / kThreads);
    static_assert(kIt * kThreads * 2 == static_cast<int>(kSlots), "whole 16-byte pairs per thread");
    const uint4 *tk = reinterpret_cast<const uint4 *>(tkl), *tv = reinterpret_cast<const uint4 *>(tvl);
    uint4 a[kIt], b[kIt];
#pragma unroll
    for (int k = 0; k < kIt; ++k) {
      a[k] = tk[threadIdx.x + k * kThreads];
      b[k] = tv[threadIdx.x + k * kThreads];
    }
#pragma unroll
    for (int k = 0; k < kIt; ++k) {
      const uint32_t j = 2 * (threadIdx.x + k * kThreads);
      *reinterpret_cast<uint4 *>(&s_tab[0][j]) = uint4{(a[k].x & 2047u) | (((a[k].x >> 11) & 2047u) << 16), a[k].y,
                                                       (a[k].z & 2047u) | (((a[k].z >> 11) & 2047u) << 16), a[k].w};
      *reinterpret_cast<uint4 *>(&s_tab[1][j]) = uint4{(b[k].x & 2047u) | (((b[k].x >> 11) & 2047u) << 16), b[k].y,
                                                       (b[k].z & 2047u) | (((b[k].z >> 11) & 2047u) << 16), b[k].w};
    }
  }
  static_assert(2 * kGqa * D * 2 <= W * BUF * 4, "query staging must fit the word buffers");
  _Float16(*s_q)[kGqa][D] = reinterpret_cast<_Float16(*)[kGqa][D]>(&s_buf[0][0]);
  for (int i = threadIdx.x; i < kGqa * D; i += kThreads) {  // the call's one query row
    const int h = i / D, dd = i % D;
    const float q = static_cast<uint32_t>(h) < gqa ? d.queries[(static_cast<size_t>(head) * gqa + h) * D + dd] : 0.0f;
    cfd::split_mul_f16(q, d.softmax_scale, s_q[0][h][dd], s_q[1][h][dd]);
  }
  __syncthreads();
  constexpr int NC = NQ / 16 > 0 ? NQ / 16 : 1;
  half4_t qhi[NC], qlo[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int qd = 16 * c + (lane >> 2);
    qhi[c] = (4 * qd < D) ? *reinterpret_cast<const half4_t *>(&s_q[0][lane & 3][4 * qd]) : half4_t{0, 0, 0, 0};
    qlo[c] = (4 * qd < D) ? *reinterpret_cast<const half4_t *>(&s_q[1][lane & 3][4 * qd]) : half4_t{0, 0, 0, 0};
  }
  float qsum[kGqa];
  {
    float part = 0.0f;
    const int h = lane >> 4;
#pragma unroll
    for (int k = 0; k < D / 16; ++k) {
      const int dd = (lane & 15) * (D / 16) + k;
      part += static_cast<float>(s_q[0][h][dd]) + static_cast<float>(s_q[1][h][dd]);
    }
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) part += __shfl_xor(part, o);
#pragma unroll
    for (int hh = 0; hh < kGqa; ++hh) qsum[hh] = __shfl(part, 16 * hh);
  }
  __syncthreads();  // s_q (aliasing the word buffers) is dead from here on

  // the seam's visible range of the query row: [window begin, query token]
  const uint32_t qtok = d.query_token_begin;
  const uint32_t wlo = (d.causal_window == 0 || qtok + 1 <= d.causal_window) ? 0u : qtok + 1 - d.causal_window;
  float m_run[kGqa], l_run[kGqa];
  int e_run = -(1 << 20);
  float4_t acc_v[D / 16];
#pragma unroll
  for (int h = 0; h < kGqa; ++h) {
    m_run[h] = -INFINITY;
    l_run[h] = 0.0f;
  }
#pragma unroll
  for (int i = 0; i < D / 16; ++i) acc_v[i] = float4_t{0, 0, 0, 0};
  uint32_t *buf = s_buf[__builtin_amdgcn_readfirstlane(wave)];
  bool bad = false;
  uint32_t pre[14];
#pragma unroll
  for (int w = 0; w < 14; ++w) pre[w] = 0;
  // the page entry of ordinal o (wave-uniform: a scalar load)
  auto entry_of = [&](uint32_t o) {
    const uint32_t oc = static_cast<uint32_t>(__builtin_popcountll(__builtin_amdgcn_ballot_w64(cinc <= o)));
    const uint32_t li = __builtin_amdgcn_readfirstlane(oc * kRouteChunk + o - __shfl(cexc, static_cast<int>(oc)));
    return list[li];
  };
  const uint32_t ostep = splits * static_cast<uint32_t>(W);
  // the first ordinal from o on (in steps of ostep) whose page has a token in [window begin, query token], and its
  // entry; pages wholly outside that range are skipped unread
  auto next_visible = [&](uint32_t o, uint4 &e) {
    for (; o < n; o += ostep) {
      e = entry_of(o);
      if (!(e.z > qtok || e.z + e.w <= wlo)) break;
    }
    return o;
  };
  // A page's header: loaded one page ahead (while the page before it is decoded). Its lane states, first raw words
  // and word streams are loaded only once the header has passed the checks, during the previous page's softmax / V
  // phase (its raw words through group_body's next-group refill).
  struct Hdr {
    const uint8_t *blob;
    uint32_t tb, tcnt, codec, cnt, chain, bd, tc01, tc23;
    float ks, vs;
  };
  auto load_hdr = [&](const uint4 &e) {
    Hdr h;
    h.blob = reinterpret_cast<const uint8_t *>(e.x | (static_cast<uint64_t>(e.y) << 32));
    h.tb = e.z;
    h.tcnt = e.w;
    h.codec = *reinterpret_cast<const uint32_t *>(h.blob);
    h.cnt = *reinterpret_cast<const uint32_t *>(h.blob + 4);
    h.chain = *reinterpret_cast<const uint16_t *>(h.blob + 8);
    h.tc01 = *reinterpret_cast<const uint32_t *>(h.blob + 12);
    h.tc23 = *reinterpret_cast<const uint32_t *>(h.blob + 16);
    h.bd = *reinterpret_cast<const uint16_t *>(h.blob + 20);
    h.ks = reinterpret_cast<const float *>(h.blob + 32)[G];
    h.vs = reinterpret_cast<const float *>(h.blob + 48)[G];
    return h;
  };
  // a self-contained group of this head_dim whose token counts match the page: full 16-token pages, then at most one
  // partial page, then empty ones (the seam's rule, kv_legacy.hip rans_stream_to_lds)
  auto page_ok = [&](const Hdr &h) {
    bool valid = h.bd == static_cast<uint32_t>(D) &&
                 (h.codec == CF_KV_CODEC_INT8 || (h.codec == CF_KV_CODEC_RANS_HYBRID && h.chain == 1));
    uint32_t total = 0;
    bool open = true;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint32_t c = ((g < 2 ? h.tc01 : h.tc23) >> (16 * (g & 1))) & 0xFFFFu;
      valid &= c <= 16u && (c == 0 || open);
      open &= c == 16u;
      total += c;
    }
    const uint32_t nk = h.cnt & 0xFFFFu, nv = h.cnt >> 16;
    return valid && total == h.tcnt && (h.codec != CF_KV_CODEC_RANS_HYBRID || nk + nv <= kCapWords);
  };
  auto raw_of = [&](const Hdr &h) { return reinterpret_cast<const uint32_t *>(h.blob + kHdr + kStateBytes); };
  uint32_t st_next[2] = {0, 0};
  // lane states and word streams of a checked RANS page into registers / the wave's buffer (whole 16-byte chunks:
  // blobs are padded to 16 bytes)
  auto stage_page = [&](const Hdr &h) {
    const uint32_t *hs = reinterpret_cast<const uint32_t *>(h.blob + kHdr);
    st_next[0] = hs[lane];
    st_next[1] = hs[64 + lane];
    constexpr int kStage16 = ((kCapWords * 2) + 1023) / 1024;
    const uint32_t nbytes = (((h.cnt & 0xFFFFu) + (h.cnt >> 16)) * 2u + 15u) & ~15u;
    const uint8_t *src = reinterpret_cast<const uint8_t *>(raw_of(h) + 2 * RAW) + 16u * lane;
#pragma unroll
    for (int k = 0; k < kStage16; ++k)
      if (1024u * k + 16u * lane < nbytes)
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint32_t *>(src + 1024 * k),
                                         (__attribute__((address_space(3))) void *)(buf + 256 * k), 16, 0, 0);
  };
  uint4 ec = {0, 0, 0, 0};
  uint32_t o = next_visible(split + splits * static_cast<uint32_t>(wave), ec);
  Hdr cur = o < n ? load_hdr(ec) : Hdr{};
  bool cur_ok = o < n && page_ok(cur);
  if (cur_ok && cur.codec == CF_KV_CODEC_RANS_HYBRID) {  // the wave's first page: nothing to overlap it with
    const uint32_t *raw = raw_of(cur);
#pragma unroll
    for (int w = 0; w < 7; ++w) {
      pre[w] = raw[w * 64 + lane];
      pre[7 + w] = raw[RAW + w * 64 + lane];
    }
    stage_page(cur);
  }
  uint4 en = {0, 0, 0, 0};
  uint32_t on = o < n ? next_visible(o + ostep, en) : n;
  while (o < n) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this page's states and word streams have landed
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    uint32_t st[2] = {st_next[0], st_next[1]};
    const Hdr nx = on < n ? load_hdr(en) : Hdr{};
    uint4 en2 = {0, 0, 0, 0};
    const uint32_t on2 = on < n ? next_visible(on + ostep, en2) : n;
    const bool nx_ok = on < n && page_ok(nx);
    const bool next_rans = nx_ok && nx.codec == CF_KV_CODEC_RANS_HYBRID;
    const uint32_t *nlw = next_rans ? raw_of(nx) : nullptr;
    auto stage_next = [&]() {  // the word buffer is free: the next page's states and word streams
      if (next_rans) stage_page(nx);
    };
    if (!cur_ok) {
      bad = true;
      if (next_rans) {
#pragma unroll
        for (int w = 0; w < 7; ++w) {
          pre[w] = nlw[w * 64 + lane];
          pre[7 + w] = nlw[RAW + w * 64 + lane];
        }
      }
      stage_next();
    } else {
      const uint32_t tcG = ((G < 2 ? cur.tc01 : cur.tc23) >> (16 * (G & 1))) & 0xFFFFu;
      const uint32_t pos = cur.tb + 16u * static_cast<uint32_t>(G) + static_cast<uint32_t>(t);
      const bool tok_ok = static_cast<uint32_t>(t) < tcG && pos >= wlo && pos <= qtok;
      // any token of the lane's 16-token page visible (behind a window the visible tokens can be a page's suffix)
      const uint32_t pg0 = cur.tb + 16u * static_cast<uint32_t>(G);
      const bool page_vis = tcG > 0 && pg0 <= qtok && pg0 + tcG - 1 >= wlo;
      if (cur.codec == CF_KV_CODEC_RANS_HYBRID) {
        uint32_t ends[2];
        group_body<D, CF_KV_CODEC_RANS_HYBRID, 0, const uint16_t *, decltype(stage_next), true, true>(
            stage_next, pre, nlw, st, raw_of(cur), reinterpret_cast<const uint16_t *>(buf), cur.cnt, s_tab, qhi, qlo,
            qsum, s_p[wave], nullptr, lane, tok_ok, cur.ks, cur.vs, e_run, m_run, l_run, acc_v, ends, page_vis);
        // a group coded on its own ends where the encoder started (2^16 in every lane) and consumed exactly its words
        const uint32_t nk = cur.cnt & 0xFFFFu, nv = cur.cnt >> 16;
        const bool ok = st[0] == 65536u && st[1] == 65536u && ends[0] == nk && ends[1] == nk + nv;
        bad |= __builtin_amdgcn_ballot_w64(!ok) != 0;
      } else {
        group_body<D, CF_KV_CODEC_INT8, 0, const uint16_t *, decltype(stage_next), false, true>(
            stage_next, pre, nlw, st, reinterpret_cast<const uint32_t *>(cur.blob + kHdr),
            static_cast<const uint16_t *>(nullptr), 0, s_tab, qhi, qlo, qsum, s_p[wave], nullptr, lane, tok_ok,
            cur.ks, cur.vs, e_run, m_run, l_run, acc_v, nullptr, page_vis);
      }
    }
    cur = nx;
    cur_ok = nx_ok;
    o = on;
    on = on2;
    en = en2;
  }

  // ---- reduce the wavefront (as kv_batched_kernel), then merge the wavefronts into the slot
#pragma unroll
  for (int i = 0; i < D / 16; ++i)
#pragma unroll
    for (int h = 0; h < kGqa; ++h) {
      float v = G < 2 ? ldexpf(acc_v[i][h], e_run) : 0.0f;
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      acc_v[i][h] = v;
    }
#pragma unroll
  for (int h = 0; h < kGqa; ++h)
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) l_run[h] += __shfl_xor(l_run[h], o);
  float *red = reinterpret_cast<float *>(buf);  // the wave's m is NaN when it refused a page
  if (lane < 16) {
#pragma unroll
    for (int i = 0; i < D / 16; ++i)
#pragma unroll
      for (int h = 0; h < kGqa; ++h) red[h * (D + 2) + t + 16 * i] = acc_v[i][h];
  }
  if (lane < kGqa) {
    red[lane * (D + 2) + D] = bad ? __builtin_nanf("") : m_run[lane];
    red[lane * (D + 2) + D + 1] = l_run[lane];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < kGqa * D; i += kThreads) {
    const int h = i / D, dd = i % D;
    if (static_cast<uint32_t>(h) >= gqa) continue;
    float m = -INFINITY;
    bool any_bad = false;
    for (int w = 0; w < W; ++w) {
      const float mw = reinterpret_cast<const float *>(s_buf[w])[h * (D + 2) + D];
      any_bad |= mw != mw;
      m = fmaxf(m, mw);  // fmaxf drops a NaN, hence the flag
    }
    float l = 0.0f, o = 0.0f;
    if (m != -INFINITY)
      for (int w = 0; w < W; ++w) {
        const float *rw = reinterpret_cast<const float *>(s_buf[w]);
        const float mw = rw[h * (D + 2) + D];
        if (mw == -INFINITY || mw != mw) continue;
        const float sc = __expf(mw - m);
        l += rw[h * (D + 2) + D + 1] * sc;
        o += rw[h * (D + 2) + dd] * sc;
      }
    pp[h * (D + 2) + dd] = o;
    if (dd == 0) {
      pp[h * (D + 2) + D] = any_bad ? __builtin_nanf("") : m;
      pp[h * (D + 2) + D + 1] = l;
    }
  }
}

// CUs of the current device (cached per thread and device).
uint32_t cu_count() {
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

// Launch shape of kv_batched_kernel: context splits per (sequence, KV head) and wavefronts per workgroup.
// Narrow (4 wavefronts, three workgroups per CU) is the base shape. Issue arbitration favours the oldest wavefronts,
// so the three workgroups of a CU finish far apart; when the grid is one round of workgroups (fewer units than three
// per CU) that spread is the tail of the whole launch. Launches with at most one (sequence, head) unit per CU go
// wide (12 wavefronts, one workgroup per CU, one round) when every wavefront still gets about 2 chain pairs or more:
// the priority-weighted pair blocks (wide_block) then let the wavefronts of a CU finish together (C4 at 4k tokens:
// 59-60 us wide with one split against 68 us for three narrow splits and their merge). Larger grids stay
// narrow: the dispatcher refills a CU as each workgroup ends, and three workgroups of different sequences on one CU
// share its L1 when their pools share groups (a common prompt prefix).
// Splits: enough workgroups to fill the chip in one round when the (sequence, head) units alone do not (a partial
// second round leaves most CUs idle at the tail), keeping at least one page group per wavefront. A caller's d->splits
// is kept.
struct BatchedPlan {
  uint32_t splits, waves;
};
constexpr uint32_t kWidePairsPerWave = 2;

BatchedPlan batched_plan(const cf_kv_batched_desc *d) {
  const uint32_t units = d->seq_count * d->kv_head_count;
  const uint32_t pairs = (d->max_groups + 1) / 2;
  const uint32_t cus = cu_count();
  auto wide_ok = [&](uint32_t s) { return pairs / s >= kWidePairsPerWave * kWavesWide; };
  const uint32_t resident = 3 * cus;
  if (d->splits) return {d->splits, units * d->splits <= cus && wide_ok(d->splits) ? 12u : 4u};
  if (units <= cus) {
    const uint32_t s = std::max<uint32_t>(1, std::min<uint32_t>(cus / units, 64));
    if (wide_ok(s)) return {s, 12u};
  }
  uint32_t s = units >= resident ? 1u : resident / units;
  s = std::min<uint32_t>(s, std::max<uint32_t>(1, d->max_groups / kWavesNarrow));
  return {std::max<uint32_t>(1, std::min<uint32_t>(s, 64)), 4u};
}

// Cascade plan: prefix splits (slots [0, ps)) sized so that the prefix pass has about two workgroups per CU, then the
// suffix splits (slots [ps, ps + ss)) over each sequence's own groups.
struct CascadePlan {
  uint32_t psplits, slots;
  BatchedPlan suffix;
};

CascadePlan cascade_plan(const cf_kv_batched_desc *d, uint32_t shared) {
  CascadePlan p{};
  const uint32_t tiles = ((d->seq_count + 15) / 16) * d->kv_head_count;
  const uint32_t want = std::max<uint32_t>(1, (2 * cu_count() + tiles - 1) / tiles);
  p.psplits = std::min<uint32_t>(want, shared);
  cf_kv_batched_desc rest = *d;
  rest.max_groups = std::max<uint32_t>(1, d->max_groups - shared);
  p.suffix = batched_plan(&rest);
  p.slots = p.psplits + p.suffix.splits;
  return p;
}

template <int D, int C>
void launch_batched(const cf_kv_batched_desc &d, const BatchedPlan &p, dim3 grid, float *ws, SplitSlots ss,
                    hipStream_t s) {
  if (p.waves == 12)
    kv_batched_kernel<D, C, kWavesWide><<<grid, 64 * kWavesWide, 0, s>>>(d, p.splits, ws, ss);
  else
    kv_batched_kernel<D, C, kWavesNarrow><<<grid, 64 * kWavesNarrow, 0, s>>>(d, p.splits, ws, ss);
}

}  // namespace

extern "C" cf_status cf_kv_validate_batched_desc(const cf_kv_batched_desc *d) {
  if (!d || d->struct_size != sizeof(cf_kv_batched_desc) || d->abi_version != CF_KV_EXT_ABI_VERSION)
    return CF_ERR_INVALID_ARGUMENT;
  if (!d->pool || !d->group_offsets || !d->seq_tokens || !d->query_pos || !d->queries || !d->output ||
      d->seq_count == 0 || d->kv_head_count == 0 || d->query_head_count == 0 ||
      d->query_head_count % d->kv_head_count != 0 || !std::isfinite(d->softmax_scale))
    return CF_ERR_INVALID_ARGUMENT;
  if (d->codec != CF_KV_CODEC_INT8 && d->codec != CF_KV_CODEC_RANS_HYBRID) return CF_ERR_UNSUPPORTED;
  if (d->codec == CF_KV_CODEC_RANS_HYBRID && !d->tables) return CF_ERR_INVALID_ARGUMENT;
  // blobs are copied in 16-byte chunks and tables read two entries per 16-byte load
  if ((reinterpret_cast<uintptr_t>(d->pool) & 15u) != 0 || (reinterpret_cast<uintptr_t>(d->tables) & 15u) != 0)
    return CF_ERR_INVALID_ARGUMENT;
  if (d->query_head_count / d->kv_head_count > kGqa) return CF_ERR_UNSUPPORTED;
  if (d->head_dim != 64 && d->head_dim != 128) return CF_ERR_UNSUPPORTED;
  if (d->seq_count > 65535 || d->kv_head_count > 65535) return CF_ERR_UNSUPPORTED;
  return CF_OK;
}

extern "C" uint64_t cf_kv_batched_workspace_bytes(const cf_kv_batched_desc *d) {
  if (cf_kv_validate_batched_desc(d) != CF_OK) return 0;
  const uint32_t s = batched_plan(d).splits;
  if (s <= 1) return 0;
  return static_cast<uint64_t>(d->seq_count) * d->kv_head_count * s * kGqa * (d->head_dim + 2) * sizeof(float);
}

namespace {

// The batched launch (decode kernel, then the split merge when the plan splits the context) with the split partials
// in `ws` (at least cf_kv_batched_workspace_bytes(d) bytes; unused when the plan does not split).
cf_status launch_batched_all(const cf_kv_batched_desc *d, const BatchedPlan &plan, float *ws, void *stream) {
  const uint32_t splits = plan.splits;
  const hipStream_t s = cfd::as_stream(stream);
  const dim3 grid(splits, d->kv_head_count, d->seq_count);
  const SplitSlots ss{0, 0, splits};
  if (d->head_dim == 128) {
    if (d->codec == CF_KV_CODEC_RANS_HYBRID) launch_batched<128, CF_KV_CODEC_RANS_HYBRID>(*d, plan, grid, ws, ss, s);
    else launch_batched<128, CF_KV_CODEC_INT8>(*d, plan, grid, ws, ss, s);
  } else {
    if (d->codec == CF_KV_CODEC_RANS_HYBRID) launch_batched<64, CF_KV_CODEC_RANS_HYBRID>(*d, plan, grid, ws, ss, s);
    else launch_batched<64, CF_KV_CODEC_INT8>(*d, plan, grid, ws, ss, s);
  }
  if (splits > 1) {
    const dim3 g2(d->kv_head_count, d->seq_count);
    if (d->head_dim == 128) kv_merge_kernel<128><<<g2, kGqa * 128, 0, s>>>(*d, splits, ws);
    else kv_merge_kernel<64><<<g2, kGqa * 64, 0, s>>>(*d, splits, ws);
  }
  return cfd::launch_status();
}

}  // namespace

extern "C" cf_status cf_kv_paged_attention_batched_async(const cf_kv_batched_desc *d, void *stream) {
  const cf_status v = cf_kv_validate_batched_desc(d);
  if (v != CF_OK) return v;
  const BatchedPlan plan = batched_plan(d);
  const uint64_t need = cf_kv_batched_workspace_bytes(d);
  if (need && (!d->workspace || d->workspace_bytes < need)) return CF_ERR_INVALID_ARGUMENT;
  return launch_batched_all(d, plan, static_cast<float *>(d->workspace), stream);
}

extern "C" uint64_t cf_kv_cascade_workspace_bytes(const cf_kv_batched_desc *d, uint32_t shared_groups) {
  if (cf_kv_validate_batched_desc(d) != CF_OK || d->head_dim != 128 || shared_groups == 0 ||
      shared_groups > d->max_groups)
    return 0;
  const CascadePlan p = cascade_plan(d, shared_groups);
  return static_cast<uint64_t>(d->seq_count) * d->kv_head_count * p.slots * kGqa * (d->head_dim + 2) * sizeof(float);
}

extern "C" cf_status cf_kv_paged_attention_cascade_async(const cf_kv_batched_desc *d, uint32_t shared_groups,
                                                          void *stream) {
  const cf_status v = cf_kv_validate_batched_desc(d);
  if (v != CF_OK) return v;
  if (d->head_dim != 128) return CF_ERR_UNSUPPORTED;
  if (shared_groups == 0 || shared_groups > d->max_groups) return CF_ERR_INVALID_ARGUMENT;
  const CascadePlan p = cascade_plan(d, shared_groups);
  const uint64_t need = cf_kv_cascade_workspace_bytes(d, shared_groups);
  if (!d->workspace || d->workspace_bytes < need) return CF_ERR_INVALID_ARGUMENT;
  const hipStream_t s = cfd::as_stream(stream);
  float *ws = static_cast<float *>(d->workspace);
  kv_prefix_kernel<<<dim3((d->seq_count + 15) / 16, d->kv_head_count, p.psplits), kPfxThreads, 0, s>>>(
      *d, shared_groups, p.psplits, ws, SplitSlots{0, 0, p.slots});
  const SplitSlots rest{shared_groups, p.psplits, p.slots};
  const dim3 grid(p.suffix.splits, d->kv_head_count, d->seq_count);
  if (d->codec == CF_KV_CODEC_RANS_HYBRID)
    launch_batched<128, CF_KV_CODEC_RANS_HYBRID>(*d, p.suffix, grid, ws, rest, s);
  else
    launch_batched<128, CF_KV_CODEC_INT8>(*d, p.suffix, grid, ws, rest, s);
  kv_merge_kernel<128><<<dim3(d->kv_head_count, d->seq_count), kGqa * 128, 0, s>>>(*d, p.slots, ws);
  return cfd::launch_status();
}

// ---- allocation-free variant of the batched entry point
// The split partials live in `scratch`, a file-scope device array of CF_KV_BATCHED_NOALLOC_SCRATCH_BYTES that each
// GPU holds until the process ends. In host code `scratch` only names the symbol: its device address on the current
// GPU comes from hipGetSymbolAddress, looked up once per device on the first call there and kept in
// g_scratch_addr. Every call on a GPU uses that GPU's one array, so calls that overlap on one GPU (other streams,
// other threads) race on it. Nothing in it needs clearing: every split workgroup writes its whole partial slot
// before the merge reads it.
static __device__ __align__(256) uint8_t scratch[CF_KV_BATCHED_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_addr[kMaxDevices] = {};

cf_status scratch_address(void **out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return CF_ERR_CUDA;
  if (dev < 0 || dev >= kMaxDevices) return CF_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_addr[dev]) {
    void *addr = nullptr;
    if (hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)) != hipSuccess || !addr) return CF_ERR_CUDA;
    g_scratch_addr[dev] = addr;
  }
  *out = g_scratch_addr[dev];
  return CF_OK;
}

}  // namespace

extern "C" cf_status cf_kv_paged_attention_batched_noalloc_async(const cf_kv_batched_desc *d, void *stream) {
  const cf_status v = cf_kv_validate_batched_desc(d);
  if (v != CF_OK) return v;
  const BatchedPlan plan = batched_plan(d);
  const uint64_t need = cf_kv_batched_workspace_bytes(d);
  if (need > CF_KV_BATCHED_NOALLOC_SCRATCH_BYTES) return CF_ERR_UNSUPPORTED;
  void *ws = nullptr;
  if (need) {
    const cf_status st = scratch_address(&ws);
    if (st != CF_OK) return st;
  }
  return launch_batched_all(d, plan, static_cast<float *>(ws), stream);
}

// ---- the seam's decode-shape route, host side (kv_seam_route.hpp)
namespace cfkv {

bool seam_route_applies(const cf_kv_paged_attention_desc &d) {
  return d.query_count == 1 && d.gqa_group_size >= 1 && d.gqa_group_size <= static_cast<uint32_t>(kGqa) &&
         (d.head_dim == 64 || d.head_dim == 128) && d.active_token_count == 0 && d.page_count > 0 && d.pages &&
         d.kv_head_count >= 1 && d.kv_head_count <= kRouteMaxHeads;
}

uint32_t seam_route_splits(const cf_kv_paged_attention_desc &d) {
  // about two pages per wavefront, within one round of workgroups (three per CU)
  const uint32_t per_head = (d.page_count + d.kv_head_count - 1) / d.kv_head_count;
  uint32_t s = std::max<uint32_t>(1, per_head / (2 * kWavesNarrow));
  s = std::min<uint32_t>(s, std::max<uint32_t>(1, 3 * cu_count() / d.kv_head_count));
  return std::min<uint32_t>(s, 64);
}

uint64_t seam_route_scratch_words(const cf_kv_paged_attention_desc &d) {
  const uint64_t h = d.kv_head_count;
  return h * seam_route_chunks(d.page_count) * kRouteInfoWords + 4 * h * d.page_count + h;
}

cf_status seam_route_launch(const cf_kv_paged_attention_desc &d, uint32_t splits, float *partial, uint32_t *scratch,
                            hipStream_t s) {
  const uint32_t chunks = seam_route_chunks(d.page_count);
  uint32_t *info = scratch;
  uint4 *lists = reinterpret_cast<uint4 *>(info + static_cast<uint64_t>(d.kv_head_count) * chunks * kRouteInfoWords);
  uint32_t *taken = reinterpret_cast<uint32_t *>(lists + static_cast<uint64_t>(d.kv_head_count) * d.page_count);
  if ((reinterpret_cast<uintptr_t>(scratch) & 15u) != 0 || chunks > 64) return CF_ERR_INVALID_ARGUMENT;
  seam_list_kernel<<<chunks, kRouteChunk, 0, s>>>(d, lists, info);
  const dim3 grid(splits, d.kv_head_count);
  if (d.head_dim == 128)
    seam_group_kernel<128><<<grid, 64 * kWavesNarrow, 0, s>>>(d, splits, info, lists, taken, partial);
  else
    seam_group_kernel<64><<<grid, 64 * kWavesNarrow, 0, s>>>(d, splits, info, lists, taken, partial);
  return cfd::launch_status();
}

}  // namespace cfkv
