// kv_batched.hip — batched compressed paged-KV attention decode on gfx950 (kv_codec_ext.h entry point).
//
// One workgroup = 4 wavefronts serves one (sequence, KV head, context split). Each wavefront walks "page quads":
// four consecutive 16-token pages, one per 16-lane group. Lane (G, t) = lane 16G + t:
//   K phase: lane decodes token t of page G (its 16 interleaved rANS states are the 16 lanes of the group);
//            every decoded quad of 4 dims goes straight into v_mfma_f32_4x4x4f16 as the B operand, with the
//            GQA group's 4 query heads (split into f16 hi + lo parts for fp32-grade scores) as the A operand, so
//            the lane ends up holding its token's 4 head scores. Nothing decoded is written anywhere.
//   softmax: one running max per head for the whole wavefront (so the 4 page groups can be summed at the end),
//            probabilities pre-scaled by the page's V scale go to a 512-byte LDS tile.
//   V phase: lane decodes dims {t + 16i} of page G, 4 tokens per quad, again straight into a 4x4x4 MFMA
//            (A = probabilities of those 4 tokens for the 4 heads, B = the 4 decoded values) accumulating the
//            lane's 4 heads x 8 dims output.
// Codec decode per quad: one rANS step (LDS slot table, 64-bit entry = freq/offset + the four 2-bit high parts
// already spread to their bytes), three bit-sliced low-part words per 4 quads, and two v_perm to build the f16
// operand (1024 + symbol; the constant 1024+128 offset is folded out with the sum of the other operand).
// Split-context partial states (m, l, acc) are merged by a second small kernel (online-softmax merge,
// reference src/runtime/kv_runtime.cpp:219-243 semantics).
#include <hip/hip_fp16.h>

#include <cmath>
#include <cstring>

#include "cf_device.hpp"
#include "chromofold/kv_codec_ext.h"

namespace {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kGqa = 4;            // MFMA rows: query heads of one KV head (gqa < 4 pads with zero queries)
constexpr uint32_t kSlots = 1u << CF_KV_RANS_PROB_BITS;
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

__device__ __forceinline__ float4_t mfma4(half4_t a, half4_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_4x4x4f16(a, b, c, 0, 0, 0);
}

// low-part byte word of quad qd (0..3) of a 16-value group from its three bit-sliced words
__device__ __forceinline__ uint32_t lows_of(uint32_t n0, uint32_t n1, uint32_t c, int qd) {
  const uint32_t n = (qd < 2) ? n0 : n1;
  const uint32_t nib = (qd & 1) ? ((n >> 4) & 0x0F0F0F0Fu) : (n & 0x0F0F0F0Fu);
  const uint32_t cr = ((c >> (2 * qd)) << 4) & 0x30303030u;
  return nib | cr;
}

struct PageRef {
  const uint8_t *blob;  // nullptr when the group has no page this iteration
  uint32_t kw, vw;      // word counts
  float ks, vs;
  uint32_t tok0;        // first token index of the page
  uint32_t ntok;        // tokens present in the page
};

// rANS step for one quad. x: lane state; cursor: word index of the group's shared stream (group-uniform).
__device__ __forceinline__ uint32_t rans_quad(const uint2 *__restrict__ tab, uint32_t &x, uint32_t &cursor,
                                              const uint16_t *__restrict__ words, bool active, int gshift,
                                              uint32_t below) {
  const uint2 e = tab[x & (kSlots - 1)];
  const uint32_t f = (e.x & (kSlots - 1)) + 1u;
  const uint32_t cs = (e.x >> 11) & (kSlots - 1);
  x = f * (x >> CF_KV_RANS_PROB_BITS) + cs;
  const bool need = active && x < 65536u;
  const uint64_t m = __ballot(need);
  const uint32_t gm = static_cast<uint32_t>(m >> gshift) & 0xFFFFu;
  if (need) x = (x << 16) | words[cursor + __popc(gm & below)];
  cursor += __popc(gm);
  return e.y;  // spread high parts
}

template <int D, int CODEC>
__global__ __launch_bounds__(kThreads) void kv_batched_kernel(cf_kv_batched_desc d, uint32_t splits,
                                                              float *__restrict__ partial) {
  constexpr int NQ = D / 4;        // quads per lane per stream
  constexpr int NG = D / 16;       // low-part groups per lane
  constexpr int LOWS = 3 * NG * 16;  // u32 words of one stream's low parts
  __shared__ uint2 s_tab[2][CODEC == CF_KV_CODEC_RANS_HYBRID ? kSlots : 1];
  __shared__ _Float16 s_q[2][kGqa][D];         // query heads, hi and lo f16 parts (softmax scale folded in)
  __shared__ _Float16 s_p[kWaves][4][kGqa][16];  // per wave: [page group][head][token] probabilities * v_scale
  __shared__ float s_red[kWaves][kGqa * (D + 2)];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int G = lane >> 4, t = lane & 15;
  const uint32_t split = blockIdx.x, head = blockIdx.y, seq = blockIdx.z;
  const uint32_t gqa = d.query_head_count / d.kv_head_count;

  // ---- stage tables and queries
  if constexpr (CODEC == CF_KV_CODEC_RANS_HYBRID) {
    const uint2 *tk = reinterpret_cast<const uint2 *>(d.tables + static_cast<size_t>(2 * head) * CF_KV_RANS_TABLE_BYTES);
    const uint2 *tv = tk + kSlots;
    for (uint32_t i = threadIdx.x; i < kSlots; i += kThreads) {
      s_tab[0][i] = tk[i];
      s_tab[1][i] = tv[i];
    }
  }
  for (int i = threadIdx.x; i < kGqa * D; i += kThreads) {
    const int h = i / D, dd = i % D;
    float q = 0.0f;
    if (static_cast<uint32_t>(h) < gqa)
      q = d.queries[(static_cast<size_t>(seq) * d.query_head_count + head * gqa + h) * D + dd] * d.softmax_scale;
    const _Float16 hi = static_cast<_Float16>(q);
    s_q[0][h][dd] = hi;
    s_q[1][h][dd] = static_cast<_Float16>(q - static_cast<float>(hi));
  }
  __syncthreads();

  // per-head sum of the query operand as the MFMA sees it (hi + lo), for the 1152 offset fold; every lane keeps
  // all heads (no cross-lane read later inside lane-divergent code)
  float qsum[kGqa];
#pragma unroll
  for (int h = 0; h < kGqa; ++h) {
    qsum[h] = 0.0f;
    for (int dd = 0; dd < D; ++dd) qsum[h] += static_cast<float>(s_q[0][h][dd]) + static_cast<float>(s_q[1][h][dd]);
  }

  const uint32_t ntok_seq = d.seq_tokens[seq];
  const uint32_t qpos = d.query_pos[seq];
  const uint32_t visible = min(ntok_seq, qpos + 1);  // tokens [0, visible) are attended
  const uint32_t npages = min((visible + 15) / 16, d.max_pages);
  const uint32_t nquads = (npages + 3) / 4;
  const uint32_t per = (nquads + splits - 1) / splits;
  const uint32_t qa = min(nquads, split * per), qb = min(nquads, qa + per);
  const uint32_t *prow = d.page_offsets + (static_cast<size_t>(seq) * d.kv_head_count + head) * d.max_pages;

  float m_run[kGqa], l_run[kGqa], corr[kGqa];
  float4_t acc_v[D / 16];
#pragma unroll
  for (int h = 0; h < kGqa; ++h) {
    m_run[h] = -INFINITY;
    l_run[h] = 0.0f;
    corr[h] = 0.0f;
  }
#pragma unroll
  for (int i = 0; i < D / 16; ++i) acc_v[i] = float4_t{0, 0, 0, 0};

  const int gshift = 16 * G;
  const uint32_t below = (1u << t) - 1u;

  for (uint32_t qi = qa + wave; qi < qb; qi += kWaves) {
    // ---- page of this lane group
    PageRef pg{};
    const uint32_t p = 4 * qi + G;
    if (p < npages) {
      pg.blob = d.pool + static_cast<size_t>(prow[p]) * 16;
      const cf_kv_rans_page_header *hd = reinterpret_cast<const cf_kv_rans_page_header *>(pg.blob);
      pg.kw = hd->k_word_count;
      pg.vw = hd->v_word_count;
      pg.ks = hd->k_scale;
      pg.vs = hd->v_scale;
      pg.tok0 = 16 * p;
      pg.ntok = min(16u, visible - 16 * p);
    }
    const bool active = pg.blob != nullptr;

    // ---- K phase: scores of token t of page G for the 4 heads
    float4_t sa = {0, 0, 0, 0}, sb = {0, 0, 0, 0};
    if constexpr (CODEC == CF_KV_CODEC_RANS_HYBRID) {
      const uint32_t *st = active ? reinterpret_cast<const uint32_t *>(pg.blob + 32) : nullptr;
      const uint32_t *lows = active ? reinterpret_cast<const uint32_t *>(pg.blob + 160) : nullptr;
      const uint16_t *words = active ? reinterpret_cast<const uint16_t *>(pg.blob + 160 + 2 * LOWS * 4) : nullptr;
      uint32_t x = active ? st[t] : 0u, cur = 0;
#pragma unroll 2
      for (int g = 0; g < NG; ++g) {
        uint32_t n0 = 0, n1 = 0, c = 0;
        if (active) {
          n0 = lows[(g * 3 + 0) * 16 + t];
          n1 = lows[(g * 3 + 1) * 16 + t];
          c = lows[(g * 3 + 2) * 16 + t];
        }
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
          const uint32_t hi = rans_quad(s_tab[0], x, cur, words, active, gshift, below);
          const uint32_t bytes = active ? (lows_of(n0, n1, c, qd) | hi) : 0x80808080u;
          const half4_t bk = bytes_to_half4(bytes);
          const int q = 4 * g + qd;
          const half4_t a_hi = *reinterpret_cast<const half4_t *>(&s_q[0][lane & 3][4 * q]);
          const half4_t a_lo = *reinterpret_cast<const half4_t *>(&s_q[1][lane & 3][4 * q]);
          sa = mfma4(a_hi, bk, sa);
          sb = mfma4(a_lo, bk, sb);
        }
      }
    } else {  // CF_KV_CODEC_INT8
      const uint32_t *kb = active ? reinterpret_cast<const uint32_t *>(pg.blob + 32) : nullptr;
#pragma unroll 4
      for (int q = 0; q < NQ; ++q) {
        const uint32_t bytes = active ? kb[q * 16 + t] : 0x80808080u;
        const half4_t bk = bytes_to_half4(bytes);
        const half4_t a_hi = *reinterpret_cast<const half4_t *>(&s_q[0][lane & 3][4 * q]);
        const half4_t a_lo = *reinterpret_cast<const half4_t *>(&s_q[1][lane & 3][4 * q]);
        sa = mfma4(a_hi, bk, sa);
        sb = mfma4(a_lo, bk, sb);
      }
    }

    // ---- online softmax over the wavefront's 64 tokens
    const bool tok_ok = active && static_cast<uint32_t>(t) < pg.ntok;
    float s[kGqa], mx[kGqa];
#pragma unroll
    for (int h = 0; h < kGqa; ++h) {
      s[h] = tok_ok ? (sa[h] + sb[h] - kOffset * qsum[h]) * pg.ks : -INFINITY;
      mx[h] = s[h];
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
#pragma unroll
      for (int h = 0; h < kGqa; ++h) mx[h] = fmaxf(mx[h], __shfl_xor(mx[h], o));
    float alpha[kGqa];
#pragma unroll
    for (int h = 0; h < kGqa; ++h) {
      const float mn = fmaxf(m_run[h], mx[h]);
      alpha[h] = (m_run[h] == -INFINITY) ? 0.0f : __expf(m_run[h] - mn);
      const float pr = tok_ok ? __expf(s[h] - mn) : 0.0f;
      l_run[h] = l_run[h] * alpha[h] + pr;
      const _Float16 pv = static_cast<_Float16>(pr * (active ? pg.vs : 0.0f));
      s_p[wave][G][h][t] = pv;
      corr[h] = corr[h] * alpha[h] + kOffset * static_cast<float>(pv);
      m_run[h] = mn;
    }
#pragma unroll
    for (int i = 0; i < D / 16; ++i)
#pragma unroll
      for (int h = 0; h < kGqa; ++h) acc_v[i][h] *= alpha[h];
    __builtin_amdgcn_wave_barrier();  // s_p written by this wave only; LDS ops of a wave complete in order

    // ---- V phase: out[h][t + 16i] += sum over tokens of p * v
    if constexpr (CODEC == CF_KV_CODEC_RANS_HYBRID) {
      const uint32_t *st = active ? reinterpret_cast<const uint32_t *>(pg.blob + 32 + 64) : nullptr;
      const uint32_t *lows = active ? reinterpret_cast<const uint32_t *>(pg.blob + 160 + LOWS * 4) : nullptr;
      const uint16_t *words =
          active ? reinterpret_cast<const uint16_t *>(pg.blob + 160 + 2 * LOWS * 4) + pg.kw : nullptr;
      uint32_t x = active ? st[t] : 0u, cur = 0;
#pragma unroll 1
      for (int tq = 0; tq < 4; ++tq) {
        const half4_t pa = *reinterpret_cast<const half4_t *>(&s_p[wave][G][lane & 3][4 * tq]);
#pragma unroll
        for (int gg = 0; gg < NG / 4; ++gg) {
          const int g = tq * (NG / 4) + gg;  // low-part group: quads 4g .. 4g+3 of this lane
          uint32_t n0 = 0, n1 = 0, c = 0;
          if (active) {
            n0 = lows[(g * 3 + 0) * 16 + t];
            n1 = lows[(g * 3 + 1) * 16 + t];
            c = lows[(g * 3 + 2) * 16 + t];
          }
#pragma unroll
          for (int qd = 0; qd < 4; ++qd) {
            const uint32_t hi = rans_quad(s_tab[1], x, cur, words, active, gshift, below);
            const uint32_t bytes = active ? (lows_of(n0, n1, c, qd) | hi) : 0x80808080u;
            const int i = 4 * gg + qd;  // dim index: lane dim t + 16 i
            acc_v[i] = mfma4(pa, bytes_to_half4(bytes), acc_v[i]);
          }
        }
      }
    } else {
      const uint32_t *vb = active ? reinterpret_cast<const uint32_t *>(pg.blob + 32 + 16 * D) : nullptr;
#pragma unroll 1
      for (int tq = 0; tq < 4; ++tq) {
        const half4_t pa = *reinterpret_cast<const half4_t *>(&s_p[wave][G][lane & 3][4 * tq]);
#pragma unroll
        for (int i = 0; i < D / 16; ++i) {
          const int q = tq * (D / 16) + i;
          const uint32_t bytes = active ? vb[q * 16 + t] : 0x80808080u;
          acc_v[i] = mfma4(pa, bytes_to_half4(bytes), acc_v[i]);
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
  }

  // ---- reduce the wavefront: sum the 4 page groups (lanes t, t+16, t+32, t+48), l and corr over all lanes
#pragma unroll
  for (int i = 0; i < D / 16; ++i)
#pragma unroll
    for (int h = 0; h < kGqa; ++h) {
      float v = acc_v[i][h];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      acc_v[i][h] = v;
    }
#pragma unroll
  for (int h = 0; h < kGqa; ++h)
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      l_run[h] += __shfl_xor(l_run[h], o);
      corr[h] += __shfl_xor(corr[h], o);
    }
  // wave partial -> LDS: [h][D] acc (minus offset correction), then m, l
  float *red = s_red[wave];
  if (lane < 16) {
#pragma unroll
    for (int i = 0; i < D / 16; ++i)
#pragma unroll
      for (int h = 0; h < kGqa; ++h) red[h * (D + 2) + t + 16 * i] = acc_v[i][h] - corr[h];
  }
  if (lane < kGqa) {
    red[lane * (D + 2) + D] = m_run[lane];
    red[lane * (D + 2) + D + 1] = l_run[lane];
  }
  __syncthreads();

  // ---- merge the 4 wavefronts; write the split partial (or the final output when splits == 1)
  for (int i = threadIdx.x; i < kGqa * D; i += kThreads) {
    const int h = i / D, dd = i % D;
    float m = -INFINITY;
    for (int w = 0; w < kWaves; ++w) m = fmaxf(m, s_red[w][h * (D + 2) + D]);
    float l = 0.0f, o = 0.0f;
    if (m != -INFINITY)
      for (int w = 0; w < kWaves; ++w) {
        const float mw = s_red[w][h * (D + 2) + D];
        if (mw == -INFINITY) continue;
        const float sc = __expf(mw - m);
        l += s_red[w][h * (D + 2) + D + 1] * sc;
        o += s_red[w][h * (D + 2) + dd] * sc;
      }
    if (splits == 1) {
      if (static_cast<uint32_t>(h) < gqa)
        d.output[(static_cast<size_t>(seq) * d.query_head_count + head * gqa + h) * D + dd] = l > 0.0f ? o / l : 0.0f;
    } else {
      float *pp = partial + ((static_cast<size_t>(seq) * d.kv_head_count + head) * splits + split) * (kGqa * (D + 2));
      pp[h * (D + 2) + dd] = o;
      if (dd == 0) {
        pp[h * (D + 2) + D] = m;
        pp[h * (D + 2) + D + 1] = l;
      }
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
  float m = -INFINITY;
  for (uint32_t s = 0; s < splits; ++s) m = fmaxf(m, pp[s * (kGqa * (D + 2)) + h * (D + 2) + D]);
  float l = 0.0f, o = 0.0f;
  if (m != -INFINITY)
    for (uint32_t s = 0; s < splits; ++s) {
      const float *q = pp + s * (kGqa * (D + 2)) + h * (D + 2);
      if (q[D] == -INFINITY) continue;
      const float sc = __expf(q[D] - m);
      l += q[D + 1] * sc;
      o += q[dd] * sc;
    }
  d.output[(static_cast<size_t>(seq) * d.query_head_count + head * gqa + h) * D + dd] = l > 0.0f ? o / l : 0.0f;
}

uint32_t choose_splits(const cf_kv_batched_desc *d) {
  if (d->splits) return d->splits;
  const uint32_t units = d->seq_count * d->kv_head_count;
  const uint32_t quads = (d->max_pages + 3) / 4;
  uint32_t s = (2048 + units - 1) / units;           // aim at ~2048 workgroups (8 per CU)
  s = std::min<uint32_t>(s, std::max<uint32_t>(1, quads / kWaves));  // keep >= one quad per wavefront
  return std::max<uint32_t>(1, std::min<uint32_t>(s, 64));
}

}  // namespace

extern "C" cf_status cf_kv_validate_batched_desc(const cf_kv_batched_desc *d) {
  if (!d || d->struct_size != sizeof(cf_kv_batched_desc) || d->abi_version != CF_KV_EXT_ABI_VERSION)
    return CF_ERR_INVALID_ARGUMENT;
  if (!d->pool || !d->page_offsets || !d->seq_tokens || !d->query_pos || !d->queries || !d->output ||
      d->seq_count == 0 || d->kv_head_count == 0 || d->query_head_count == 0 ||
      d->query_head_count % d->kv_head_count != 0 || !std::isfinite(d->softmax_scale))
    return CF_ERR_INVALID_ARGUMENT;
  if (d->codec != CF_KV_CODEC_INT8 && d->codec != CF_KV_CODEC_RANS_HYBRID) return CF_ERR_UNSUPPORTED;
  if (d->codec == CF_KV_CODEC_RANS_HYBRID && !d->tables) return CF_ERR_INVALID_ARGUMENT;
  if (d->query_head_count / d->kv_head_count > kGqa) return CF_ERR_UNSUPPORTED;
  if (d->head_dim != 64 && d->head_dim != 128) return CF_ERR_UNSUPPORTED;
  if (d->seq_count > 65535 || d->kv_head_count > 65535) return CF_ERR_UNSUPPORTED;
  return CF_OK;
}

extern "C" uint64_t cf_kv_batched_workspace_bytes(const cf_kv_batched_desc *d) {
  if (cf_kv_validate_batched_desc(d) != CF_OK) return 0;
  const uint32_t s = choose_splits(d);
  if (s <= 1) return 0;
  return static_cast<uint64_t>(d->seq_count) * d->kv_head_count * s * kGqa * (d->head_dim + 2) * sizeof(float);
}

extern "C" cf_status cf_kv_paged_attention_batched_async(const cf_kv_batched_desc *d, void *stream) {
  const cf_status v = cf_kv_validate_batched_desc(d);
  if (v != CF_OK) return v;
  const uint32_t splits = choose_splits(d);
  const uint64_t need = cf_kv_batched_workspace_bytes(d);
  if (need && (!d->workspace || d->workspace_bytes < need)) return CF_ERR_INVALID_ARGUMENT;
  const hipStream_t s = cfd::as_stream(stream);
  float *ws = static_cast<float *>(d->workspace);
  const dim3 grid(splits, d->kv_head_count, d->seq_count);
#define CF_LAUNCH(D, C) kv_batched_kernel<D, C><<<grid, kThreads, 0, s>>>(*d, splits, ws)
  if (d->head_dim == 128) {
    if (d->codec == CF_KV_CODEC_RANS_HYBRID) CF_LAUNCH(128, CF_KV_CODEC_RANS_HYBRID);
    else CF_LAUNCH(128, CF_KV_CODEC_INT8);
  } else {
    if (d->codec == CF_KV_CODEC_RANS_HYBRID) CF_LAUNCH(64, CF_KV_CODEC_RANS_HYBRID);
    else CF_LAUNCH(64, CF_KV_CODEC_INT8);
  }
#undef CF_LAUNCH
  if (splits > 1) {
    const dim3 g2(d->kv_head_count, d->seq_count);
    if (d->head_dim == 128) kv_merge_kernel<128><<<g2, kGqa * 128, 0, s>>>(*d, splits, ws);
    else kv_merge_kernel<64><<<g2, kGqa * 64, 0, s>>>(*d, splits, ws);
  }
  return cfd::launch_status();
}
