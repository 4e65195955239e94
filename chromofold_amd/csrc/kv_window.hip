// kv_window.hip — non-paged causal-windowed attention over block-Huffman K/V, decoded inside the consumer
// (cf_kv_attn_fused_async) and its decode-then-dense twin (cf_kv_attn_dense_async), on gfx950.
//
// Semantics of reference src/cuda/fused_kv_attention.cu:27-161: query i (< nq <= seq) attends rows
// j in [max(0, i - window + 1), i]; K[j][c] = (q - zero) * kscale[c] (per channel), V[j][c] = (q - zero) * vscale[j]
// (per token); score = (sum_c Q[i][c] K[j][c]) * sscale; out[i] = softmax-weighted sum of V rows. Same argument
// checks and status codes (dim > 128 or window > 512 -> CF_ERR_UNSUPPORTED). Both entry points here share one
// attention kernel and feed it bit-identical dequantised rows, so fused == dense bit for bit, as in the reference.
//
// gfx950 layout. The reference runs one thread per query and decodes every row of its window for that query
// (window-fold redundant decode, per-thread score/accumulator arrays in scratch). Here a 256-thread workgroup owns
// 32 consecutive queries; the rows their windows cover are decoded ONCE per workgroup, 64 rows at a time, straight
// into LDS (one lane per code block, a register bit window, the LUTs staged in LDS), then:
//   scores   lane = (query, 8-row group): 8 dot products over LDS rows, the K row read is a wave broadcast;
//   softmax  online across the 64-row chunks (running max / sum per query, 8 lanes per query, xor-shuffles);
//   PV       lane = (query, every 8th dim): 16 fp32 accumulators per lane.
// Row decode work drops from window x queries to (window + 32) x queries / 32.
#include <cmath>

#include "cf_device.hpp"
#include "chromofold/chromofold.h"
#include "huffman_core.hpp"

namespace {

constexpr int kThreads = 256;
constexpr int kQ = 32;       // queries per workgroup
constexpr int kRows = 64;    // K/V rows staged per chunk
constexpr int kMaxDim = CF_KV_MAX_HEAD_DIM;
constexpr int kLd = kMaxDim + 1;     // padded LDS row stride (floats)
constexpr int kLutStageBits = 12;    // LUTs of up to 2^12 entries are staged in LDS
constexpr int kMaxLen = 24;          // longest supported code lookahead

struct WinArgs {
  const uint32_t *kw, *vw;
  const int32_t *kb, *vb, *kl, *vl;
  int kmax, vmax;
  const float *kscale, *vscale, *Q;
  const float *Kd, *Vd;  // dense rows (the materialising path), else null
  float *out;
  int seq, dim, nq, window, block, zero;
  float sscale;
};

// decode symbols [s0, s1) of one stream (rows of `dim` symbols starting at row r0) into dst rows (stride kLd),
// dequantised; one thread per code block intersecting the range, threads [t0, t0 + nthreads)
template <bool kPerToken>
__device__ void decode_rows(const uint32_t *__restrict__ words, const int32_t *__restrict__ boff,
                            const int32_t *__restrict__ lut, int maxlen, int block, int zero,
                            const float *__restrict__ scale, int dim, int64_t r0, int nr, float *__restrict__ dst,
                            int t, int nthreads) {
  const int64_t s0 = r0 * dim, s1 = (r0 + nr) * dim;
  const int64_t b0 = s0 / block, b1 = (s1 + block - 1) / block;
  for (int64_t b = b0 + t; b < b1; b += nthreads) {
    const int64_t first = b * block, last = min(first + static_cast<int64_t>(block), s1);
    cfh::BitReader br(words, boff[b]);
    for (int64_t i = first; i < last; ++i) {
      const int e = br.decode(lut, maxlen);
      if (i < s0) continue;
      const int rel = static_cast<int>(i - s0);  // < kRows * kMaxDim
      const int r = rel / dim, c = rel - r * dim;
      const float s = kPerToken ? scale[r0 + r] : scale[c];
      dst[r * kLd + c] = static_cast<float>((e & 0xff) - zero) * s;
    }
  }
}

template <bool kDense>
__global__ void __launch_bounds__(kThreads) win_attn_kernel(WinArgs a) {
  __shared__ float s_q[kQ * kLd];
  __shared__ float s_k[kRows * kLd];
  __shared__ float s_v[kRows * kLd];
  __shared__ float s_p[kQ * (kRows + 1)];
  __shared__ int32_t s_lut[kDense ? 1 : 2 << kLutStageBits];
  const int t = threadIdx.x;
  const int dim = a.dim;
  const int i0 = blockIdx.x * kQ;
  const int nqt = min(kQ, a.nq - i0);
  for (int e = t; e < kQ * dim; e += kThreads) {
    const int r = e / dim, c = e - r * dim;
    s_q[r * kLd + c] = r < nqt ? a.Q[static_cast<int64_t>(i0 + r) * dim + c] : 0.f;
  }
  const int32_t *klut = a.kl, *vlut = a.vl;
  if constexpr (!kDense) {
    if (a.kmax <= kLutStageBits && a.vmax <= kLutStageBits) {
      for (int e = t; e < (1 << a.kmax); e += kThreads) s_lut[e] = a.kl[e];
      for (int e = t; e < (1 << a.vmax); e += kThreads) s_lut[(1 << kLutStageBits) + e] = a.vl[e];
      klut = s_lut;
      vlut = s_lut + (1 << kLutStageBits);
    }
  }
  // scores: query sq, rows sg*8 .. +8 of the chunk
  const int sq = t & (kQ - 1), sg = t >> 5;
  const int qi_s = i0 + sq;
  // PV: query pq, dims part + 8*j
  const int pq = t >> 3, part = t & 7;
  const int qi_p = i0 + pq;
  float acc[kMaxDim / 8];
#pragma unroll
  for (int j = 0; j < kMaxDim / 8; ++j) acc[j] = 0.f;
  float m = -INFINITY, l = 0.f;

  const int r_lo = max(0, i0 - a.window + 1), r_hi = i0 + nqt - 1;  // rows the tile's windows cover (inclusive)
  for (int c0 = r_lo; c0 <= r_hi; c0 += kRows) {
    const int nr = min(kRows, r_hi - c0 + 1);
    __syncthreads();  // previous chunk consumed (and Q / LUT staged on the first pass)
    if constexpr (kDense) {
      for (int e = t; e < nr * dim; e += kThreads) {
        const int r = e / dim, c = e - r * dim;
        s_k[r * kLd + c] = a.Kd[static_cast<int64_t>(c0 + r) * dim + c];
        s_v[r * kLd + c] = a.Vd[static_cast<int64_t>(c0 + r) * dim + c];
      }
    } else {
      if (t < kThreads / 2)
        decode_rows<false>(a.kw, a.kb, klut, a.kmax, a.block, a.zero, a.kscale, dim, c0, nr, s_k, t, kThreads / 2);
      else
        decode_rows<true>(a.vw, a.vb, vlut, a.vmax, a.block, a.zero, a.vscale, dim, c0, nr, s_v, t - kThreads / 2,
                          kThreads / 2);
    }
    __syncthreads();
    {  // scores of (sq, rows sg*8 .. +8): d outer so each Q element is read once
      float s[8];
#pragma unroll
      for (int rr = 0; rr < 8; ++rr) s[rr] = 0.f;
      const float *qrow = s_q + sq * kLd;
      const float *krow = s_k + (sg * 8) * kLd;
      for (int c = 0; c < dim; ++c) {
        const float qv = qrow[c];
#pragma unroll
        for (int rr = 0; rr < 8; ++rr) s[rr] += qv * krow[rr * kLd + c];
      }
#pragma unroll
      for (int rr = 0; rr < 8; ++rr) {
        const int r = sg * 8 + rr, j = c0 + r;
        const bool vis = sq < nqt && r < nr && j <= qi_s && j > qi_s - a.window;
        s_p[sq * (kRows + 1) + r] = vis ? s[rr] * a.sscale : -INFINITY;
      }
    }
    __syncthreads();
    // online softmax for query pq over this chunk: lanes part = 0..7 own rows part*8 .. +8
    float cm = -INFINITY;
    float *prow = s_p + pq * (kRows + 1);
#pragma unroll
    for (int rr = 0; rr < 8; ++rr) cm = fmaxf(cm, prow[part * 8 + rr]);
    cm = fmaxf(cm, __shfl_xor(cm, 1));
    cm = fmaxf(cm, __shfl_xor(cm, 2));
    cm = fmaxf(cm, __shfl_xor(cm, 4));
    const float mn = fmaxf(m, cm);
    float ps = 0.f;
    if (mn != -INFINITY) {
#pragma unroll
      for (int rr = 0; rr < 8; ++rr) {
        const float p = expf(prow[part * 8 + rr] - mn);  // exp(-inf) = 0 for hidden rows
        prow[part * 8 + rr] = p;
        ps += p;
      }
    }
    ps += __shfl_xor(ps, 1);
    ps += __shfl_xor(ps, 2);
    ps += __shfl_xor(ps, 4);
    __syncthreads();  // every p of the chunk written before the PV reads
    if (mn != -INFINITY) {
      const float alpha = expf(m - mn);  // m = -inf on the first visible chunk -> 0
      l = l * alpha + ps;
#pragma unroll
      for (int j = 0; j < kMaxDim / 8; ++j) acc[j] *= alpha;
      for (int r = 0; r < nr; ++r) {
        const float p = prow[r];
        const float *vrow = s_v + r * kLd;
#pragma unroll
        for (int j = 0; j < kMaxDim / 8; ++j) {
          const int c = part + 8 * j;
          if (c < dim) acc[j] += p * vrow[c];
        }
      }
      m = mn;
    }
  }
  if (pq < nqt) {
    const float inv = 1.f / l;  // row qi_p itself is always visible, so l > 0
    float *o = a.out + static_cast<int64_t>(qi_p) * dim;
#pragma unroll
    for (int j = 0; j < kMaxDim / 8; ++j) {
      const int c = part + 8 * j;
      if (c < dim) o[c] = acc[j] * inv;
    }
  }
}

// decode every row of one stream to dense fp32 [seq, dim] (one thread per code block)
template <bool kPerToken>
__global__ void __launch_bounds__(kThreads) decode_dense_kernel(const uint32_t *__restrict__ words,
                                                                const int32_t *__restrict__ boff,
                                                                const int32_t *__restrict__ lut, int maxlen, int block,
                                                                int seq, int dim, int zero,
                                                                const float *__restrict__ scale,
                                                                float *__restrict__ dense) {
  const int64_t b = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t n = static_cast<int64_t>(seq) * dim;
  const int64_t first = b * block;
  if (first >= n) return;
  const int64_t last = min(first + static_cast<int64_t>(block), n);
  cfh::BitReader br(words, boff[b]);
  for (int64_t i = first; i < last; ++i) {
    const int e = br.decode(lut, maxlen);
    const int64_t r = i / dim;
    const float s = kPerToken ? scale[r] : scale[i - r * dim];
    dense[i] = static_cast<float>((e & 0xff) - zero) * s;
  }
}

// reference fused_kv_attention.cu:101-113, plus the longest lookahead this decoder supports
cf_status validate(const uint32_t *kw, const int32_t *kb, const int32_t *kl, int kmax, const uint32_t *vw,
                   const int32_t *vb, const int32_t *vl, int vmax, const float *kscale, const float *vscale,
                   const float *Q, const float *out, int seq, int dim, int nq, int window, int block, float sscale) {
  if (!kw || !kb || !kl || !vw || !vb || !vl || !kscale || !vscale || !Q || !out) return CF_ERR_INVALID_ARGUMENT;
  if (seq <= 0 || dim <= 0 || nq < 0 || nq > seq || window <= 0 || block <= 0 || kmax <= 0 || vmax <= 0)
    return CF_ERR_INVALID_ARGUMENT;
  if (!std::isfinite(sscale)) return CF_ERR_INVALID_ARGUMENT;
  if (dim > CF_KV_MAX_HEAD_DIM || window > CF_KV_MAX_WINDOW || kmax > kMaxLen || vmax > kMaxLen)
    return CF_ERR_UNSUPPORTED;
  return CF_OK;
}

}  // namespace

extern "C" cf_status cf_kv_attn_fused_async(const uint32_t *kw, const int32_t *kb, const int32_t *kl, int kmax,
                                            const uint32_t *vw, const int32_t *vb, const int32_t *vl, int vmax,
                                            const float *kscale, const float *vscale, const float *Q, float *out,
                                            int seq, int dim, int nq, int window, int block, int zero, float sscale,
                                            void *stream) {
  const cf_status st = validate(kw, kb, kl, kmax, vw, vb, vl, vmax, kscale, vscale, Q, out, seq, dim, nq, window,
                                block, sscale);
  if (st != CF_OK || nq == 0) return st;
  const WinArgs a{kw, vw, kb, vb, kl, vl, kmax, vmax, kscale, vscale, Q, nullptr, nullptr, out,
                  seq, dim, nq, window, block, zero, sscale};
  win_attn_kernel<false><<<cfd::grid_for(nq, kQ), kThreads, 0, cfd::as_stream(stream)>>>(a);
  return cfd::launch_status();
}

extern "C" cf_status cf_kv_attn_dense_async(const uint32_t *kw, const int32_t *kb, const int32_t *kl, int kmax,
                                            const uint32_t *vw, const int32_t *vb, const int32_t *vl, int vmax,
                                            const float *kscale, const float *vscale, const float *Q, float *Kd,
                                            float *Vd, float *out, int seq, int dim, int nq, int window, int block,
                                            int zero, float sscale, void *stream) {
  const cf_status st = validate(kw, kb, kl, kmax, vw, vb, vl, vmax, kscale, vscale, Q, out, seq, dim, nq, window,
                                block, sscale);
  if (st != CF_OK) return st;
  if (!Kd || !Vd) return CF_ERR_INVALID_ARGUMENT;
  if (nq == 0) return CF_OK;
  const hipStream_t s = cfd::as_stream(stream);
  const int64_t nblocks = (static_cast<int64_t>(seq) * dim + block - 1) / block;
  const unsigned g = cfd::grid_for(static_cast<size_t>(nblocks), kThreads);
  decode_dense_kernel<false><<<g, kThreads, 0, s>>>(kw, kb, kl, kmax, block, seq, dim, zero, kscale, Kd);
  decode_dense_kernel<true><<<g, kThreads, 0, s>>>(vw, vb, vl, vmax, block, seq, dim, zero, vscale, Vd);
  const WinArgs a{kw, vw, kb, vb, kl, vl, kmax, vmax, kscale, vscale, Q, Kd, Vd, out,
                  seq, dim, nq, window, block, zero, sscale};
  win_attn_kernel<true><<<cfd::grid_for(nq, kQ), kThreads, 0, s>>>(a);
  return cfd::launch_status();
}
