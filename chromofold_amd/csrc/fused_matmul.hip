// fused_matmul.hip — decode-in-matmul on gfx950: y[b, m] = sum_k x[b, k] * W[m, k] with W held only in its
// entropy-coded form (the dense weight matrix never exists in memory).
//
//   cf_fused_matmul_async  reference src/cuda/fused_matmul.cu:17-38, 67-80: one block-Huffman stream over row-major
//                          W (block_off every `block` symbols, one LUT), W = (q - zero) * scale per tensor, fp32 x;
//   cf_dense_matmul_async  reference src/cuda/fused_matmul.cu:41-65, 83-96: decode W to dense fp32 (the reference's
//                          exact values), then the reference's k-outer / b-inner fp32 GEMM order per output.
// (The band-table int4 format of chromofold_qw.h has its own kernel in qw_matmul.hip.)
//
// A 1024-thread workgroup (16 waves) owns 16 rows of W:
//   decode   lanes decode the code blocks / segments covering the tile's 16 rows x a 4096-column chunk straight
//            into LDS as u8 symbols (register bit window, LUT staged in LDS);
//   MFMA     v_mfma_f32_16x16x16_bf16 with A = x (batch x k, 16 batch rows per tile) and B = the decoded symbols
//            (k x 16 rows). Symbols are small integers, exact in bf16. fp32 activations are split exactly into three
//            bf16 terms (x = h + m + l, 8 mantissa bits each), so every product is exact and only the fp32
//            accumulation rounds. The 16 waves split the k-steps; per-wave partial
//            tiles are reduced through LDS in a fixed order (deterministic), scaled, and written once — y needs no
//            prior zeroing and is never read-modify-written.
// Batches are padded to tiles of 16 (MFMA rows); 4 batch tiles (B <= 64) are served per pass over W.
#include <cmath>

#include "cf_device.hpp"
#include "chromofold/chromofold_extra.h"
#include "huffman_core.hpp"

namespace {

typedef short bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kTM = 16;                // W rows per workgroup (MFMA N)
constexpr int kKC = 4096;              // columns staged per chunk
// Symbol tile layout: 64-column segments 68 bytes apart inside a row (the 64 lanes of a wave, one segment each,
// write word q of their segments to 64 distinct banks: 17 * s + q), rows kLdB bytes apart (kLdB / 4 = 4 mod 64:
// the B-fragment read of 16 rows x 4 column groups hits 64 distinct banks).
constexpr int kSegB = 68;
constexpr int kLdB = (kKC / 64) * kSegB + 16;
constexpr int kBT = 4;                 // batch tiles of 16 per pass
constexpr int kLutBits = 12;           // LUTs up to 2^12 entries are staged in LDS
constexpr int kSmemW = kTM * kLdB;     // u8 symbol tile
constexpr int kSmemRed = kWaves * kBT * 256 * 4;
constexpr int kSmemTile = kSmemW > kSmemRed ? kSmemW : kSmemRed;

static_assert(kTM * (kKC / 64) == kThreads, "one 64-column segment per lane per chunk");

struct Args {
  const uint32_t *words;
  const int32_t *block_off;
  const int32_t *lut;
  int maxlen, block;
  const float *x;
  float *y;
  int B, M, K;
  float scale;
  int zero;   // value subtracted from every symbol
};

// x = h + m + l exactly: each term keeps the next 8 significant bits (bf16 truncation)
__device__ __forceinline__ void split3(float x, short &h, short &m, short &l) {
  const uint32_t hb = __float_as_uint(x) & 0xFFFF0000u;
  const float r1 = x - __uint_as_float(hb);
  const uint32_t mb = __float_as_uint(r1) & 0xFFFF0000u;
  const float r2 = r1 - __uint_as_float(mb);
  h = static_cast<short>(hb >> 16);
  m = static_cast<short>(mb >> 16);
  l = static_cast<short>(__float_as_uint(r2) >> 16);
}

__device__ __forceinline__ short bf16_of_int(int v) {  // |v| <= 256: exact
  return static_cast<short>(__float_as_uint(static_cast<float>(v)) >> 16);
}

__global__ void __launch_bounds__(kThreads) fused_matmul_kernel(Args a) {
  __shared__ __attribute__((aligned(16))) uint8_t s_tile[kSmemTile];
  __shared__ int32_t s_lut[1 << kLutBits];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int m0 = blockIdx.x * kTM;
  const int B = a.B, M = a.M, K = a.K;
  const int zc = min(255, max(0, a.zero));  // symbols are u8: q - zc stays within +-255

  // the code table, staged in LDS when it fits
  const int32_t *lut = a.lut;
  const int maxlen = a.maxlen;
  if (a.maxlen <= kLutBits) {
    for (int e = t; e < (1 << a.maxlen); e += kThreads) s_lut[e] = a.lut[e];
    lut = s_lut;
  }

  for (int bt0 = 0; bt0 < (B + 15) / 16; bt0 += kBT) {
    f32x4_t acc[kBT];
#pragma unroll
    for (int i = 0; i < kBT; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    for (int kc0 = 0; kc0 < K; kc0 += kKC) {
      const int kc1 = min(K, kc0 + kKC);
      __syncthreads();  // previous chunk (or the table staging) done
      {  // decode: lane -> (row r, 64-column segment s) of the chunk; 4 symbols per LDS word write
        const int r = t >> 6, s = t & 63;
        const int m = m0 + r, k0 = kc0 + 64 * s;
        uint32_t *dst = reinterpret_cast<uint32_t *>(s_tile + r * kLdB + kSegB * s);
        const int n = (m < M && k0 < kc1) ? min(64, kc1 - k0) : 0;
        const uint32_t pad = static_cast<uint32_t>(zc) * 0x01010101u;  // padding contributes q - zc = 0
        // skip-decode from the start of the code block holding W[m, k0]
        const int64_t f = static_cast<int64_t>(m) * K + k0;
        const int64_t bs = n > 0 ? f / a.block : 0;
        cfh::BitReader br(a.words, static_cast<int64_t>(a.block_off[bs]));
        if (n > 0)
          for (int64_t i = bs * a.block; i < f; ++i) br.decode(lut, maxlen);
#pragma unroll 4
        for (int q = 0; q < 16; ++q) {
          uint32_t w = pad;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (4 * q + e < n) w = (w & ~(0xFFu << (8 * e))) | ((br.decode(lut, maxlen) & 0xFFu) << (8 * e));
          dst[q] = w;
        }
      }
      __syncthreads();
      // MFMA: wave takes k-steps wave, wave + 16, ...; lane's B fragment = rows (lane & 15), k = 4 * (lane >> 4)
      const int nsteps = (kc1 - kc0 + 15) / 16;
      const int bn = lane & 15, bk = 4 * (lane >> 4);
      for (int st = wave; st < nsteps; st += kWaves) {
        const int kk = st * 16 + bk;  // column within the chunk
        const uint32_t q4 = *reinterpret_cast<const uint32_t *>(s_tile + bn * kLdB + (kk >> 6) * kSegB + (kk & 63));
        bf16x4_t bfrag;
        bfrag[0] = bf16_of_int(static_cast<int>(q4 & 0xff) - zc);
        bfrag[1] = bf16_of_int(static_cast<int>((q4 >> 8) & 0xff) - zc);
        bfrag[2] = bf16_of_int(static_cast<int>((q4 >> 16) & 0xff) - zc);
        bfrag[3] = bf16_of_int(static_cast<int>(q4 >> 24) - zc);
        const int k = kc0 + kk;
#pragma unroll
        for (int i = 0; i < kBT; ++i) {
          const int b = (bt0 + i) * 16 + (lane & 15);
          if ((bt0 + i) * 16 >= B) break;  // wave-uniform
          const float *xr = a.x + static_cast<int64_t>(b) * K;
          bf16x4_t ah, am, al;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float xv = (b < B && k + e < K) ? xr[k + e] : 0.f;
            short h, mm, l;
            split3(xv, h, mm, l);
            ah[e] = h;
            am[e] = mm;
            al[e] = l;
          }
          acc[i] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ah, bfrag, acc[i], 0, 0, 0);
          acc[i] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(am, bfrag, acc[i], 0, 0, 0);
          acc[i] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(al, bfrag, acc[i], 0, 0, 0);
        }
      }
    }
    // cross-wave reduction in a fixed order, then one write of y per (b, m)
    __syncthreads();
    float *red = reinterpret_cast<float *>(s_tile);
#pragma unroll
    for (int i = 0; i < kBT; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) red[(wave * kBT + i) * 256 + lane * 4 + e] = acc[i][e];
    __syncthreads();
    {
      const int i = t >> 8, idx = t & 255;  // tile i of the pass, fragment slot idx = lane * 4 + reg
      const int fl = idx >> 2, fr = idx & 3;
      const int b = (bt0 + i) * 16 + 4 * (fl >> 4) + fr, m = m0 + (fl & 15);
      float s = 0.f;
      for (int w = 0; w < kWaves; ++w) s += red[(w * kBT + i) * 256 + idx];
      if (b < B && m < M) {
        // out-of-range zero points: the u8 symbols were offset by zc, the rest is -(zero - zc) * sum_k x[b, k]
        float corr = 0.f;
        if (a.zero != zc) {
          const float *xr = a.x + static_cast<int64_t>(b) * K;
          for (int k = 0; k < K; ++k) corr += xr[k];
          corr *= static_cast<float>(a.zero - zc);
        }
        a.y[static_cast<int64_t>(b) * M + m] = (s - corr) * a.scale;
      }
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------------------------ materialising twin (reference)
__global__ void __launch_bounds__(256) decode_dense_kernel(const uint32_t *__restrict__ words,
                                                           const int32_t *__restrict__ block_off,
                                                           const int32_t *__restrict__ lut, int maxlen, int block,
                                                           int64_t n, float scale, int zero, float *__restrict__ W) {
  const int64_t b = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t first = b * block;
  if (first >= n) return;
  const int64_t last = min(first + static_cast<int64_t>(block), n);
  cfh::BitReader br(words, static_cast<int64_t>(block_off[b]));
  for (int64_t i = first; i < last; ++i) W[i] = static_cast<float>((br.decode(lut, maxlen) & 0xff) - zero) * scale;
}

// one lane per output column m, the reference's k-outer / b-inner fp32 order; y accumulated in registers
template <int BMAX>
__global__ void __launch_bounds__(256) dense_gemm_kernel(const float *__restrict__ W, const float *__restrict__ x,
                                                         float *__restrict__ y, int B, int M, int K) {
  const int m = blockIdx.x * 256 + threadIdx.x;
  if (m >= M) return;
  for (int b0 = 0; b0 < B; b0 += BMAX) {
    const int nb = min(BMAX, B - b0);
    float acc[BMAX];
#pragma unroll
    for (int i = 0; i < BMAX; ++i) acc[i] = 0.f;
    const float *wr = W + static_cast<int64_t>(m) * K;
    for (int k = 0; k < K; ++k) {
      const float w = wr[k];
#pragma unroll
      for (int i = 0; i < BMAX; ++i)
        if (i < nb) acc[i] += x[static_cast<int64_t>(b0 + i) * K + k] * w;
    }
    for (int i = 0; i < nb; ++i) y[static_cast<int64_t>(b0 + i) * M + m] = acc[i];
  }
}

}  // namespace

extern "C" cf_status cf_fused_matmul_async(const uint32_t *words, const int32_t *block_off, const int32_t *lut,
                                           int maxlen, int block, const float *x, float *y, int B, int M, int K,
                                           float scale, int zero, void *stream) {
  if (!words || !block_off || !lut || !x || !y) return CF_ERR_INVALID_ARGUMENT;
  if (M == 0) return CF_OK;
  if (B < 0 || M < 0 || K < 0 || block <= 0 || maxlen <= 0) return CF_ERR_INVALID_ARGUMENT;
  if (maxlen > 24) return CF_ERR_UNSUPPORTED;
  if (B == 0) return CF_OK;
  Args a{};
  a.words = words;
  a.block_off = block_off;
  a.lut = lut;
  a.maxlen = maxlen;
  a.block = block;
  a.x = x;
  a.y = y;
  a.B = B;
  a.M = M;
  a.K = K;
  a.scale = scale;
  a.zero = zero;
  fused_matmul_kernel<<<cfd::grid_for(M, kTM), kThreads, 0, cfd::as_stream(stream)>>>(a);
  return cfd::launch_status();
}

extern "C" cf_status cf_dense_matmul_async(const uint32_t *words, const int32_t *block_off, const int32_t *lut,
                                           int maxlen, int block, const float *x, float *W, float *y, int B, int M,
                                           int K, float scale, int zero, void *stream) {
  if (!words || !block_off || !lut || !x || !W || !y) return CF_ERR_INVALID_ARGUMENT;
  if (M == 0) return CF_OK;
  if (B < 0 || M < 0 || K < 0 || block <= 0 || maxlen <= 0) return CF_ERR_INVALID_ARGUMENT;
  if (maxlen > 24) return CF_ERR_UNSUPPORTED;
  const hipStream_t s = cfd::as_stream(stream);
  const int64_t n = static_cast<int64_t>(M) * K;
  if (n > 0)
    decode_dense_kernel<<<cfd::grid_for(static_cast<size_t>((n + block - 1) / block), 256), 256, 0, s>>>(
        words, block_off, lut, maxlen, block, n, scale, zero, W);
  if (B > 0) dense_gemm_kernel<16><<<cfd::grid_for(M, 256), 256, 0, s>>>(W, x, y, B, M, K);
  return cfd::launch_status();
}
