// nibble_mfma.hip — attention over sealed int4 nibble pages on the matrix cores (head_dim 128).
//
// Same contract as nib_attn_kernel (nibble_kv.hip) for the sealed pages of an item: key position p counts for query
// position P when p <= P and, with a window w > 0, p + w > P; softmax with a running maximum in log2 units; the
// split partials (m, l, unnormalised acc) go to the same workspace rows, and the same merge kernel finishes them.
// The item's active fp32 page stays with the VALU kernel.
//
// Layout. A workgroup = 4 wavefronts serves one (item, query token, KV head, group of 4 query heads, context
// split); each wavefront walks 64-slot tiles = four 16-token chunks of pages (chunk G of a tile on lanes
// 16G..16G+15, a page of N tokens giving ceil(N/16) chunks).
//   staging:  global_load_lds copies a chunk's 16 K rows and 16 V rows of this KV head (64 B each) into LDS, the
//             four 16-byte pieces of row r stored in the order piece ^ (r & 3) so that the lanes' row reads below
//             hit different banks; the next tile's copies and its lanes' scales are in flight while the current
//             tile is computed.
//   K phase:  lane = token. Each 4-dim quad of the lane's row becomes the f16 B operand of v_mfma_f32_4x4x4f16
//             (nibble - 8, exact: 0x6400 | nibble is 1024 + nibble in f16, then one packed f16 subtract of 1032 per
//             two values), with the 4 query heads (split into f16 hi + lo for fp32-grade scores) broadcast as the A
//             operand, accumulating one score per head in the lane. One accumulator pair per scale block of the row
//             (the page's block size is 32, 64 or a multiple of 128): score = sum over blocks of k_scale * acc.
//   softmax:  one running maximum per head for each chunk group (a 16-lane DPP row, so the maximum is four DPP
//             steps), merged across the groups once after the loop; p goes to LDS with the tokens' V scales.
//   V phase:  lane (G, t) owns dims 8t..8t+7 of chunk G's tokens: it reads word t of four rows, transposes the
//             4 x 8 nibbles with v_perm into eight f16 B operands (4 tokens x 1 dim), and the A operand is p times
//             the V scale of its 32-dim block for those 4 tokens, as f16 hi + lo.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <utility>

#include "cf_device.hpp"
#include "nibble_kv.hpp"
#include "nibble_page.hpp"

namespace cfnib {
namespace {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

constexpr int kD = 128;
constexpr int kWaves = 4;
constexpr uint32_t kRowBytes = kD / 2;                    // nibbles of one token's row of one KV head
constexpr uint32_t kChunkStride = 16 * kRowBytes + 64;   // staged 16-row chunk + a bank offset between chunks
constexpr uint32_t kTileBytes = 4 * kChunkStride;
constexpr float kOff = 1032.0f;                           // operand 1024 + nibble, value nibble - 8
constexpr float kNegInf = -__builtin_huge_valf();

__device__ inline half4_t as_half4(uint32_t lo, uint32_t hi) {
  half4_t h;
  uint32_t *w = reinterpret_cast<uint32_t *>(&h);
  w[0] = lo;
  w[1] = hi;
  return h;
}

// Two f16 lanes holding 1024 + n (the 0x6400 | n bit trick) -> n - 8, exact, in one packed f16 add.
__device__ inline uint32_t minus_1032(uint32_t x) {
  half2_t h = __builtin_bit_cast(half2_t, x);
  h = h - half2_t{static_cast<_Float16>(kOff), static_cast<_Float16>(kOff)};
  return __builtin_bit_cast(uint32_t, h);
}

// x = four nibbles n0 | n1 << 4 | n2 << 8 | n3 << 12 (x < 65536)  ->  (n0 - 8, ..., n3 - 8) as f16
__device__ inline half4_t nib_quad(uint32_t x) {
  const uint32_t lo = (((x << 12) | x) & 0x000F000Fu) | 0x64006400u;
  const uint32_t hi = (((x << 4) | (x >> 8)) & 0x000F000Fu) | 0x64006400u;
  return as_half4(minus_1032(lo), minus_1032(hi));
}

// Pointers read from the item table are generic; these casts make their loads global (vector) or constant
// (scalar) accesses, which the compiler does not have to order against the LDS DMA the way it orders FLAT loads.
#define CF_GLOBAL __attribute__((address_space(1)))
#define CF_CONST __attribute__((address_space(4)))
template <typename T>
__device__ inline const CF_GLOBAL T *gptr(const T *p) {
  return (const CF_GLOBAL T *)p;  // an address-space conversion (C-style cast)
}
template <typename T>
__device__ inline const CF_CONST T *cptr(const T *p) {
  return (const CF_CONST T *)p;
}

__device__ inline float load_q(const void *base, uint32_t type, uint64_t off) {
  const CF_GLOBAL char *p = gptr(static_cast<const char *>(base)) + off;
  if (type == CF_DEVICE_F16) return static_cast<float>(*reinterpret_cast<const CF_GLOBAL _Float16 *>(p));
  if (type == CF_DEVICE_BF16) return __uint_as_float(uint32_t(*reinterpret_cast<const CF_GLOBAL uint16_t *>(p)) << 16);
  return *reinterpret_cast<const CF_GLOBAL float *>(p);
}

template <int CTRL>
__device__ inline float dpp_mov(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xf, 0xf, false));
}

// Maximum over the 16 lanes of a DPP row; every lane of the row receives it.
__device__ inline float row_max(float x) {
  x = fmaxf(x, dpp_mov<0xb1>(x));   // quad_perm [1,0,3,2]
  x = fmaxf(x, dpp_mov<0x4e>(x));   // quad_perm [2,3,0,1]
  x = fmaxf(x, dpp_mov<0x141>(x));  // row_half_mirror
  x = fmaxf(x, dpp_mov<0x140>(x));  // row_mirror
  return x;
}

__device__ inline void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// MODE 1 / 2 / 4: sealed pages with that many scale blocks per row (block size known for the request).
// MODE kMfmaContract: a batched-items request (two's-complement nibbles, per-row scale blocks, no causal bound and
// an inclusive window): each page's own block size (a multiple of 32) gives one scale per 32-dim quarter of a row,
// and pages that mfma_page_ok refuses are left to the VALU kernel.
template <int MODE>
__global__ __launch_bounds__(256) void nib_mfma_kernel(const AttnItem *__restrict__ items, AttnShape sh,
                                                       uint32_t qchunks, float *__restrict__ ws) {
  constexpr bool PG = MODE == static_cast<int>(kMfmaContract);
  constexpr int NB = PG ? 4 : MODE;
  constexpr uint32_t sx = PG ? 0x88888888u : 0u;  // two's-complement nibbles -> offset-8 (n ^ 8 = n + 8 mod 16)
  __shared__ __attribute__((aligned(16))) uint8_t s_kv[kWaves][2][2][kTileBytes];  // [wave][buffer][K, V]
  __shared__ __attribute__((aligned(16))) float s_p[kWaves][4][64];                // p per [head][slot]
  __shared__ float s_vs[kWaves][64][NB];                                           // V scales per slot
  const AttnItem &it = items[blockIdx.z];
  if (it.mfma_nb != static_cast<uint32_t>(MODE)) return;
  const uint32_t split = blockIdx.x;
  if (split >= it.page_splits) return;
  const uint32_t kvh = sh.kv_heads, gqa = sh.gqa;
  const uint32_t per_tok = qchunks * kvh;
  const uint32_t qt = blockIdx.y / per_tok;
  if (qt >= it.q_tokens) return;
  const uint32_t rest = blockIdx.y - qt * per_tok;
  const uint32_t h = rest / qchunks, qc = rest - h * qchunks;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int G = lane >> 4, t = lane & 15;
  const uint32_t qpos = it.q_begin + qt;
  const uint32_t window = it.window;

  // ---- queries (scaled to log2 units) as f16 hi + lo in LDS, then in registers
  _Float16(*s_q)[4][kD] = reinterpret_cast<_Float16(*)[4][kD]>(&s_kv[0][0][0][0]);
  for (int i = threadIdx.x; i < 4 * kD; i += 256) {
    const int j = i / kD, dd = i % kD;
    float q = 0.0f;
    if (qc * 4 + j < gqa)
      q = load_q(it.q, it.q_type, uint64_t(qt) * it.q_token_stride + uint64_t(h * gqa + qc * 4 + j) * it.q_head_stride +
                                       uint64_t(dd) * it.q_elem_stride);
    cfd::split_mul_f16(q, it.scale_log2, s_q[0][j][dd], s_q[1][j][dd]);
  }
  __syncthreads();
  half4_t qhi[2], qlo[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int qd = 16 * c + (lane >> 2);
    qhi[c] = *reinterpret_cast<const half4_t *>(&s_q[0][lane & 3][4 * qd]);
    qlo[c] = *reinterpret_cast<const half4_t *>(&s_q[1][lane & 3][4 * qd]);
  }
  __syncthreads();  // the query staging aliases wave 0's tile buffers

  const uint32_t cpp = (sh.page_size + 15u) / 16u;
  const uint32_t nchunks = it.page_count * cpp;
  const uint32_t ntiles = (nchunks + 3u) / 4u;
  const uint32_t tb = split * it.units_per_split;
  const uint32_t te = min(ntiles, tb + it.units_per_split);
  const cf_device_page_descriptor *pages = it.pages;

  float m_run[4], l_run[4];
  float4_t acc[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    m_run[j] = kNegInf;
    l_run[j] = 0.0f;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = float4_t{0, 0, 0, 0};

  // per-lane metadata of the tile in flight: this lane's token (row of chunk G), its visibility and scales
  bool n_ok = false;
  float n_ks[NB], n_vs[NB];
#pragma unroll
  for (int s = 0; s < NB; ++s) n_ks[s] = n_vs[s] = 0.0f;

  // Descriptor fields of a tile's four chunks, fetched one tile ahead of its copies with vector loads (they land
  // under the same vmcnt wait as the copies, and unlike scalar loads they do not hold up the LDS reads).
  struct TileDesc {
    const uint8_t *kp[4], *vp[4];
    uint32_t tc[4];
    const float *ks, *vs;  // this lane's chunk (G)
    uint32_t tb, bs;
  };
  auto fetch = [&](uint32_t tile, TileDesc &d) {
    const CF_GLOBAL cf_device_page_descriptor *gp = gptr(pages);
#pragma unroll
    for (int C = 0; C < 4; ++C) {
      const uint32_t ch = 4u * tile + C;
      d.tc[C] = 0u;
      if (ch < nchunks) {
        const uint32_t p = ch / cpp;
        d.kp[C] = gp[p].key_payload;
        d.vp[C] = gp[p].value_payload;
        d.tc[C] = gp[p].token_count;
        if constexpr (PG) {  // a refused page: no tokens here (the VALU kernel reads it)
          if (!mfma_page_ok(d.kp[C], d.vp[C], gp[p].key_scales, gp[p].value_scales, gp[p].block_size,
                            gp[p].head_dim, d.tc[C], it.mfma_cap))
            d.tc[C] = 0u;
        }
      }
    }
    const uint32_t mine = 4u * tile + G;
    if (mine < nchunks) {
      const uint32_t p = mine / cpp;
      d.ks = gp[p].key_scales;
      d.vs = gp[p].value_scales;
      d.tb = gp[p].token_begin;
      d.bs = gp[p].block_size;
    }
  };
  // copies of tile `tile` into buffer `buf`, and this lane's scales for it (the descriptors have landed)
  auto stage = [&](uint32_t tile, const TileDesc &d, int buf) {
#pragma unroll
    for (int C = 0; C < 4; ++C) {
      const uint32_t ch = 4u * tile + C;
      const uint32_t off = (ch % cpp) * 16u;
      const uint32_t tc = __builtin_amdgcn_readfirstlane(d.tc[C]);
      if (ch >= nchunks || off >= tc) continue;  // past the split / a partial page's empty chunk: masked slots
      const uint32_t r = static_cast<uint32_t>(lane) >> 2, piece = (lane & 3) ^ (r & 3);
      const uint32_t row = min(off + r, tc - 1u);  // slots past the page's tokens re-read its last row
      const uint64_t goff = (uint64_t(row) * kvh + h) * kRowBytes + 16u * piece;
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const CF_GLOBAL uint32_t *>(gptr(d.kp[C]) + goff),
                                       (__attribute__((address_space(3))) void *)(&s_kv[wave][buf][0][C * kChunkStride]),
                                       16, 0, 0);
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const CF_GLOBAL uint32_t *>(gptr(d.vp[C]) + goff),
                                       (__attribute__((address_space(3))) void *)(&s_kv[wave][buf][1][C * kChunkStride]),
                                       16, 0, 0);
    }
    n_ok = false;
    const uint32_t mine = 4u * tile + G;
    const uint32_t my_tc = G == 0 ? d.tc[0] : G == 1 ? d.tc[1] : G == 2 ? d.tc[2] : d.tc[3];
    const uint32_t off = (mine % cpp) * 16u;
    if (mine < nchunks && off < my_tc) {
      const uint32_t tok = off + static_cast<uint32_t>(t);
      const uint32_t pos = d.tb + tok;
      const uint32_t row = min(tok, my_tc - 1u) * kvh + h;  // token-head row of the page
      if constexpr (PG) {
        n_ok = tok < my_tc && (window == 0u || uint64_t(pos) + window >= qpos);
        // ceil(128 / block_size) blocks per row; quarter s (dims 32 s .. 32 s + 31) lies in block 32 s / block_size
        const uint32_t bs = d.bs, rb = row * ((128u + bs - 1u) / bs);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const uint32_t bi = rb + (32u * s) / bs;
          n_ks[s] = gptr(d.ks)[bi];
          n_vs[s] = gptr(d.vs)[bi];
        }
      } else {
        n_ok = tok < my_tc && pos <= qpos && (window == 0u || uint64_t(pos) + window > qpos);
        // first scale of the row: block = row * 128 / block_size (block_size 32 / 64 / a multiple of 128)
        const uint32_t bi = NB == 4 ? row * 4u : NB == 2 ? row * 2u : row / (d.bs / 128u);
#pragma unroll
        for (int s = 0; s < NB; ++s) {
          n_ks[s] = gptr(d.ks)[bi + s];
          n_vs[s] = gptr(d.vs)[bi + s];
        }
      }
    }
  };

  int cur = 0;
  uint32_t tile = tb + wave;
  TileDesc dnext;
  if (tile < te) {
    fetch(tile, dnext);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    stage(tile, dnext, 0);
    if (tile + kWaves < te) fetch(tile + kWaves, dnext);
  }
  for (; tile < te; tile += kWaves) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this tile's rows and scales, the next tile's descriptors
    wave_sync_lds();
    const bool tok_ok = n_ok;
    float ks[NB], vs[NB];
#pragma unroll
    for (int s = 0; s < NB; ++s) {
      ks[s] = n_ks[s];
      vs[s] = n_vs[s];
    }
    if (tile + kWaves < te) {
      stage(tile + kWaves, dnext, cur ^ 1);
      if (tile + 2 * kWaves < te) fetch(tile + 2 * kWaves, dnext);
    }

    // ---- K: one score per head for this lane's token
    // four independent accumulator chains (x hi / lo): chain c holds quads of scale block c / (4 / NB), and the
    // quad order below makes consecutive MFMAs hit different chains
    constexpr int CPS = 4 / NB;  // chains per scale block
    float4_t sa[4], sb[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) sa[c] = sb[c] = float4_t{0, 0, 0, 0};
    {
      const uint8_t *kb = &s_kv[wave][cur][0][G * kChunkStride + t * kRowBytes];
      uint4 pc[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) pc[k] = *reinterpret_cast<const uint4 *>(kb + 16 * (k ^ (t & 3)));
      const uint32_t w16[16] = {pc[0].x ^ sx, pc[0].y ^ sx, pc[0].z ^ sx, pc[0].w ^ sx, pc[1].x ^ sx, pc[1].y ^ sx,
                                pc[1].z ^ sx, pc[1].w ^ sx, pc[2].x ^ sx, pc[2].y ^ sx, pc[2].z ^ sx, pc[2].w ^ sx,
                                pc[3].x ^ sx, pc[3].y ^ sx, pc[3].z ^ sx, pc[3].w ^ sx};
      [&]<int... I>(std::integer_sequence<int, I...>) {
        (
            [&] {
              constexpr int c = I % 4;                         // chain
              constexpr int blk = c / CPS, sub = c % CPS;      // scale block, position among its chains
              constexpr int q = blk * (32 / NB) + CPS * (I / 4) + sub;  // quad = dims 4q..4q+3
              const uint32_t w = w16[q / 2];
              const half4_t b = nib_quad((q & 1) ? (w >> 16) : (w & 0xFFFFu));
              sa[c] = __builtin_amdgcn_mfma_f32_4x4x4f16(qhi[q / 16], b, sa[c], 4, q % 16, 0);
              sb[c] = __builtin_amdgcn_mfma_f32_4x4x4f16(qlo[q / 16], b, sb[c], 4, q % 16, 0);
            }(),
            ...);
      }(std::make_integer_sequence<int, 32>{});
    }
    // softmax: one running maximum per head for each 16-lane chunk group (a DPP row), merged after the loop
    float sc[4], mx[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v = 0.0f;
#pragma unroll
      for (int c = 0; c < 4; ++c) v = fmaf(ks[c / CPS], sa[c][j] + sb[c][j], v);
      sc[j] = tok_ok ? v : kNegInf;
      mx[j] = row_max(sc[j]);
    }
    // raise the running maxima (and rescale the accumulators) only when some lane's maximum grew
    bool grow = false;
#pragma unroll
    for (int j = 0; j < 4; ++j) grow |= mx[j] > m_run[j];
    if (__ballot(grow) != 0) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float mn = fmaxf(m_run[j], mx[j]);
        const float alpha = (m_run[j] == kNegInf) ? 0.0f : __builtin_amdgcn_exp2f(m_run[j] - mn);
        l_run[j] *= alpha;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e][j] *= alpha;
        m_run[j] = mn;
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float p = tok_ok ? __builtin_amdgcn_exp2f(sc[j] - m_run[j]) : 0.0f;
      l_run[j] += p;
      s_p[wave][j][lane] = p;
    }
#pragma unroll
    for (int s = 0; s < NB; ++s) s_vs[wave][lane][s] = vs[s];
    wave_sync_lds();

    // ---- V: out[head][8t + e] += sum over 4 tokens of p * v_scale * (nibble - 8)
    {
      const uint8_t *vb = &s_kv[wave][cur][1][G * kChunkStride];
      const int vset = NB == 4 ? (t >> 2) : NB == 2 ? (t >> 3) : 0;
#pragma unroll
      for (int tq = 0; tq < 4; ++tq) {
        const int slot = 16 * G + 4 * tq;
        const float4 pp = *reinterpret_cast<const float4 *>(&s_p[wave][lane & 3][slot]);
        const float pk[4] = {pp.x, pp.y, pp.z, pp.w};
        half4_t a, al;  // p * v_scale as f16 hi + lo (fp32-grade weights, like the query operand)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          _Float16 h, l;
          cfd::split_mul_f16(pk[k], s_vs[wave][slot + k][vset], h, l);
          a[k] = h;
          al[k] = l;
        }
        uint32_t wk[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
          wk[k] = *reinterpret_cast<const uint32_t *>(vb + (4 * tq + k) * kRowBytes + 16 * ((t >> 2) ^ k) + 4 * (t & 3)) ^
                  sx;
        half4_t bv[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {  // byte j of the four words: dims 8t + 2j (low nibbles), 8t + 2j + 1 (high)
          const uint32_t sel = uint32_t(j) | 0x0c00u | (uint32_t(4 + j) << 16) | 0x0c000000u;
          const uint32_t x01 = __builtin_amdgcn_perm(wk[1], wk[0], sel);  // [w0.bj, 0, w1.bj, 0]
          const uint32_t x23 = __builtin_amdgcn_perm(wk[3], wk[2], sel);
          bv[2 * j] = as_half4(minus_1032((x01 & 0x000F000Fu) | 0x64006400u),
                               minus_1032((x23 & 0x000F000Fu) | 0x64006400u));
          bv[2 * j + 1] = as_half4(minus_1032(((x01 >> 4) & 0x000F000Fu) | 0x64006400u),
                                   minus_1032(((x23 >> 4) & 0x000F000Fu) | 0x64006400u));
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = __builtin_amdgcn_mfma_f32_4x4x4f16(a, bv[e], acc[e], 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = __builtin_amdgcn_mfma_f32_4x4x4f16(al, bv[e], acc[e], 0, 0, 0);
      }
    }
    wave_sync_lds();
    cur ^= 1;
  }

  // ---- wavefront partial: bring the four chunk groups to a common maximum, then sum them (l over all lanes)
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float mw = fmaxf(m_run[j], __shfl_xor(m_run[j], 16));
    mw = fmaxf(mw, __shfl_xor(mw, 32));
    const float f = (m_run[j] == kNegInf) ? 0.0f : __builtin_amdgcn_exp2f(m_run[j] - mw);
    l_run[j] *= f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e][j] *= f;
    m_run[j] = mw;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v = acc[e][j];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      acc[e][j] = v;
    }
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) l_run[j] += __shfl_xor(l_run[j], o);
  __syncthreads();  // every wave is done with its tile buffers: reuse them for the partials
  float(*red)[4][kD + 2] = reinterpret_cast<float(*)[4][kD + 2]>(&s_kv[0][0][0][0]);
  if (lane < 16) {
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int j = 0; j < 4; ++j) red[wave][j][8 * t + e] = acc[e][j];
  }
  if (lane < 4) {
    red[wave][lane][kD] = m_run[lane];
    red[wave][lane][kD + 1] = l_run[lane];
  }
  __syncthreads();
  const uint32_t stride = kD + 4u;
  float *base = ws + it.ws_offset + (uint64_t(split) * it.q_tokens + qt) * sh.q_heads * stride;
  for (int i = threadIdx.x; i < 4 * kD; i += 256) {
    const int j = i / kD, dd = i % kD;
    if (qc * 4 + j >= gqa) continue;
    float m = kNegInf;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) m = fmaxf(m, red[w][j][kD]);
    float l = 0.0f, o = 0.0f;
    if (m != kNegInf)
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float mw = red[w][j][kD];
        if (mw == kNegInf) continue;
        const float f = __builtin_amdgcn_exp2f(mw - m);
        l = fmaf(red[w][j][kD + 1], f, l);
        o = fmaf(red[w][j][dd], f, o);
      }
    float *row = base + uint64_t(h * gqa + qc * 4 + j) * stride;
    row[dd] = o;
    if (dd == 0) {
      row[kD] = m;
      row[kD + 1] = l;
    }
  }
}

}  // namespace

hipError_t launch_nib_mfma(uint32_t nb, const AttnItem *items, uint32_t nitems, uint32_t max_page_splits,
                           uint32_t max_qtok, const AttnShape &sh, float *ws, hipStream_t stream) {
  if (sh.head_dim != kD || max_page_splits == 0) return hipSuccess;
  const uint32_t qchunks = (sh.gqa + 3u) / 4u;
  const uint64_t ydim = uint64_t(max_qtok) * qchunks * sh.kv_heads;
  if (ydim > 65535u) return hipErrorInvalidValue;
  const dim3 grid(max_page_splits, static_cast<uint32_t>(ydim), nitems);
  switch (nb) {
    case 1: nib_mfma_kernel<1><<<grid, 256, 0, stream>>>(items, sh, qchunks, ws); break;
    case 2: nib_mfma_kernel<2><<<grid, 256, 0, stream>>>(items, sh, qchunks, ws); break;
    case kMfmaContract: nib_mfma_kernel<kMfmaContract><<<grid, 256, 0, stream>>>(items, sh, qchunks, ws); break;
    default: nib_mfma_kernel<4><<<grid, 256, 0, stream>>>(items, sh, qchunks, ws); break;
  }
  return hipPeekAtLastError();
}

}  // namespace cfnib
