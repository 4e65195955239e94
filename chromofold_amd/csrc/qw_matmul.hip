// qw_matmul.hip — decode-in-matmul over the band-table int4 Huffman format (CF_QW_CODEC_HUFFMAN,
// include/chromofold/chromofold_qw.h; the rANS codec's kernel is in qw_rans.hip) on gfx950:
// y[b, m] = sum_k x[b, k] * (sym[m, k] - zero) * scale[m, k / 64], the weight matrix held only in its coded form.
//
// One 1024-thread workgroup (16 waves) owns one band of 16 rows (so one code table) and walks K in chunks of 4096
// columns; lane (wave r, lane s) owns segment s of row r within the chunk:
//   stage    each wave copies its row's code words for the chunk into LDS; every load of the chunk is issued as
//            straight-line code before the first is waited for (rows whose codes do not fit the per-row budget
//            are read from global memory instead: same results, slower);
//   table    the band's 16 code lengths become a 4096-entry table over a 12-bit lookahead that yields up to three
//            symbols per lookup, built in two LDS passes while the loads are in flight;
//   decode   each lane streams its segment through a 64-bit register window (two 32-bit halves, the next word
//            prefetched one refill ahead), writing u8 symbols into a bank-staggered LDS tile;
//   MFMA     v_mfma_f32_16x16x16_bf16 with A = x (16 batch rows per tile, up to 4 tiles per launch) and B = the
//            decoded symbols minus `zero` (exact small integers in bf16); each wave owns 4 whole segments, so the
//            segment's scale multiplies its 4-step partial once;
//   reduce   the 16 waves' partial tiles are summed through LDS in a fixed order (deterministic) and y is written
//            once — no prior zeroing, no read-modify-write.
// Batches above 64 rows run as several launches of up to 4 tiles each.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "cf_device.hpp"
#include "chromofold/chromofold_qw.h"
#include "qw_internal.hpp"

namespace {

typedef short bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kRows = CF_QW_BAND_ROWS;  // rows per workgroup = one band
constexpr int kKC = 64 * CF_QW_SEG_COLS;  // columns per chunk: one segment per lane of a row's wave
constexpr int kSegB = 68;                 // bytes per segment in the symbol tile (odd word stride: no bank pile-up)
constexpr int kLdB = 64 * kSegB + 16;     // bytes per row of the tile
constexpr int kLook = CF_QW_MAX_CODE_LENGTH;  // lookahead bits (12)
constexpr int kRowWords = 640;            // staged code words per row (5 bits per symbol over a full chunk)
constexpr int kSlack = 5;                 // words the reader may touch past the word holding a segment's last bit
constexpr int kMaxTiles = 4;

static_assert(kRows == 16 && kWaves == kRows, "one wave per band row");
static_assert(kLook == 12, "the table covers a 12-bit lookahead");

struct QwArgs {
  const uint32_t *words;
  uint64_t word_count;
  const uint32_t *seg_off;
  const uint8_t *code_len;
  const float *scales;
  const uint16_t *x;
  float *y;
  int B, M, K, zero, bt0;  // bt0: first 16-row batch tile of this launch
};

__device__ __forceinline__ short bf16_of_int(int v) {  // |v| <= 15: exact
  return static_cast<short>(__float_as_uint(static_cast<float>(v)) >> 16);
}

// Barrier for LDS traffic only: waits for this wave's LDS operations, not for its global loads in flight (a
// __syncthreads also waits for those).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt left at their maxima
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// The band table. Canonical codes are assigned in (length, symbol) order, so the symbols' 12-bit left-justified
// ranges are consecutive in that order: the code under a lookahead v is the last present symbol (in canonical
// order) whose range starts at or below v. Pass 1 writes that single-symbol table (sym | len << 8) into `tmp`;
// pass 2 chains up to three consecutive codes that fit in the lookahead:
//   entry = s1 | s2 << 8 | s3 << 16 | bits << 24 | count << 28.
// `lens` holds the band's 16 code lengths, one byte each (symbol u in byte u % 4 of lens[u / 4]).
__device__ void build_table(const uint4 lens, uint32_t *__restrict__ lut, uint32_t *__restrict__ tmp,
                            uint32_t *__restrict__ s_meta) {
  const int t = threadIdx.x;
  uint32_t *s_start = s_meta;      // [16] range starts in canonical order (4096 past the present symbols)
  uint32_t *s_code = s_meta + 16;  // [16] sym | len << 8 in canonical order
  if (t < 16) {
    uint32_t lw[4] = {lens.x, lens.y, lens.z, lens.w};
    // pin the first use here: hoisted out of the caller's chunk loop it would wait for the load before the
    // chunk's other loads are issued
    asm volatile("" : "+v"(lw[0]), "+v"(lw[1]), "+v"(lw[2]), "+v"(lw[3]));
    const int L = static_cast<int>((lw[t >> 2] >> (8 * (t & 3))) & 0xFFu);
    uint32_t code = 0;
    int rank = 0, present = 0, absent_before = 0;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int Lu = static_cast<int>((lw[u >> 2] >> (8 * (u & 3))) & 0xFFu);
      present += Lu != 0;
      absent_before += (Lu == 0 && u < t);
      if (Lu != 0 && (Lu < L || (Lu == L && u < t))) {
        code += 1u << (kLook - Lu);  // left-justified: the earlier codes' range sizes
        ++rank;
      }
    }
    if (L > 0) {
      s_start[rank] = code;
      s_code[rank] = static_cast<uint32_t>(t | (L << 8));
    } else {  // absent symbols fill the tail slots [present, 16) with starts no lookahead reaches
      s_start[present + absent_before] = 1u << kLook;
      s_code[present + absent_before] = 0;
    }
  }
  lds_barrier();
  for (int e = t; e < (1 << kLook); e += kThreads) {
    int idx = -1;  // the first canonical range starts at 0, so idx >= 0
#pragma unroll
    for (int u = 0; u < 16; ++u) idx += s_start[u] <= static_cast<uint32_t>(e);
    tmp[e] = s_code[idx];
  }
  lds_barrier();
  constexpr uint32_t kMask = (1u << kLook) - 1;
  for (int e = t; e < (1 << kLook); e += kThreads) {
    const uint32_t f1 = tmp[e], l1 = f1 >> 8;
    const uint32_t r1 = (static_cast<uint32_t>(e) << l1) & kMask;
    const uint32_t f2 = tmp[r1], l2 = f2 >> 8;
    const uint32_t f3 = tmp[(r1 << l2) & kMask], l3 = f3 >> 8;
    const bool two = l1 + l2 <= kLook, three = two && l1 + l2 + l3 <= kLook;
    const uint32_t bits = l1 + (two ? l2 : 0u) + (three ? l3 : 0u);
    const uint32_t count = 1u + two + three;
    lut[e] = (f1 & 0xFFu) | ((f2 & 0xFFu) << 8) | ((f3 & 0xFFu) << 16) | (bits << 24) | (count << 28);
  }
}

// Decode n symbols of one segment from bit `pos` of `src` (words indexable up to the row's staged end) into dst.
// The window is {hi, lo}, MSB-aligned, nb valid bits (>= 32 before every lookup, so the 12-bit lookahead is in hi);
// `nw` is the next word, fetched one refill ahead. Each lookup writes 3 bytes (up to 3 symbols; unused slots are
// overwritten by later lookups or the caller's padding), so dst needs 2 bytes of room past symbol n.
// Reads stay within kSlack words past the word that holds the segment's last bit.
template <typename Src>
__device__ __forceinline__ void decode_segment(const Src &src, uint32_t pos, int n, const uint32_t *__restrict__ lut,
                                               uint8_t *__restrict__ dst) {
  const int i = static_cast<int>(pos >> 5);
  const uint32_t b = pos & 31;
  const uint32_t w0 = src(i), w1 = src(i + 1);
  uint32_t hi = static_cast<uint32_t>(((static_cast<uint64_t>(w0) << 32) | w1) >> (32 - b));
  uint32_t lo = w1 << b;
  int nb = 64 - static_cast<int>(b);
  uint32_t nw = src(i + 2);
  int next = i + 3;
  uint8_t *end = dst + n;
  while (dst < end) {
    const uint32_t e = lut[hi >> (32 - kLook)];
    // three byte stores: LDS stores of 2 or 4 bytes at addresses they are not aligned to are far slower
    dst[0] = static_cast<uint8_t>(e);
    dst[1] = static_cast<uint8_t>(e >> 8);
    dst[2] = static_cast<uint8_t>(e >> 16);
    const uint32_t len = (e >> 24) & 15u;  // 1..12
    hi = __builtin_amdgcn_alignbit(hi, lo, 32u - len);
    lo <<= len;
    nb -= static_cast<int>(len);
    dst += e >> 28;
    if (nb < 32) {  // every valid bit is in hi and lo is zero: append the next word
      hi |= nw >> nb;
      lo = nw << (32 - nb);
      nb += 32;
      nw = src(next++);
    }
  }
}

// x[b, k..k+7] as 4 words (two bf16 each): the A operands of two MFMA k-steps. FAST: K is a multiple of 64 and rows
// past the batch read the last row (their outputs are never written); otherwise element-wise, zero past K or B.
template <bool FAST>
__device__ __forceinline__ uint4 x_frag8(const uint16_t *__restrict__ x, int b, int B, int k, int K) {
  if constexpr (FAST) {
    return *reinterpret_cast<const uint4 *>(x + static_cast<int64_t>(min(b, B - 1)) * K + k);
  } else {
    uint32_t v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (b < B && k + e < K) ? x[static_cast<int64_t>(b) * K + k + e] : 0u;
    return make_uint4(v[0] | (v[1] << 16), v[2] | (v[3] << 16), v[4] | (v[5] << 16), v[6] | (v[7] << 16));
  }
}

template <int NT, bool FAST, int XR>
__global__ void __launch_bounds__(kThreads) qw_matmul_kernel(QwArgs a) {
  static_assert(XR == 0 || (XR == 1 && NT == 1 && FAST), "a staged x row: one batch row, whole segments");
  // XR = 1 (a batch of one row): the chunk's x columns staged once per workgroup (8 bytes per thread) instead of
  // every lane loading its 16-byte fragments from global memory, where the 16 row lanes of a lane group would all
  // fetch the same row
  __shared__ __attribute__((aligned(16))) uint16_t s_x[XR ? kKC : 8];
  static_assert(kKC == 4 * kThreads, "one 8-byte x load per thread covers a chunk");
  // one LDS block so that the table sits at address 0 (its lookups need no base add)
  constexpr int kLutB = (1 << kLook) * 4, kTileB = kRows * kLdB, kCodeB = kRows * kRowWords * 4;
  __shared__ __attribute__((aligned(16))) uint8_t smem[kLutB + kTileB + kCodeB + 32 * 4];
  uint32_t *s_lut = reinterpret_cast<uint32_t *>(smem);
  uint8_t *s_tile = smem + kLutB;  // symbols; the table's first pass and the final reduction reuse it
  auto s_code = reinterpret_cast<uint32_t (*)[kRowWords]>(smem + kLutB + kTileB);
  uint32_t *s_meta = reinterpret_cast<uint32_t *>(smem + kLutB + kTileB + kCodeB);
  static_assert(kTileB % 16 == 0, "staged words stay 16-byte aligned");
  static_assert(kTileB >= kWaves * NT * 256 * 4, "reduction fits the tile");
  static_assert(kTileB >= (1 << kLook) * 4, "table pass 1 fits the tile");
  static_assert(kRowWords % 64 == 0, "staging covers kRowWords in rows of 64 words");
  constexpr int kStageWords = kRowWords / 64;  // staged words per lane

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int m0 = blockIdx.x * kRows;
  const int M = a.M, K = a.K, B = a.B;
  const int nseg = (K + 63) / 64;
  const uint64_t total_segs = static_cast<uint64_t>(M) * nseg;
  const int zc = a.zero;
  const int row = m0 + wave;  // the wave's row for staging and decoding
  const int bn = lane & 15, bk = 4 * (lane >> 4);
  const int mrow = m0 + bn;  // the lane's output row in the MFMA phase

  f32x4_t acc[NT];
#pragma unroll
  for (int i = 0; i < NT; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // the band's code lengths: one 16-byte load (cf_qw_validate requires a 16-byte aligned table), issued first and
  // first used by the table build, after every other load of the chunk is in flight
  // (a vector load: a scalar one would be waited for at once, before the loads below are issued)
  uint32_t vzero;
  asm volatile("v_mov_b32 %0, 0" : "=v"(vzero));
  const uint4 lens = *reinterpret_cast<const uint4 *>(a.code_len + static_cast<size_t>(m0 / kRows) * 16 + vzero);
  bool table_done = false;
  for (int kc0 = 0; kc0 < K; kc0 += kKC) {
    const int kc1 = min(K, kc0 + kKC);
    const int seg0 = kc0 / 64, nsc = (kc1 - kc0 + 63) / 64;
    // ---- issue this chunk's global loads as straight-line code (clamped addresses, results selected) so that
    // none waits for another: the code range, the lane's segment start, the staged words, scales, first x
    uint32_t base_word, pos;
    uint64_t need = ~0ull;
    {
      const uint64_t first = static_cast<uint64_t>(min(row, M - 1)) * nseg + seg0;
      const uint64_t last = first + nsc;  // the segment after the chunk's last
      const uint32_t b0 = a.seg_off[first];
      const uint32_t b1 = a.seg_off[min(last, total_segs - 1)];
      pos = a.seg_off[first + min(lane, nsc - 1)];
      const uint64_t bit1 = last < total_segs ? static_cast<uint64_t>(b1) : a.word_count * 32;
      base_word = (b0 >> 5) & ~3u;
      if (row < M) need = (bit1 >> 5) + kSlack + 1 - base_word;
    }
    const bool staged = need <= static_cast<uint64_t>(kRowWords);  // wave-uniform
    // staged word 64 r + lane: every load instruction reads 64 consecutive words; words past the stream read 0
    uint32_t stage[kStageWords];
#pragma unroll
    for (int r = 0; r < kStageWords; ++r) {
      const uint64_t g = static_cast<uint64_t>(base_word) + 64u * r + lane;
      const uint32_t v = a.words[min(g, a.word_count - 1)];
      stage[r] = g < a.word_count ? v : 0u;
    }
    // scales of the lane's output row for the wave's 4 segments (clamped: a row past M has all-zero operands in the
    // tile, and a segment past the chunk is never used, so neither needs a select that would wait for the load)
    float sc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      sc[j] = a.scales[static_cast<uint64_t>(min(mrow, M - 1)) * nseg + seg0 + min(wave + 16 * j, nsc - 1)];
    // x fragments of segment j in buffer j % XB: with one tile the first segment's load runs during the decode and
    // the next segment's during the current one's MFMAs; with 2-4 tiles (register budget) each segment loads just
    // before its MFMAs
    constexpr int XB = NT == 1 ? 2 : 1;
    // Within each 32-column half p of a segment, MFMA k-step 2p + h gives lane group g = lane >> 4 the columns
    // 32p + 8g + 4h .. +3 (for A and B alike, so the sum is unchanged): a lane's x for both steps is one 16-byte load.
    uint4 xf[XB][2][NT];
    auto load_x = [&](int j, uint4 (&f)[2][NT]) {
      const int sg = wave + 16 * j;
      if (sg >= nsc) return;
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int i = 0; i < NT; ++i) {
          if constexpr (XR)
            f[p][i] = *reinterpret_cast<const uint4 *>(s_x + 64 * sg + 32 * p + 2 * bk);
          else
            f[p][i] = x_frag8<FAST>(a.x, (a.bt0 + i) * 16 + (lane & 15), B, kc0 + 64 * sg + 32 * p + 2 * bk, K);
        }
    };
    uint2 xs = make_uint2(0u, 0u);
    if constexpr (XR)  // columns kc0 + 4 t .. + 3 of row 0 (clamped inside the matrix: K is a multiple of 64)
      xs = *reinterpret_cast<const uint2 *>(a.x + min(kc0 + 4 * t, K - 4));
    else if constexpr (XB == 2)
      load_x(0, xf[0]);  // in flight during the table build and the decode
    // ---- the band's table (first chunk only; LDS work while the loads above are in flight)
    if (!table_done) {
      build_table(lens, s_lut, reinterpret_cast<uint32_t *>(s_tile), s_meta);
      table_done = true;
    }
    if (staged) {
#pragma unroll
      for (int r = 0; r < kStageWords; ++r) s_code[wave][64 * r + lane] = stage[r];
    }
    if constexpr (XR) *reinterpret_cast<uint2 *>(s_x + 4 * t) = xs;
    __syncthreads();  // staged words and the table visible; table pass 1 is done with the tile
    // ---- decode: lane = segment of the wave's row
    {
      uint8_t *dst = s_tile + wave * kLdB + lane * kSegB;
      const int k0 = kc0 + 64 * lane;
      const int n = (row < M && lane < nsc) ? min(64, kc1 - k0) : 0;
      if (n > 0) {
        const uint32_t rel = pos - (base_word << 5);
        if (staged) {
          const uint32_t *w = s_code[wave];
          decode_segment([w](int j) { return w[j]; }, rel, n, s_lut, dst);
        } else {
          const uint32_t *w = a.words + base_word;
          const int64_t lim = static_cast<int64_t>(a.word_count) - base_word;
          decode_segment([w, lim](int j) { return j < lim ? w[j] : 0u; }, rel, n, s_lut, dst);
        }
      }
      // columns past the segment's symbols contribute (zero - zero) = 0
      for (int j = n; j < 64; ++j) dst[j] = static_cast<uint8_t>(zc);
    }
    __syncthreads();
    if constexpr (XR) load_x(0, xf[0]);
    // ---- MFMA: the wave owns segments wave, wave + 16, wave + 32, wave + 48 of the chunk; segment j + 1's x
    // fragments load while segment j's MFMAs run
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int sg = wave + 16 * j;
      if (sg >= nsc) break;  // wave-uniform
      if constexpr (XB == 2) {
        if (j + 1 < 4) load_x(j + 1, xf[(j + 1) % XB]);
      } else {
        load_x(j, xf[0]);
      }
      f32x4_t part[NT];
#pragma unroll
      for (int i = 0; i < NT; ++i) part[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const int p = st >> 1, h = st & 1;
        const uint32_t q4 =
            *reinterpret_cast<const uint32_t *>(s_tile + bn * kLdB + sg * kSegB + 32 * p + 2 * bk + 4 * h);
        bf16x4_t bfrag;
        bfrag[0] = bf16_of_int(static_cast<int>(q4 & 0xffu) - zc);
        bfrag[1] = bf16_of_int(static_cast<int>((q4 >> 8) & 0xffu) - zc);
        bfrag[2] = bf16_of_int(static_cast<int>((q4 >> 16) & 0xffu) - zc);
        bfrag[3] = bf16_of_int(static_cast<int>(q4 >> 24) - zc);
#pragma unroll
        for (int i = 0; i < NT; ++i) {
          const uint4 v4 = xf[j % XB][p][i];
          const uint32_t w0 = h ? v4.z : v4.x, w1 = h ? v4.w : v4.y;
          bf16x4_t afrag;
          afrag[0] = static_cast<short>(w0 & 0xFFFFu);
          afrag[1] = static_cast<short>(w0 >> 16);
          afrag[2] = static_cast<short>(w1 & 0xFFFFu);
          afrag[3] = static_cast<short>(w1 >> 16);
          part[i] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(afrag, bfrag, part[i], 0, 0, 0);
        }
      }
#pragma unroll
      for (int i = 0; i < NT; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[i][e] += sc[j] * part[i][e];  // lane's output column is row bn
    }
    __syncthreads();  // tile and staged words free for the next chunk
  }

  // ---- fixed-order cross-wave reduction, one write of y per (b, m)
  float *red = reinterpret_cast<float *>(s_tile);
#pragma unroll
  for (int i = 0; i < NT; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) red[(wave * NT + i) * 256 + lane * 4 + e] = acc[i][e];
  __syncthreads();
  if (t < NT * 256) {
    const int i = t >> 8, idx = t & 255;  // tile i, fragment slot idx = lane * 4 + register
    const int fl = idx >> 2, fr = idx & 3;
    const int b = (a.bt0 + i) * 16 + 4 * (fl >> 4) + fr, m = m0 + (fl & 15);
    float s = 0.f;
    for (int w = 0; w < kWaves; ++w) s += red[(w * NT + i) * 256 + idx];
    if (b < B && m < M) a.y[static_cast<int64_t>(b) * M + m] = s;
  }
}

template <int NT>
void launch_qw(const QwArgs &a, unsigned grid, hipStream_t s) {
  // 16-byte x loads need whole segments and a 16-byte aligned x
  if ((a.K & 63) == 0 && (reinterpret_cast<uintptr_t>(a.x) & 15) == 0)
    if (NT == 1 && a.B == 1)
      qw_matmul_kernel<NT, true, NT == 1 ? 1 : 0><<<grid, kThreads, 0, s>>>(a);
    else
      qw_matmul_kernel<NT, true, 0><<<grid, kThreads, 0, s>>>(a);
  else
    qw_matmul_kernel<NT, false, 0><<<grid, kThreads, 0, s>>>(a);
}

}  // namespace

extern "C" cf_status cf_qw_validate(const cf_qw_matrix *w) {
  if (!w || w->struct_size != sizeof(cf_qw_matrix) || w->abi_version != CF_QW_ABI_VERSION)
    return CF_ERR_INVALID_ARGUMENT;
  if (w->codec != CF_QW_CODEC_HUFFMAN && w->codec != CF_QW_CODEC_RANS) return CF_ERR_UNSUPPORTED;
  if (w->rows == 0 || w->cols == 0 || w->rows > (1u << 30) || w->cols > (1u << 30)) return CF_ERR_INVALID_ARGUMENT;
  if (!w->words || !w->offsets || !w->tables || !w->scales || w->word_count == 0) return CF_ERR_INVALID_ARGUMENT;
  if (w->zero < 0 || w->zero > 15) return CF_ERR_INVALID_ARGUMENT;
  if ((reinterpret_cast<uintptr_t>(w->tables) & 15) != 0) return CF_ERR_INVALID_ARGUMENT;
  return w->codec == CF_QW_CODEC_RANS ? cfqw::rans_validate(w) : CF_OK;
}

extern "C" cf_status cf_qw_matmul_async(const cf_qw_matrix *w, const uint16_t *x, float *y, uint32_t batch,
                                        void *stream) {
  const cf_status st = cf_qw_validate(w);
  if (st != CF_OK) return st;
  if (!x || !y) return CF_ERR_INVALID_ARGUMENT;
  if (batch == 0) return CF_OK;
  if (batch > (1u << 20)) return CF_ERR_UNSUPPORTED;
  if (w->codec == CF_QW_CODEC_RANS) return cfqw::rans_matmul(w, x, y, batch, cfd::as_stream(stream));
  QwArgs a{};
  a.words = w->words;
  a.word_count = w->word_count;
  a.seg_off = w->offsets;
  a.code_len = w->tables;
  a.scales = w->scales;
  a.x = x;
  a.y = y;
  a.B = static_cast<int>(batch);
  a.M = static_cast<int>(w->rows);
  a.K = static_cast<int>(w->cols);
  a.zero = w->zero;
  const hipStream_t s = cfd::as_stream(stream);
  const unsigned grid = cfd::grid_for(a.M, kRows);
  const int tiles = (a.B + 15) / 16;
  for (int bt0 = 0; bt0 < tiles; bt0 += kMaxTiles) {
    a.bt0 = bt0;
    switch (min(kMaxTiles, tiles - bt0)) {
      case 1: launch_qw<1>(a, grid, s); break;
      case 2: launch_qw<2>(a, grid, s); break;
      case 3: launch_qw<3>(a, grid, s); break;
      default: launch_qw<4>(a, grid, s); break;
    }
    const cf_status ls = cfd::launch_status();
    if (ls != CF_OK) return ls;
  }
  return CF_OK;
}
