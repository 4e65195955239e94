// oracle_succinct.cpp — TEST INFRASTRUCTURE ONLY. CPU restatement of the reference's succinct-structure
// algorithms, used as the checker for the HIP kernels. Only tests/, __graft_entry__.smoke() and bench.py's
// cpu_baseline leg may load this library; the product (libchromofold.so) never links or calls it.
//
// What it restates (reference paths are inside the reference tree):
//   RRR tables            tools/build_index.cpp:31-42
//   rrr_encode            tools/build_index.cpp:90-148
//   two_level samples     tools/build_index.cpp:151-161
//   build_wavelet         tools/build_index.cpp:172-218   (wavelet matrix: stable zeros-then-ones partition)
//   rank1/access/rank     tools/build_index.cpp:221-279 and include/chromofold/detail/rrr_wavelet_device.cuh:40-149
//   FM C/marks/msb/sval   tools/build_index.cpp:455-469
//   FM backward/locate    tools/build_index.cpp:283-319 and include/chromofold/detail/fm_search_device.cuh:31-62
//   naive search          tools/build_index.cpp:322-333
//   suffix array          include/chromofold/detail/suffix_cpu.hpp:31-48 (prefix doubling), plus a radix
//                         prefix-doubling variant for large n (same unique result)
//   packed wavelet        include/chromofold/detail/access_device.cuh:12-47, src/cuda/rank.cu:14-52
//   RRR bitvector rank1   src/cuda/rrr.cu:42-63
//
// Parity pins (see tests): every function here is checked against the reference's committed fixtures
// (tiny.cfrw / tiny.cffm / tiny.cfwv / tiny.cfrr), against closed forms (access(i) == seq[i],
// rank(c,i) == count, count == naive substring search, SA sortedness on tiny inputs by brute force) and,
// where the reference tool compiles here (oracle/_ref/build_index), against its arrays byte-for-byte.
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <numeric>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

namespace {

constexpr int kT = 15;  // bits per RRR block
constexpr int kS = 64;  // blocks per superblock
constexpr int kK = 32;  // superblocks per anchor

struct Tables {
  int64_t binom[16][16];
  int width[16];
  Tables() {
    std::memset(binom, 0, sizeof binom);
    for (int n = 0; n < 16; ++n) {
      binom[n][0] = 1;
      for (int k = 1; k <= n; ++k) binom[n][k] = binom[n - 1][k - 1] + binom[n - 1][k];
    }
    for (int k = 0; k < 16; ++k) {
      const int64_t c = binom[kT][k];
      int w = 0;
      while ((int64_t(1) << w) < c) ++w;
      width[k] = c > 1 ? w : 0;
    }
  }
};
const Tables &tables() {
  static Tables t;
  return t;
}

// ---------------------------------------------------------------- RRR wavelet matrix
struct Rrrw {
  int bits = 0, cwords = 0, nsb = 0, na = 0;
  int64_t n = 0, rrr_bytes = 0;
  std::vector<uint32_t> classes, offsets;
  std::vector<int32_t> rank_a, off_a, offbase, zeros;
  std::vector<uint16_t> rank_d, off_d;
};

struct Plane {
  std::vector<uint32_t> cls_words, off_words;
  std::vector<int32_t> sbrank, sboff;
  int nblocks = 0, nsb = 0, cwords = 0, zeros = 0;
  int64_t class_bits = 0, offset_bits = 0;
};

Plane encode_plane(const std::vector<uint8_t> &bit) {
  const Tables &tb = tables();
  Plane p;
  const int64_t n = (int64_t)bit.size();
  p.nblocks = (int)((n + kT - 1) / kT);
  p.cwords = (int)(((int64_t)p.nblocks * 4 + 31) / 32 + 1);
  p.cls_words.assign(p.cwords, 0u);
  std::vector<int> cls(p.nblocks);
  std::vector<int64_t> off(p.nblocks), obit(p.nblocks + 1, 0), ccum(p.nblocks + 1, 0);
  int64_t ones = 0;
  for (int b = 0; b < p.nblocks; ++b) {
    int k = 0;
    int64_t o = 0;
    for (int c = 0; c < kT; ++c) {
      const int64_t i = (int64_t)b * kT + c;
      if (i < n && bit[i]) {
        ++k;
        o += tb.binom[c][k];  // combinatorial number system rank of the set-bit positions
      }
    }
    cls[b] = k;
    off[b] = o;
    ones += k;
    p.cls_words[((int64_t)b * 4) >> 5] |= (uint32_t)k << (((int64_t)b * 4) & 31);
    obit[b + 1] = obit[b] + tb.width[k];
    ccum[b + 1] = ccum[b] + k;
  }
  p.class_bits = (int64_t)p.nblocks * 4;
  p.offset_bits = obit[p.nblocks];
  p.zeros = (int)(n - ones);
  p.off_words.assign((size_t)((obit[p.nblocks] + 31) / 32 + 2), 0u);
  for (int b = 0; b < p.nblocks; ++b) {
    const int w = tb.width[cls[b]];
    if (w == 0) continue;
    const int64_t at = obit[b];
    const uint64_t v = (uint64_t)off[b] << (at & 31);
    p.off_words[at >> 5] |= (uint32_t)v;
    if ((at & 31) + w > 32) p.off_words[(at >> 5) + 1] |= (uint32_t)(v >> 32);
  }
  p.nsb = (p.nblocks + kS - 1) / kS;
  p.sbrank.resize(p.nsb + 1);
  p.sboff.resize(p.nsb + 1);
  for (int i = 0; i <= p.nsb; ++i) {
    const int64_t b = std::min<int64_t>((int64_t)i * kS, p.nblocks);
    p.sbrank[i] = (int32_t)ccum[b];
    p.sboff[i] = (int32_t)obit[b];
  }
  return p;
}

void split_two_level(const int32_t *cum, int m, std::vector<int32_t> &anchors, std::vector<uint16_t> &delta) {
  const int na = (m + kK - 1) / kK;
  for (int a = 0; a < na; ++a) anchors.push_back(cum[(int64_t)a * kK]);
  const size_t base = anchors.size() - na;
  for (int i = 0; i < m; ++i) delta.push_back((uint16_t)(cum[i] - anchors[base + i / kK]));
}

Rrrw build_rrrw(const uint32_t *tok, int64_t n, int bits) {
  Rrrw w;
  w.bits = bits;
  w.n = n;
  std::vector<uint32_t> cur(tok, tok + n), nxt(n);
  std::vector<int32_t> sbr, sbo;
  int64_t owords = 0, stored_bits = 0;
  std::vector<uint8_t> plane(n);
  for (int lvl = 0; lvl < bits; ++lvl) {
    for (int64_t i = 0; i < n; ++i) plane[i] = (uint8_t)((cur[i] >> (bits - 1 - lvl)) & 1u);
    Plane p = encode_plane(plane);
    if (lvl == 0) {
      w.cwords = p.cwords;
      w.nsb = p.nsb;
    }
    w.classes.insert(w.classes.end(), p.cls_words.begin(), p.cls_words.end());
    w.offbase.push_back((int32_t)(owords * 32));
    w.offsets.insert(w.offsets.end(), p.off_words.begin(), p.off_words.end());
    owords += (int64_t)p.off_words.size();
    w.zeros.push_back(p.zeros);
    sbr.insert(sbr.end(), p.sbrank.begin(), p.sbrank.end());
    sbo.insert(sbo.end(), p.sboff.begin(), p.sboff.end());
    stored_bits += p.class_bits + p.offset_bits;
    int64_t z = 0;
    for (int64_t i = 0; i < n; ++i)
      if (!plane[i]) nxt[z++] = cur[i];
    for (int64_t i = 0; i < n; ++i)
      if (plane[i]) nxt[z++] = cur[i];
    cur.swap(nxt);
  }
  const int m = w.nsb + 1;
  w.na = (m + kK - 1) / kK;
  for (int lvl = 0; lvl < bits; ++lvl) {
    split_two_level(sbr.data() + (int64_t)lvl * m, m, w.rank_a, w.rank_d);
    split_two_level(sbo.data() + (int64_t)lvl * m, m, w.off_a, w.off_d);
  }
  w.rrr_bytes = stored_bits / 8 + (int64_t)(w.rank_a.size() + w.off_a.size()) * 4 +
                (int64_t)(w.rank_d.size() + w.off_d.size()) * 2;
  return w;
}

}  // namespace

extern "C" {

// Host-pointer twin of cf_rrrw_view (widths/binomials are the fixed tables above).
struct or_rrrw {
  const uint32_t *classes;
  const uint32_t *offsets;
  const int32_t *rank_a;
  const uint16_t *rank_d;
  const int32_t *off_a;
  const uint16_t *off_d;
  const int32_t *offbase;
  const int32_t *zeros;
  int bits, cwords, nsb, na;
};

void or_rrr_tables(int32_t *binom256, int32_t *width16) {
  const Tables &t = tables();
  for (int i = 0; i < 16; ++i)
    for (int j = 0; j < 16; ++j) binom256[i * 16 + j] = (int32_t)t.binom[i][j];
  for (int k = 0; k < 16; ++k) width16[k] = t.width[k];
}

int or_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void or_set_threads(int t) {
#ifdef _OPENMP
  if (t > 0) omp_set_num_threads(t);
#else
  (void)t;
#endif
}

// ---- build: returns an opaque handle; sizes via or_rrrw_info, arrays via or_rrrw_copy ----
void *or_rrrw_build(const uint32_t *tokens, int64_t n, int bits) { return new Rrrw(build_rrrw(tokens, n, bits)); }

// info: [bits, cwords, nsb, na, owords, classes_len, rank_a_len, rank_d_len, rrr_bytes_lo, rrr_bytes_hi]
void or_rrrw_info(void *h, int64_t *info) {
  const Rrrw &w = *static_cast<Rrrw *>(h);
  info[0] = w.bits;
  info[1] = w.cwords;
  info[2] = w.nsb;
  info[3] = w.na;
  info[4] = (int64_t)w.offsets.size();
  info[5] = (int64_t)w.classes.size();
  info[6] = (int64_t)w.rank_a.size();
  info[7] = (int64_t)w.rank_d.size();
  info[8] = w.rrr_bytes;
}

void or_rrrw_copy(void *h, uint32_t *classes, uint32_t *offsets, int32_t *rank_a, uint16_t *rank_d, int32_t *off_a,
                  uint16_t *off_d, int32_t *offbase, int32_t *zeros) {
  const Rrrw &w = *static_cast<Rrrw *>(h);
  std::copy(w.classes.begin(), w.classes.end(), classes);
  std::copy(w.offsets.begin(), w.offsets.end(), offsets);
  std::copy(w.rank_a.begin(), w.rank_a.end(), rank_a);
  std::copy(w.rank_d.begin(), w.rank_d.end(), rank_d);
  std::copy(w.off_a.begin(), w.off_a.end(), off_a);
  std::copy(w.off_d.begin(), w.off_d.end(), off_d);
  std::copy(w.offbase.begin(), w.offbase.end(), offbase);
  std::copy(w.zeros.begin(), w.zeros.end(), zeros);
}

void or_rrrw_free(void *h) { delete static_cast<Rrrw *>(h); }

}  // extern "C"

namespace {

inline int class_at(const uint32_t *cls, int64_t j) { return (int)((cls[(j * 4) >> 5] >> ((j * 4) & 31)) & 15u); }

inline int read_bits(const uint32_t *s, int64_t at, int w) {
  if (w == 0) return 0;
  const int b = (int)(at & 31);
  uint32_t v = s[at >> 5] >> b;
  if (b + w > 32) v |= s[(at >> 5) + 1] << (32 - b);
  return (int)(v & ((w >= 32) ? 0xFFFFFFFFu : ((1u << w) - 1u)));
}

// enumerative unrank: greedy largest position c with C(c, i) <= r, for i = class .. 1
inline uint32_t unrank(int k, int r) {
  const Tables &tb = tables();
  uint32_t word = 0;
  for (int i = k; i >= 1; --i) {
    int c = kT - 1;
    while (tb.binom[c][i] > r) --c;
    word |= 1u << c;
    r -= (int)tb.binom[c][i];
  }
  return word;
}

inline int rank1_level(const or_rrrw &v, int lvl, int pos, int *bit_out) {
  const Tables &tb = tables();
  const uint32_t *cls = v.classes + (int64_t)lvl * v.cwords;
  const int blk = pos / kT, b = pos % kT, sbi = blk / kS, a = sbi / kK;
  int r = v.rank_a[(int64_t)lvl * v.na + a] + (int)v.rank_d[(int64_t)lvl * (v.nsb + 1) + sbi];
  int64_t obit = (int64_t)v.off_a[(int64_t)lvl * v.na + a] + (int)v.off_d[(int64_t)lvl * (v.nsb + 1) + sbi];
  for (int j = sbi * kS; j < blk; ++j) {
    const int k = class_at(cls, j);
    r += k;
    obit += tb.width[k];
  }
  if (b > 0 || bit_out) {
    const int k = class_at(cls, blk);
    const uint32_t word = unrank(k, read_bits(v.offsets, (int64_t)v.offbase[lvl] + obit, tb.width[k]));
    if (bit_out) *bit_out = (int)((word >> b) & 1u);
    r += __builtin_popcount(word & ((1u << b) - 1u));
  }
  return r;
}

inline uint32_t access_one(const or_rrrw &v, int i) {
  uint32_t val = 0;
  for (int lvl = 0; lvl < v.bits; ++lvl) {
    int bit = 0;
    const int r = rank1_level(v, lvl, i, &bit);
    val = (val << 1) | (uint32_t)bit;
    i = bit ? v.zeros[lvl] + r : i - r;
  }
  return val;
}

inline uint32_t rank_one(const or_rrrw &v, int c, int i) {
  int p = 0, q = i;
  for (int lvl = 0; lvl < v.bits; ++lvl) {
    const int rp = rank1_level(v, lvl, p, nullptr), rq = rank1_level(v, lvl, q, nullptr);
    if ((c >> (v.bits - 1 - lvl)) & 1) {
      p = v.zeros[lvl] + rp;
      q = v.zeros[lvl] + rq;
    } else {
      p -= rp;
      q -= rq;
    }
  }
  return (uint32_t)(q - p);
}

}  // namespace

extern "C" {

int or_rrrw_rank1(const or_rrrw *v, int lvl, int pos) { return rank1_level(*v, lvl, pos, nullptr); }

void or_rrrw_access(const or_rrrw *v, const uint32_t *pos, uint32_t *out, int64_t count) {
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < count; ++t) out[t] = access_one(*v, (int)pos[t]);
}

void or_rrrw_rank(const or_rrrw *v, const uint32_t *sym, const uint32_t *pos, uint32_t *out, int64_t count) {
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < count; ++t) out[t] = rank_one(*v, (int)sym[t], (int)pos[t]);
}

// ---------------------------------------------------------------- suffix array
// Literal prefix doubling with comparison sort (reference suffix_cpu.hpp:31-48). O(n log^2 n): small n only.
void or_suffix_array_doubling(const int32_t *s, int32_t n, int32_t *sa_out) {
  std::vector<int> sa(n), rk(n), tmp(n);
  for (int i = 0; i < n; ++i) {
    sa[i] = i;
    rk[i] = s[i];
  }
  for (int k = 1;; k <<= 1) {
    auto second = [&](int i) { return i + k < n ? rk[i + k] : -1; };
    auto less = [&](int a, int b) { return rk[a] != rk[b] ? rk[a] < rk[b] : second(a) < second(b); };
    std::sort(sa.begin(), sa.end(), less);
    tmp[sa[0]] = 0;
    for (int i = 1; i < n; ++i) tmp[sa[i]] = tmp[sa[i - 1]] + (less(sa[i - 1], sa[i]) ? 1 : 0);
    rk = tmp;
    if (rk[sa[n - 1]] == n - 1) break;
  }
  std::copy(sa.begin(), sa.end(), sa_out);
}

// Prefix doubling with stable counting sorts (Manber-Myers style); same unique SA, O(n log n), for large n.
void or_suffix_array_radix(const int32_t *s, int32_t n, int32_t *sa_out) {
  if (n <= 0) return;
  int32_t maxv = 0;
  for (int i = 0; i < n; ++i) maxv = std::max(maxv, s[i]);
  std::vector<int32_t> rk(s, s + n), sa(n), sa2(n), cnt(std::max<int64_t>(maxv, n) + 2), tmp(n);
  // initial order by symbol
  std::fill(cnt.begin(), cnt.end(), 0);
  for (int i = 0; i < n; ++i) cnt[rk[i] + 1]++;
  for (size_t i = 1; i < cnt.size(); ++i) cnt[i] += cnt[i - 1];
  for (int i = 0; i < n; ++i) sa[cnt[rk[i]]++] = i;
  // dense ranks
  tmp[sa[0]] = 0;
  for (int i = 1; i < n; ++i) tmp[sa[i]] = tmp[sa[i - 1]] + (rk[sa[i]] != rk[sa[i - 1]] ? 1 : 0);
  rk = tmp;
  for (int64_t k = 1; rk[sa[n - 1]] != n - 1; k <<= 1) {
    // order by second key: suffixes with i+k >= n first (in increasing i), then by rk[i+k]
    int p = 0;
    for (int i = (int)std::max<int64_t>(0, n - k); i < n; ++i) sa2[p++] = i;
    for (int j = 0; j < n; ++j)
      if (sa[j] >= k) sa2[p++] = (int)(sa[j] - k);
    // stable counting sort by first key
    std::fill(cnt.begin(), cnt.begin() + n + 1, 0);
    for (int i = 0; i < n; ++i) cnt[rk[i] + 1]++;
    for (int i = 1; i <= n; ++i) cnt[i] += cnt[i - 1];
    for (int j = 0; j < n; ++j) sa[cnt[rk[sa2[j]]]++] = sa2[j];
    auto second = [&](int i) { return i + k < n ? rk[i + k] : -1; };
    tmp[sa[0]] = 0;
    for (int i = 1; i < n; ++i) {
      const int a = sa[i - 1], b = sa[i];
      tmp[b] = tmp[a] + ((rk[a] != rk[b] || second(a) != second(b)) ? 1 : 0);
    }
    rk = tmp;
  }
  std::copy(sa.begin(), sa.end(), sa_out);
}

// ---------------------------------------------------------------- FM-index
// C-table, mark plane, its SB=8 directory and sampled SA values (reference build_index.cpp:455-469).
// mwords must hold (n+31)/32 words, msb ((n+31)/32+7)/8+1 entries; returns the sval count written.
int32_t or_fm_build(const int32_t *sa, const int32_t *bwt, int32_t n, int32_t sigma, int32_t sa_sample, int32_t *C,
                    uint32_t *mwords, int32_t *msb, int32_t *sval) {
  std::vector<int64_t> cnt(sigma, 0);
  for (int i = 0; i < n; ++i) cnt[bwt[i]]++;
  int64_t acc = 0;
  for (int c = 0; c < sigma; ++c) {
    C[c] = (int32_t)acc;
    acc += cnt[c];
  }
  const int nw = (n + 31) / 32, nb = (nw + 7) / 8;
  std::fill(mwords, mwords + nw, 0u);
  int32_t ns = 0;
  for (int i = 0; i < n; ++i)
    if (sa[i] % sa_sample == 0) {
      mwords[i >> 5] |= 1u << (i & 31);
      sval[ns++] = sa[i];
    }
  int64_t run = 0;
  for (int j = 0; j <= nb; ++j) {
    msb[j] = (int32_t)run;
    if (j < nb)
      for (int k = j * 8; k < std::min(nw, j * 8 + 8); ++k) run += __builtin_popcount(mwords[k]);
  }
  return ns;
}

struct or_fm {
  or_rrrw w;
  const int32_t *C;
  const uint32_t *mwords;
  const int32_t *msb;
  const int32_t *sval;
  int sigma, n, sa_sample;
};

static inline int packed_rank1(const uint32_t *w, const int32_t *sb, int pos) {
  const int word = pos >> 5, bit = pos & 31, blk = word / 8;
  int r = sb[blk];
  for (int k = blk * 8; k < word; ++k) r += __builtin_popcount(w[k]);
  if (bit) r += __builtin_popcount(w[word] & ((1u << bit) - 1u));
  return r;
}

static inline void fm_backward(const or_fm &f, const int32_t *pat, int len, int &lo, int &hi) {
  lo = 0;
  hi = f.n;
  for (int k = len - 1; k >= 0; --k) {
    const int c = pat[k];
    if (c < 0 || c >= f.sigma) {
      lo = hi = 0;
      continue;
    }
    if (lo < hi) {
      lo = f.C[c] + (int)rank_one(f.w, c, lo);
      hi = f.C[c] + (int)rank_one(f.w, c, hi);
    }
  }
}

void or_fm_ranges(const or_fm *f, const int32_t *pat, const int32_t *pstart, const int32_t *plen, int32_t *lo,
                  int32_t *hi, int64_t npat) {
#pragma omp parallel for schedule(dynamic, 64)
  for (int64_t t = 0; t < npat; ++t) {
    int a, b;
    fm_backward(*f, pat + pstart[t], plen[t], a, b);
    lo[t] = a;
    hi[t] = b;
  }
}

void or_fm_count(const or_fm *f, const int32_t *pat, const int32_t *pstart, const int32_t *plen, uint32_t *out,
                 int64_t npat) {
#pragma omp parallel for schedule(dynamic, 64)
  for (int64_t t = 0; t < npat; ++t) {
    int a, b;
    fm_backward(*f, pat + pstart[t], plen[t], a, b);
    out[t] = (uint32_t)(b - a);
  }
}

void or_fm_locate(const or_fm *f, const int32_t *rows, int32_t *out, int64_t nocc) {
#pragma omp parallel for schedule(dynamic, 64)
  for (int64_t t = 0; t < nocc; ++t) {
    int p = rows[t], steps = 0;
    while (!((f->mwords[p >> 5] >> (p & 31)) & 1u)) {
      const int c = (int)access_one(f->w, p);
      p = f->C[c] + (int)rank_one(f->w, c, p);
      ++steps;
    }
    const int idx = packed_rank1(f->mwords, f->msb, p);
    out[t] = (int32_t)(((int64_t)f->sval[idx] + steps) % f->n);
  }
}

// Ground truth: number of occurrences (and optionally positions) of pat (original alphabet) in seq.
int64_t or_naive_positions(const int32_t *seq, int64_t n, const int32_t *pat, int m, int32_t *pos_out,
                           int64_t cap) {
  int64_t found = 0;
  if (m <= 0 || m > n) return 0;
  for (int64_t i = 0; i + m <= n; ++i) {
    int j = 0;
    while (j < m && seq[i + j] == pat[j]) ++j;
    if (j == m) {
      if (pos_out && found < cap) pos_out[found] = (int32_t)i;
      ++found;
    }
  }
  return found;
}

// ---------------------------------------------------------------- packed wavelet matrix (SB = 8 words)
// bitplanes [levels*nwords], superblocks [levels*(nblocks+1)], zeros [levels]; nblocks = (nwords+7)/8.
void or_packed_build(const uint32_t *tok, int64_t n, int levels, uint32_t *bitplanes, int32_t *superblocks,
                     int32_t *zeros) {
  const int64_t nwords = (n + 31) / 32, nblocks = (nwords + 7) / 8;
  std::vector<uint32_t> cur(tok, tok + n), nxt(n);
  for (int lvl = 0; lvl < levels; ++lvl) {
    uint32_t *w = bitplanes + lvl * nwords;
    int32_t *sb = superblocks + lvl * (nblocks + 1);
    std::fill(w, w + nwords, 0u);
    int64_t z = 0;
    for (int64_t i = 0; i < n; ++i)
      if ((cur[i] >> (levels - 1 - lvl)) & 1u) w[i >> 5] |= 1u << (i & 31);
    int64_t run = 0;
    for (int64_t b = 0; b <= nblocks; ++b) {
      sb[b] = (int32_t)run;
      if (b < nblocks)
        for (int64_t k = b * 8; k < std::min(nwords, b * 8 + 8); ++k) run += __builtin_popcount(w[k]);
    }
    for (int64_t i = 0; i < n; ++i)
      if (!((cur[i] >> (levels - 1 - lvl)) & 1u)) nxt[z++] = cur[i];
    zeros[lvl] = (int32_t)z;
    for (int64_t i = 0; i < n; ++i)
      if ((cur[i] >> (levels - 1 - lvl)) & 1u) nxt[z++] = cur[i];
    cur.swap(nxt);
  }
}

void or_packed_access(const uint32_t *bitplanes, const int32_t *superblocks, const int32_t *zeros, int levels,
                      int nwords, int nblocks, const uint32_t *pos, uint32_t *out, int64_t count) {
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < count; ++t) {
    int i = (int)pos[t];
    uint32_t v = 0;
    for (int lvl = 0; lvl < levels; ++lvl) {
      const uint32_t *w = bitplanes + (int64_t)lvl * nwords;
      const int r = packed_rank1(w, superblocks + (int64_t)lvl * (nblocks + 1), i);
      const int b = (int)((w[i >> 5] >> (i & 31)) & 1u);
      v = (v << 1) | (uint32_t)b;
      i = b ? zeros[lvl] + r : i - r;
    }
    out[t] = v;
  }
}

void or_packed_rank(const uint32_t *bitplanes, const int32_t *superblocks, const int32_t *zeros, int levels,
                    int nwords, int nblocks, const uint32_t *sym, const uint32_t *pos, uint32_t *out,
                    int64_t count) {
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < count; ++t) {
    const int c = (int)sym[t];
    int p = 0, q = (int)pos[t];
    for (int lvl = 0; lvl < levels; ++lvl) {
      const uint32_t *w = bitplanes + (int64_t)lvl * nwords;
      const int32_t *sb = superblocks + (int64_t)lvl * (nblocks + 1);
      const int rp = packed_rank1(w, sb, p), rq = packed_rank1(w, sb, q);
      if ((c >> (levels - 1 - lvl)) & 1) {
        p = zeros[lvl] + rp;
        q = zeros[lvl] + rq;
      } else {
        p -= rp;
        q -= rq;
      }
    }
    out[t] = (uint32_t)(q - p);
  }
}

int or_packed_rank1(const uint32_t *w, const int32_t *sb, int pos) { return packed_rank1(w, sb, pos); }

// ---------------------------------------------------------------- single RRR bitvector (.cfrr, one-level samples)
void or_rrr_rank1(const uint32_t *classes, const uint32_t *offsets, const int32_t *sbrank, const int32_t *sboff,
                  const uint32_t *pos, uint32_t *out, int64_t count) {
  const Tables &tb = tables();
  for (int64_t t = 0; t < count; ++t) {
    const int p = (int)pos[t], blk = p / kT, b = p % kT, sbi = blk / kS;
    int r = sbrank[sbi];
    int64_t obit = sboff[sbi];
    for (int j = sbi * kS; j < blk; ++j) {
      const int k = class_at(classes, j);
      r += k;
      obit += tb.width[k];
    }
    if (b > 0) {
      const int k = class_at(classes, blk);
      r += __builtin_popcount(unrank(k, read_bits(offsets, obit, tb.width[k])) & ((1u << b) - 1u));
    }
    out[t] = (uint32_t)r;
  }
}

// Encode a single 0/1 plane the .cfrr way (one-level int32 samples). Output sizes: cwords, owords, nsb+1.
void *or_rrr_plane_build(const uint8_t *bits, int64_t n) { return new Plane(encode_plane(std::vector<uint8_t>(bits, bits + n))); }
void or_rrr_plane_info(void *h, int64_t *info) {
  const Plane &p = *static_cast<Plane *>(h);
  info[0] = p.nblocks;
  info[1] = p.nsb;
  info[2] = p.cwords;
  info[3] = (int64_t)p.off_words.size();
  info[4] = p.class_bits;
  info[5] = p.offset_bits;
  info[6] = p.zeros;
}
void or_rrr_plane_copy(void *h, uint32_t *classes, uint32_t *offsets, int32_t *sbrank, int32_t *sboff) {
  const Plane &p = *static_cast<Plane *>(h);
  std::copy(p.cls_words.begin(), p.cls_words.end(), classes);
  std::copy(p.off_words.begin(), p.off_words.end(), offsets);
  std::copy(p.sbrank.begin(), p.sbrank.end(), sbrank);
  std::copy(p.sboff.begin(), p.sboff.end(), sboff);
}
void or_rrr_plane_free(void *h) { delete static_cast<Plane *>(h); }

// decode every block of an RRR stream back into bits (inverse of encode; pins the enumerative code)
void or_rrr_decode_all(const uint32_t *classes, const uint32_t *offsets, int64_t nblocks, int64_t off_base_bit,
                       uint8_t *bits_out) {
  const Tables &tb = tables();
  int64_t obit = off_base_bit;
  for (int64_t b = 0; b < nblocks; ++b) {
    const int k = class_at(classes, b);
    const uint32_t word = unrank(k, read_bits(offsets, obit, tb.width[k]));
    obit += tb.width[k];
    for (int c = 0; c < kT; ++c) bits_out[b * kT + c] = (uint8_t)((word >> c) & 1u);
  }
}

}  // extern "C"
