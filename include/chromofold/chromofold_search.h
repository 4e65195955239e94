/* chromofold_search.h — C ABI of the RRR-backed wavelet matrix and the FM-index (compressed-domain search).
 *
 * Drop-in for the reference include/chromofold/chromofold_search.h: the view structs are byte-identical
 * (cf_rrrw_view 96 B, cf_fm_view 144 B on x86-64) and the five entry points keep their signatures.
 * All pointers are device pointers; views are POD and passed by value; `stream` is a hipStream_t as void*.
 *
 * RRR constants are fixed by the on-disk format (.cfrw/.cffm) and the committed fixtures:
 * T = 15-bit blocks, S = 64 blocks per rank superblock, K = 32 superblocks per int32 anchor.
 */
#ifndef CHROMOFOLD_SEARCH_H
#define CHROMOFOLD_SEARCH_H

#include "chromofold/chromofold.h"

#ifdef __cplusplus
extern "C" {
#endif

/* reference chromofold_search.h:27-42 */
typedef struct cf_rrrw_view {
  const uint32_t *classes; /* [bits * cwords]    4-bit block classes (popcounts) per level, LSB-first nibbles */
  const uint32_t *offsets; /* [owords]           enumerative offsets of all levels, LSB-first, width[class] bits */
  const int32_t *rank_a;   /* [bits * na]        rank anchor every K superblocks */
  const uint16_t *rank_d;  /* [bits * (nsb+1)]   rank delta per superblock, relative to its anchor */
  const int32_t *off_a;    /* [bits * na]        offset-bit anchor */
  const uint16_t *off_d;   /* [bits * (nsb+1)]   offset-bit delta per superblock */
  const int32_t *offbase;  /* [bits]             bit position of each level's slice inside offsets[] */
  const int32_t *zeros;    /* [bits]             number of 0-bits per level */
  const int *width;        /* [16]               offset width per class: ceil(log2 C(15,k)), 0 when C(15,k) <= 1 */
  const int *binom;        /* [16 * 16]          Pascal's triangle C(n,k) at [n*16 + k] */
  int bits;                /* levels */
  int cwords;              /* class words per level */
  int nsb;                 /* superblocks per level */
  int na;                  /* anchors per level */
} cf_rrrw_view;

/* reference chromofold_search.h:46-55 */
typedef struct cf_fm_view {
  cf_rrrw_view w;         /* RRR wavelet matrix of the BWT */
  const int32_t *C;       /* [sigma]  exclusive prefix counts of BWT symbols */
  const uint32_t *mwords; /* packed mark plane: bit p set <=> SA[p] % sa_sample == 0 */
  const int32_t *msb;     /* cumulative popcount of mwords every CF_WAVELET_SB words */
  const int32_t *sval;    /* sampled SA values in SA order */
  int sigma;
  int n;                  /* BWT length (text + sentinel) */
  int sa_sample;
} cf_fm_view;

/* access: out[t] = token at positions[t]. Replaces reference chromofold_search.h:59 (src/cuda/rrr_wavelet.cu:25-45). */
cf_status cf_rrrw_access_async(cf_rrrw_view v, const uint32_t *positions, uint32_t *out, size_t count,
                               void *stream);
/* rank: out[t] = #{ j < positions[t] : seq[j] == symbols[t] }. Replaces reference chromofold_search.h:62
 * (src/cuda/rrr_wavelet.cu:47-67). */
cf_status cf_rrrw_rank_async(cf_rrrw_view v, const uint32_t *symbols, const uint32_t *positions, uint32_t *out,
                             size_t count, void *stream);

/* count: out[t] = occurrences of pattern t (symbols already shifted +1 into the sentinel alphabet).
 * Replaces reference chromofold_search.h:68 (src/cuda/fm_search.cu:51-62). */
cf_status cf_fm_count_async(cf_fm_view v, const int32_t *pat, const int32_t *pstart, const int32_t *plen,
                            uint32_t *out, size_t npat, void *stream);
/* ranges: SA interval [lo, hi) per pattern. Replaces reference chromofold_search.h:71 (src/cuda/fm_search.cu:64-76). */
cf_status cf_fm_ranges_async(cf_fm_view v, const int32_t *pat, const int32_t *pstart, const int32_t *plen,
                             int32_t *lo_out, int32_t *hi_out, size_t npat, void *stream);
/* locate: out[t] = text position of SA row r_in[t]. Replaces reference chromofold_search.h:74
 * (src/cuda/fm_search.cu:78-89). */
cf_status cf_fm_locate_async(cf_fm_view v, const int32_t *r_in, int32_t *out, size_t nocc, void *stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* CHROMOFOLD_SEARCH_H */
