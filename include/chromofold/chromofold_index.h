/* chromofold_index.h — ADDITIVE: on-device construction helpers for the compressed-domain search index.
 *
 * The reference builds its FM-index suffix array with a C++ host-vector function (reference
 * src/cuda/suffix_array.cu:42, `void cf_gpu_suffix_array(const std::vector<int>&, std::vector<int>&)`), declared
 * by its callers; that function is exported unchanged (C++ linkage, see the bottom of this header). The C entry
 * points below are the device-pointer form of the same build for callers that keep the text in HBM.
 */
#ifndef CHROMOFOLD_INDEX_H
#define CHROMOFOLD_INDEX_H

#include <stdint.h>

#include "chromofold/chromofold.h"
#include "chromofold/chromofold_search.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Workspace bytes cf_suffix_array needs for a text of n symbols with values in [0, max_symbol] (0 if the
 * packed pair key would exceed 64 bits). Host only. */
uint64_t cf_suffix_array_workspace_bytes(int32_t n, int32_t max_symbol);

/* Suffix array of s[0..n) (device pointers; s must end with a unique smallest sentinel for the usual FM-index
 * text, as the reference builder writes it) by prefix doubling on the GPU. Synchronises `stream` once per
 * doubling round to test convergence (the round count is data dependent), like the reference's thrust build.
 * No counterpart in the reference C ABI; replaces reference src/cuda/suffix_array.cu:42-65. */
cf_status cf_suffix_array(const int32_t *s, int32_t n, int32_t max_symbol, int32_t *sa_out, void *workspace,
                          uint64_t workspace_bytes, void *stream);

/* ---- on-device RRR wavelet matrix build (the .cfrw arrays of cf_rrrw_view) ----
 * Layout identical to the reference builder (tools/build_index.cpp:90-218): T = 15-bit blocks, 64 blocks per
 * superblock, 32 superblocks per anchor, class nibbles LSB-first, offsets LSB-first packed per level with
 * offbase[level] = bit offset of the level's first offset word. */
typedef struct cf_rrrw_layout {
  uint64_t n;
  uint32_t bits, nblocks, cwords, nsb, na;
  uint32_t owords;              /* total offset words over all levels */
  uint64_t rrr_bytes;           /* stored class + offset bits / 8 + sample bytes (the .cfrw header figure) */
  uint32_t level_owords[32];    /* offset words of each level (2 words of padding included) */
} cf_rrrw_layout;

typedef struct cf_rrrw_arrays { /* device outputs, sized from the layout */
  uint32_t *classes;  /* [bits * cwords] */
  uint32_t *offsets;  /* [owords] */
  int32_t *rank_a;    /* [bits * na] */
  uint16_t *rank_d;   /* [bits * (nsb + 1)] */
  int32_t *off_a;     /* [bits * na] */
  uint16_t *off_d;    /* [bits * (nsb + 1)] */
  int32_t *offbase;   /* [bits] */
  int32_t *zeros;     /* [bits] */
} cf_rrrw_arrays;

/* Workspace for cf_rrrw_build (0 if n or bits are out of range: n < 2^31, 1 <= bits <= 31). Host only. */
uint64_t cf_rrrw_build_workspace_bytes(uint64_t n, uint32_t bits);

/* Builds every level of the RRR wavelet matrix of tokens[0..n) (device, values < 2^bits) inside the workspace and
 * reports the sizes; synchronises `stream` once at the end (the offset-stream lengths are data dependent).
 * No counterpart in the reference C ABI (its builder is the CPU tool tools/build_index.cpp). */
cf_status cf_rrrw_build(const uint32_t *tokens, uint64_t n, uint32_t bits, void *workspace, uint64_t workspace_bytes,
                        cf_rrrw_layout *layout, void *stream);

/* Copies a built matrix from the workspace into caller arrays (asynchronous device-to-device copies). */
cf_status cf_rrrw_build_copy(const void *workspace, const cf_rrrw_layout *layout, const cf_rrrw_arrays *out,
                             void *stream);

/* ---- on-device FM-index side arrays (reference tools/build_index.cpp:368-371, 455-469) ----
 * From the text s[0..n) (device, ending in the unique sentinel 0, symbols < sigma) and its suffix array: bwt[i] =
 * s[sa[i] - 1] (cyclic), C[c] = #symbols < c, mark plane mwords[(n + 31) / 32] (bit i set when sa[i] % sa_sample == 0)
 * with its directory msb[nb + 1] (cumulative marks every 8 words, nb = ((n + 31) / 32 + 7) / 8), and sval (sa of the
 * marked rows in row order; *sval_count receives their number after the one synchronisation). */
uint64_t cf_fm_build_workspace_bytes(int32_t n, int32_t sigma);
cf_status cf_fm_build_aux(const int32_t *s, const int32_t *sa, int32_t n, int32_t sigma, int32_t sa_sample,
                          uint32_t *bwt, int32_t *C, uint32_t *mwords, int32_t *msb, int32_t *sval, int32_t *sval_count,
                          void *workspace, uint64_t workspace_bytes, void *stream);

/* ---- derived on-device line layout of an RRR wavelet matrix (no counterpart in the reference; the .cfrw on disk
 * and the cf_rrrw_view arrays are unchanged). Built once per loaded matrix from its view; access and rank over it
 * return exactly what cf_rrrw_access_async / cf_rrrw_rank_async return for positions in [0, n] (positions past n
 * give unspecified values, never an out-of-bounds read). One 64-byte line per level for access and for rank (the
 * RRR rank walks two chains of three or four lines per level). Layout of `lines` (u32 words, 16-byte aligned):
 *   [bits][nrec][16] records, nrec = 2 * nsb + 1: word 0 = ones of the level before bit 480 r, words 1..15 = level
 *   bits [480 r, 480 r + 480) LSB-first;
 *   then [2^bits] int32 base[c] = -(position where the wavelet rank walk of symbol c from 0 ends), so that
 *   rank(c, i) = (end of the walk of i) + base[c].
 * Size: (bits * nrec * 16 + 2^bits) * 4 bytes; supported for bits <= 24 (cf_rrrw_lines_bytes returns 0 otherwise,
 * or when the view's anchors do not cover superblock nsb). */
uint64_t cf_rrrw_lines_bytes(cf_rrrw_view v);
cf_status cf_rrrw_lines_build_async(cf_rrrw_view v, uint32_t *lines, uint64_t bytes, void *stream);
cf_status cf_rrrw_access_lines_async(cf_rrrw_view v, const uint32_t *lines, const uint32_t *positions, uint32_t *out,
                                     size_t count, void *stream);
cf_status cf_rrrw_rank_lines_async(cf_rrrw_view v, const uint32_t *lines, const uint32_t *symbols,
                                   const uint32_t *positions, uint32_t *out, size_t count, void *stream);

/* ---- derived on-device 4-ary layout of an RRR wavelet matrix (no counterpart in the reference; the .cfrw on disk
 * and the cf_rrrw_view arrays are unchanged). The sequence (n symbols: the view does not hold n) read as base-4
 * digits, most significant first, in L4 = ceil(bits / 2) levels of a 4-ary wavelet matrix: access and rank read L4
 * 64-byte records per query (8 at bits 15) instead of the binary layouts' `bits`. Results equal cf_rrrw_access_async
 * / cf_rrrw_rank_async for positions in [0, n] (past n: unspecified values, never an out-of-bounds read). Level 0
 * holds every position's top digit in sequence order; level l + 1 the positions of level l stably sorted by their
 * digit l. Layout of `quads` (u32 words, 16-byte aligned):
 *   [L4][nrec][16] records, nrec = n / 208 + 1: words 0..2 = how many of digits 0, 1, 2 the level holds before
 *   position 208 r, words 3..15 = the level's digits at positions [208 r, 208 r + 208), 16 two-bit digits per word,
 *   LSB-first;
 *   then Z [L4][4] u32 (Z[l][d] = positions of level l whose digit is below d);
 *   then [2^bits] int32 base[c] = -(where the walk of symbol c from position 0 ends), rank(c, i) = walk(i) + base[c].
 * bits <= 24 and n < 2^31 (the byte counts are 0 otherwise). The build decodes the sequence from the view into
 * `workspace` (cf_rrrw_quads_workspace_bytes, 256-byte aligned) and sorts it level by level there. */
uint64_t cf_rrrw_quads_bytes(cf_rrrw_view v, uint64_t n);
uint64_t cf_rrrw_quads_workspace_bytes(cf_rrrw_view v, uint64_t n);
cf_status cf_rrrw_quads_build_async(cf_rrrw_view v, uint64_t n, uint32_t *quads, uint64_t bytes, void *workspace,
                                    uint64_t workspace_bytes, void *stream);
cf_status cf_rrrw_access_quads_async(cf_rrrw_view v, uint64_t n, const uint32_t *quads, const uint32_t *positions,
                                     uint32_t *out, size_t count, void *stream);
cf_status cf_rrrw_rank_quads_async(cf_rrrw_view v, uint64_t n, const uint32_t *quads, const uint32_t *symbols,
                                   const uint32_t *positions, uint32_t *out, size_t count, void *stream);

/* cf_sparse_gather_fused_async (chromofold_extra.h, reference src/cuda/sparse_gather.cu:55-66) over the line layout:
 * out[t, :] = emb[access(pos[t]), :] for t < count, the same bytes, each query's access walk reading one 64-byte
 * line per level. Same argument rules (count 0 or dim <= 0: nothing to do). */
cf_status cf_sparse_gather_fused_lines_async(cf_rrrw_view v, const uint32_t *lines, const float *emb, int dim,
                                             const uint32_t *pos, float *out, size_t count, void *stream);

/* The same gather over the 4-ary layout (cf_rrrw_quads_build_async, n the sequence's length): each query's access
 * walk reads one 64-byte record per 4-ary level (8 at 15 bits instead of the line layout's 15). Same bytes out, same
 * argument rules; quads 16-byte aligned. */
cf_status cf_sparse_gather_fused_quads_async(cf_rrrw_view v, uint64_t n, const uint32_t *quads, const float *emb,
                                             int dim, const uint32_t *pos, float *out, size_t count, void *stream);

/* ---- derived on-device line layout for FM search (no counterpart in the reference; the .cffm on disk and the
 * cf_fm_view arrays are unchanged). Built once per loaded index from its cf_fm_view; the search entry points below
 * return exactly what cf_fm_count_async / cf_fm_ranges_async / cf_fm_locate_async return for the same view, with one
 * 64-byte line per rank1 instead of the RRR level's three or four and fewer rank1 per step (2 per level for
 * backward search, 1 for an LF step). Layout of `lines` (u32 words, 64-byte aligned):
 *   [bits][nrec][16] records, nrec = n / 480 + 1: word 0 = ones of the level before bit 480 r, words 1..15 = level
 *   bits [480 r, 480 r + 480) LSB-first;
 *   then [sigma] int32 lfb[c] = C[c] - (position where the wavelet rank walk of symbol c from 0 ends).
 * Size: (bits * nrec * 16 + sigma) * 4 bytes, about 1.07 bits per BWT bit per level. */

/* Bytes of the line layout of `v` (0 if the view is out of range). Host only. */
uint64_t cf_fm_lines_bytes(cf_fm_view v);
/* Builds the line layout of `v` into `lines` (device, >= cf_fm_lines_bytes(v) bytes, 16-byte aligned), stream
 * ordered after whatever wrote the view's arrays. Reads the view's RRR arrays, C and zeros. */
cf_status cf_fm_lines_build_async(cf_fm_view v, uint32_t *lines, uint64_t bytes, void *stream);
/* cf_fm_count_async / cf_fm_ranges_async / cf_fm_locate_async (chromofold_search.h) over the line layout built
 * from the same view: same arguments, same results. */
cf_status cf_fm_count_lines_async(cf_fm_view v, const uint32_t *lines, const int32_t *pat, const int32_t *pstart,
                                  const int32_t *plen, uint32_t *out, size_t npat, void *stream);
cf_status cf_fm_ranges_lines_async(cf_fm_view v, const uint32_t *lines, const int32_t *pat, const int32_t *pstart,
                                   const int32_t *plen, int32_t *lo_out, int32_t *hi_out, size_t npat, void *stream);
cf_status cf_fm_locate_lines_async(cf_fm_view v, const uint32_t *lines, const int32_t *r_in, int32_t *out,
                                   size_t nocc, void *stream);

/* ---- derived on-device 4-ary layout for FM search (no counterpart in the reference; the .cffm on disk and the
 * cf_fm_view arrays are unchanged): the 4-ary layout of cf_rrrw_quads_* (above) of the BWT (n = view.n), with the
 * per-symbol table holding lfb[c] = C[c] - (where the walk of c from position 0 ends) for c < sigma instead of
 * base[]. Backward search then walks lo and hi through ceil(bits / 2) records per pattern symbol (the line layout:
 * bits), and an LF step of locate one walk; results equal cf_fm_count_async / cf_fm_ranges_async /
 * cf_fm_locate_async for the same view. Layout of `quads`: [L4][nrec][16] records, nrec = n / 208 + 1, then
 * Z [L4][4], then [sigma] int32 lfb. bits <= 24, sigma <= 2^bits (the byte counts are 0 otherwise). The build decodes
 * the BWT from the view into `workspace` (cf_fm_quads_workspace_bytes, 256-byte aligned). */
uint64_t cf_fm_quads_bytes(cf_fm_view v);
uint64_t cf_fm_quads_workspace_bytes(cf_fm_view v);
cf_status cf_fm_quads_build_async(cf_fm_view v, uint32_t *quads, uint64_t bytes, void *workspace,
                                  uint64_t workspace_bytes, void *stream);
cf_status cf_fm_count_quads_async(cf_fm_view v, const uint32_t *quads, const int32_t *pat, const int32_t *pstart,
                                  const int32_t *plen, uint32_t *out, size_t npat, void *stream);
cf_status cf_fm_ranges_quads_async(cf_fm_view v, const uint32_t *quads, const int32_t *pat, const int32_t *pstart,
                                   const int32_t *plen, int32_t *lo_out, int32_t *hi_out, size_t npat, void *stream);
cf_status cf_fm_locate_quads_async(cf_fm_view v, const uint32_t *quads, const int32_t *r_in, int32_t *out,
                                   size_t nocc, void *stream);

/* ---- on-disk formats: .cfrw v1 and .cffm v1 (host files; host arrays) ----
 * Byte-compatible with the reference writer (tools/build_index.cpp:413-438 and 496-526; exporter docstrings
 * tools/export_rrr_wavelet.py:11-19, tools/export_fm_index.py:19-29): magic, version 1, little-endian header
 * scalars without padding, then the arrays back to back. The files also carry the benchmark's query and golden
 * sections (counts may be 0). No counterpart in the reference C ABI (its reader/writers are its tools and test
 * drivers). Readers validate magic, version and the exact file size implied by the header; read into caller-owned
 * host arrays sized from the header (cf_rrrw_arrays then holds HOST pointers). */
typedef struct cf_rrrw_file_header {
  uint64_t n, rrr_bytes, packed_bytes;
  uint32_t bits, vocab, nblocks, nsb, cwords, na, owords;
  uint32_t nq, nr; /* access queries (pos, golden) and rank queries (c, i, golden) in the file */
  float h0;
} cf_rrrw_file_header;

typedef struct cf_rrrw_file_queries { /* host arrays: [nq] / [nr]; may be NULL when the count is 0 */
  uint32_t *pos, *access_golden, *rank_c, *rank_i, *rank_golden;
} cf_rrrw_file_queries;

cf_status cf_rrrw_file_read_header(const char *path, cf_rrrw_file_header *header);
cf_status cf_rrrw_file_read(const char *path, const cf_rrrw_file_header *header, const cf_rrrw_arrays *host_arrays,
                            const cf_rrrw_file_queries *queries);
cf_status cf_rrrw_file_write(const char *path, const cf_rrrw_file_header *header, const cf_rrrw_arrays *host_arrays,
                             const cf_rrrw_file_queries *queries);

typedef struct cf_fm_file_header {
  uint64_t n, rrr_bytes;
  uint32_t bits, vocab, sigma, nblocks, nsb, cwords, na, owords, sa_sample;
  uint32_t mwords, msb, nsval;    /* mark plane words, mark directory entries, sampled SA values */
  uint32_t npat, patflat, nloc;   /* pattern section: patterns, flattened symbols, located occurrences */
  uint32_t reserved;              /* 0 (not in the file) */
} cf_fm_file_header;

typedef struct cf_fm_file_arrays { /* host arrays sized from the header */
  int32_t *C;              /* [sigma] */
  uint32_t *mwords;        /* [mwords] */
  int32_t *msb;            /* [msb] */
  int32_t *sval;           /* [nsval] */
  int32_t *pat;            /* [patflat] symbols + 1, as the reference writes them */
  int32_t *pstart, *plen;  /* [npat] */
  uint32_t *count_golden;  /* [npat] */
  int32_t *locoff;         /* [npat + 1] */
  int32_t *locpos;         /* [nloc] */
} cf_fm_file_arrays;

cf_status cf_fm_file_read_header(const char *path, cf_fm_file_header *header);
cf_status cf_fm_file_read(const char *path, const cf_fm_file_header *header, const cf_rrrw_arrays *host_wavelet,
                          const cf_fm_file_arrays *host_arrays);
cf_status cf_fm_file_write(const char *path, const cf_fm_file_header *header, const cf_rrrw_arrays *host_wavelet,
                           const cf_fm_file_arrays *host_arrays);

#ifdef __cplusplus
} /* extern "C" */

#include <vector>
/* reference src/cuda/suffix_array.cu:42 (C++ linkage, host vectors, allocates and synchronises) */
void cf_gpu_suffix_array(const std::vector<int> &s, std::vector<int> &out);
#endif

#endif /* CHROMOFOLD_INDEX_H */
