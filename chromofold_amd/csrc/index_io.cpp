// index_io.cpp — the reference's on-disk index formats, .cfrw v1 and .cffm v1, read and written by the library.
//
// Layouts follow the reference writer field for field (tools/build_index.cpp:413-438 for .cfrw, :496-526 for
// .cffm; the same as the exporter docstrings tools/export_rrr_wavelet.py:11-19 and tools/export_fm_index.py:19-29):
// a 4-byte magic, little-endian scalars with no padding, then the arrays back to back. Besides the index both
// formats carry the benchmark's query and golden sections; the library keeps them so a file round-trips byte for
// byte, and they may be empty (count 0) in files it writes. Readers check the magic, the version and that the file
// size equals what the header implies before anything is copied.
#include <cstdio>
#include <cstring>
#include <vector>

#include "chromofold/chromofold_index.h"

static_assert(sizeof(cf_rrrw_file_header) == 64, "no padding: headers are compared byte for byte");
static_assert(sizeof(cf_fm_file_header) == 80, "no padding: headers are compared byte for byte");

namespace {

struct File {
  FILE *f = nullptr;
  explicit File(const char *path, const char *mode) : f(std::fopen(path, mode)) {}
  ~File() {
    if (f) std::fclose(f);
  }
  File(const File &) = delete;
  File &operator=(const File &) = delete;
};

template <typename T>
bool put(FILE *f, const T &v) {
  return std::fwrite(&v, sizeof v, 1, f) == 1;
}

bool put_array(FILE *f, const void *p, uint64_t count, size_t elem) {
  if (count == 0) return true;
  if (!p) return false;
  return std::fwrite(p, elem, count, f) == count;
}

template <typename T>
bool get(FILE *f, T *v) {
  return std::fread(v, sizeof *v, 1, f) == 1;
}

bool get_array(FILE *f, void *p, uint64_t count, size_t elem) {
  if (count == 0) return true;
  if (!p) return false;
  return std::fread(p, elem, count, f) == count;
}

long file_size(FILE *f) {
  const long at = std::ftell(f);
  if (std::fseek(f, 0, SEEK_END) != 0) return -1;
  const long size = std::ftell(f);
  std::fseek(f, at, SEEK_SET);
  return size;
}

// bytes of the arrays that follow a .cfrw header
uint64_t cfrw_payload(const cf_rrrw_file_header &h) {
  const uint64_t b = h.bits;
  return 4 * b * h.cwords + 4ull * h.owords + 4 * b * h.na + 2 * b * (h.nsb + 1ull) + 4 * b * h.na +
         2 * b * (h.nsb + 1ull) + 4 * b + 4 * b + 4ull * h.nq * 2 + 4ull * h.nr * 3;
}

constexpr uint64_t kCfrwHeader = 4 + 4 + 8 + 4 * 9 + 8 + 8 + 4;  // magic .. h0

uint64_t cffm_payload(const cf_fm_file_header &h) {
  const uint64_t b = h.bits;
  return 4 * b * h.cwords + 4ull * h.owords + 4 * b * h.na + 2 * b * (h.nsb + 1ull) + 4 * b * h.na +
         2 * b * (h.nsb + 1ull) + 4 * b + 4 * b + 4ull * h.sigma + 4ull * h.mwords + 4ull * h.msb + 4ull * h.nsval +
         4ull * h.patflat + 4ull * h.npat * 3 + 4ull * (h.npat + 1ull) + 4ull * h.nloc;
}

constexpr uint64_t kCffmHeader = 4 + 4 + 8 + 4 * 15 + 8;  // magic, version, n, 15 u32 fields, rrr_bytes

bool header_ok(uint32_t bits, uint32_t cwords, uint64_t n) { return bits >= 1 && bits <= 31 && cwords > 0 && n > 0; }

bool write_wavelet(FILE *f, uint32_t bits, uint32_t cwords, uint32_t owords, uint32_t na, uint32_t nsb,
                   const cf_rrrw_arrays *w) {
  const uint64_t b = bits;
  return put_array(f, w->classes, b * cwords, 4) && put_array(f, w->offsets, owords, 4) &&
         put_array(f, w->rank_a, b * na, 4) && put_array(f, w->rank_d, b * (nsb + 1ull), 2) &&
         put_array(f, w->off_a, b * na, 4) && put_array(f, w->off_d, b * (nsb + 1ull), 2) &&
         put_array(f, w->offbase, b, 4) && put_array(f, w->zeros, b, 4);
}

bool read_wavelet(FILE *f, uint32_t bits, uint32_t cwords, uint32_t owords, uint32_t na, uint32_t nsb,
                  const cf_rrrw_arrays *w) {
  const uint64_t b = bits;
  return get_array(f, w->classes, b * cwords, 4) && get_array(f, w->offsets, owords, 4) &&
         get_array(f, w->rank_a, b * na, 4) && get_array(f, w->rank_d, b * (nsb + 1ull), 2) &&
         get_array(f, w->off_a, b * na, 4) && get_array(f, w->off_d, b * (nsb + 1ull), 2) &&
         get_array(f, w->offbase, b, 4) && get_array(f, w->zeros, b, 4);
}

}  // namespace

extern "C" cf_status cf_rrrw_file_read_header(const char *path, cf_rrrw_file_header *h) {
  if (!path || !h) return CF_ERR_INVALID_ARGUMENT;
  File file(path, "rb");
  if (!file.f) return CF_ERR_INVALID_ARGUMENT;
  char magic[4];
  uint32_t version = 0;
  cf_rrrw_file_header r{};
  if (!get(file.f, &magic) || std::memcmp(magic, "CFRW", 4) != 0 || !get(file.f, &version) || version != 1)
    return CF_ERR_INVALID_ARGUMENT;
  if (!get(file.f, &r.n) || !get(file.f, &r.bits) || !get(file.f, &r.vocab) || !get(file.f, &r.nblocks) ||
      !get(file.f, &r.nsb) || !get(file.f, &r.cwords) || !get(file.f, &r.na) || !get(file.f, &r.owords) ||
      !get(file.f, &r.nq) || !get(file.f, &r.nr) || !get(file.f, &r.rrr_bytes) || !get(file.f, &r.packed_bytes) ||
      !get(file.f, &r.h0))
    return CF_ERR_INVALID_ARGUMENT;
  if (!header_ok(r.bits, r.cwords, r.n) || file_size(file.f) != static_cast<long>(kCfrwHeader + cfrw_payload(r)))
    return CF_ERR_INVALID_ARGUMENT;
  *h = r;
  return CF_OK;
}

extern "C" cf_status cf_rrrw_file_read(const char *path, const cf_rrrw_file_header *h, const cf_rrrw_arrays *w,
                                       const cf_rrrw_file_queries *q) {
  if (!path || !h || !w) return CF_ERR_INVALID_ARGUMENT;
  cf_rrrw_file_header check{};
  const cf_status st = cf_rrrw_file_read_header(path, &check);
  if (st != CF_OK) return st;
  if (std::memcmp(&check, h, sizeof check) != 0) return CF_ERR_INVALID_ARGUMENT;  // the caller sized from this header
  if ((h->nq || h->nr) && !q) return CF_ERR_INVALID_ARGUMENT;
  File file(path, "rb");
  if (!file.f || std::fseek(file.f, static_cast<long>(kCfrwHeader), SEEK_SET) != 0) return CF_ERR_INVALID_ARGUMENT;
  if (!read_wavelet(file.f, h->bits, h->cwords, h->owords, h->na, h->nsb, w)) return CF_ERR_INVALID_ARGUMENT;
  if (h->nq || h->nr) {
    if (!get_array(file.f, q->pos, h->nq, 4) || !get_array(file.f, q->access_golden, h->nq, 4) ||
        !get_array(file.f, q->rank_c, h->nr, 4) || !get_array(file.f, q->rank_i, h->nr, 4) ||
        !get_array(file.f, q->rank_golden, h->nr, 4))
      return CF_ERR_INVALID_ARGUMENT;
  }
  return CF_OK;
}

extern "C" cf_status cf_rrrw_file_write(const char *path, const cf_rrrw_file_header *h, const cf_rrrw_arrays *w,
                                        const cf_rrrw_file_queries *q) {
  if (!path || !h || !w || !header_ok(h->bits, h->cwords, h->n) || ((h->nq || h->nr) && !q))
    return CF_ERR_INVALID_ARGUMENT;
  File file(path, "wb");
  if (!file.f) return CF_ERR_INVALID_ARGUMENT;
  const uint32_t version = 1;
  bool ok = std::fwrite("CFRW", 1, 4, file.f) == 4 && put(file.f, version) && put(file.f, h->n) &&
            put(file.f, h->bits) && put(file.f, h->vocab) && put(file.f, h->nblocks) && put(file.f, h->nsb) &&
            put(file.f, h->cwords) && put(file.f, h->na) && put(file.f, h->owords) && put(file.f, h->nq) &&
            put(file.f, h->nr) && put(file.f, h->rrr_bytes) && put(file.f, h->packed_bytes) && put(file.f, h->h0);
  ok = ok && write_wavelet(file.f, h->bits, h->cwords, h->owords, h->na, h->nsb, w);
  if (ok && (h->nq || h->nr))
    ok = put_array(file.f, q->pos, h->nq, 4) && put_array(file.f, q->access_golden, h->nq, 4) &&
         put_array(file.f, q->rank_c, h->nr, 4) && put_array(file.f, q->rank_i, h->nr, 4) &&
         put_array(file.f, q->rank_golden, h->nr, 4);
  ok = ok && std::fflush(file.f) == 0;
  return ok ? CF_OK : CF_ERR_INVALID_ARGUMENT;
}

extern "C" cf_status cf_fm_file_read_header(const char *path, cf_fm_file_header *h) {
  if (!path || !h) return CF_ERR_INVALID_ARGUMENT;
  File file(path, "rb");
  if (!file.f) return CF_ERR_INVALID_ARGUMENT;
  char magic[4];
  uint32_t version = 0;
  cf_fm_file_header r{};
  r.reserved = 0;
  if (!get(file.f, &magic) || std::memcmp(magic, "CFFM", 4) != 0 || !get(file.f, &version) || version != 1)
    return CF_ERR_INVALID_ARGUMENT;
  if (!get(file.f, &r.n) || !get(file.f, &r.bits) || !get(file.f, &r.vocab) || !get(file.f, &r.sigma) ||
      !get(file.f, &r.nblocks) || !get(file.f, &r.nsb) || !get(file.f, &r.cwords) || !get(file.f, &r.na) ||
      !get(file.f, &r.owords) || !get(file.f, &r.sa_sample) || !get(file.f, &r.mwords) || !get(file.f, &r.msb) ||
      !get(file.f, &r.nsval) || !get(file.f, &r.npat) || !get(file.f, &r.patflat) || !get(file.f, &r.nloc) ||
      !get(file.f, &r.rrr_bytes))
    return CF_ERR_INVALID_ARGUMENT;
  if (!header_ok(r.bits, r.cwords, r.n) || file_size(file.f) != static_cast<long>(kCffmHeader + cffm_payload(r)))
    return CF_ERR_INVALID_ARGUMENT;
  *h = r;
  return CF_OK;
}

extern "C" cf_status cf_fm_file_read(const char *path, const cf_fm_file_header *h, const cf_rrrw_arrays *w,
                                     const cf_fm_file_arrays *fm) {
  if (!path || !h || !w || !fm) return CF_ERR_INVALID_ARGUMENT;
  cf_fm_file_header check{};
  const cf_status st = cf_fm_file_read_header(path, &check);
  if (st != CF_OK) return st;
  if (std::memcmp(&check, h, sizeof check) != 0) return CF_ERR_INVALID_ARGUMENT;
  File file(path, "rb");
  if (!file.f || std::fseek(file.f, static_cast<long>(kCffmHeader), SEEK_SET) != 0) return CF_ERR_INVALID_ARGUMENT;
  const bool ok = read_wavelet(file.f, h->bits, h->cwords, h->owords, h->na, h->nsb, w) &&
                  get_array(file.f, fm->C, h->sigma, 4) && get_array(file.f, fm->mwords, h->mwords, 4) &&
                  get_array(file.f, fm->msb, h->msb, 4) && get_array(file.f, fm->sval, h->nsval, 4) &&
                  get_array(file.f, fm->pat, h->patflat, 4) && get_array(file.f, fm->pstart, h->npat, 4) &&
                  get_array(file.f, fm->plen, h->npat, 4) && get_array(file.f, fm->count_golden, h->npat, 4) &&
                  get_array(file.f, fm->locoff, h->npat + 1ull, 4) && get_array(file.f, fm->locpos, h->nloc, 4);
  return ok ? CF_OK : CF_ERR_INVALID_ARGUMENT;
}

extern "C" cf_status cf_fm_file_write(const char *path, const cf_fm_file_header *h, const cf_rrrw_arrays *w,
                                      const cf_fm_file_arrays *fm) {
  if (!path || !h || !w || !fm || !header_ok(h->bits, h->cwords, h->n)) return CF_ERR_INVALID_ARGUMENT;
  File file(path, "wb");
  if (!file.f) return CF_ERR_INVALID_ARGUMENT;
  const uint32_t version = 1;
  // with no pattern section the offsets array still has its one entry (npat + 1), 0
  const int32_t zero = 0;
  const int32_t *locoff = (h->npat == 0 && !fm->locoff) ? &zero : fm->locoff;
  bool ok = std::fwrite("CFFM", 1, 4, file.f) == 4 && put(file.f, version) && put(file.f, h->n) &&
            put(file.f, h->bits) && put(file.f, h->vocab) && put(file.f, h->sigma) && put(file.f, h->nblocks) &&
            put(file.f, h->nsb) && put(file.f, h->cwords) && put(file.f, h->na) && put(file.f, h->owords) &&
            put(file.f, h->sa_sample) && put(file.f, h->mwords) && put(file.f, h->msb) && put(file.f, h->nsval) &&
            put(file.f, h->npat) && put(file.f, h->patflat) && put(file.f, h->nloc) && put(file.f, h->rrr_bytes);
  ok = ok && write_wavelet(file.f, h->bits, h->cwords, h->owords, h->na, h->nsb, w) &&
       put_array(file.f, fm->C, h->sigma, 4) && put_array(file.f, fm->mwords, h->mwords, 4) &&
       put_array(file.f, fm->msb, h->msb, 4) && put_array(file.f, fm->sval, h->nsval, 4) &&
       put_array(file.f, fm->pat, h->patflat, 4) && put_array(file.f, fm->pstart, h->npat, 4) &&
       put_array(file.f, fm->plen, h->npat, 4) && put_array(file.f, fm->count_golden, h->npat, 4) &&
       put_array(file.f, locoff, h->npat + 1ull, 4) && put_array(file.f, fm->locpos, h->nloc, 4) &&
       std::fflush(file.f) == 0;
  return ok ? CF_OK : CF_ERR_INVALID_ARGUMENT;
}
