/* chromofold_measure.h — ADDITIVE measurement helpers. No counterpart in the reference: these kernels exist only to
 * measure the device, so that the decode kernels' HBM figures can be quoted against what the chip sustains as well
 * as against its nominal peak. */
#ifndef CHROMOFOLD_MEASURE_H
#define CHROMOFOLD_MEASURE_H

#include <stddef.h>
#include <stdint.h>

#include "chromofold/chromofold.h"

#ifdef __cplusplus
extern "C" {
#endif

/* The fixed key of the measurement kernels' folds (below). */
#define CF_MEASURE_FOLD_KEY 0x2545F491u

/* Read `bytes` bytes of device memory at `src` once (16-byte non-temporal loads, one workgroup per 64 KiB chunk,
 * every byte read exactly once). Each workgroup folds its chunk into a 32-bit XOR of its 32-bit words and stores it
 * to *sink only when it equals CF_MEASURE_FOLD_KEY: that keeps the loads alive without an atomic per workgroup, and
 * for ordinary data the sink is left as it was. src 16-byte aligned, bytes a multiple of 16; sink device memory. Asynchronous on `stream`; allocates
 * nothing. The achieved read bandwidth is bytes / kernel time. */
cf_status cf_stream_read_async(const void *src, uint64_t bytes, uint32_t *sink, void *stream);

/* Cache bandwidth: `passes` passes over `bytes` at `src` with ordinary 16-byte loads, each pass giving every
 * workgroup another workgroup's chunk on the same XCD (so after the first pass the data comes from that XCD's L2,
 * or from the Infinity Cache when `bytes` exceeds the L2s, and never from the CU's own L1). Achieved rate =
 * passes * bytes / kernel time. Same argument rules as cf_stream_read_async; passes >= 1. */
cf_status cf_cache_read_async(const void *src, uint64_t bytes, uint32_t passes, uint32_t *sink, void *stream);

/* LDS bandwidth: two workgroups per CU each fill 64 KiB of LDS and read it `passes` times with conflict-free
 * 16-byte reads; cf_lds_read_bytes(passes) is the bytes read per launch (on the current device). */
cf_status cf_lds_read_async(uint32_t passes, uint32_t *sink, void *stream);
uint64_t cf_lds_read_bytes(uint32_t passes);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* CHROMOFOLD_MEASURE_H */
