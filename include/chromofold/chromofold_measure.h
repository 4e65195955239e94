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

/* Read `bytes` bytes of device memory at `src` once (16-byte loads, every byte read exactly once, no writes but one
 * 32-bit XOR of all data per workgroup into *sink, which keeps the loads alive). src 16-byte aligned, bytes a
 * multiple of 16; sink device memory. Asynchronous on `stream`; allocates nothing. The achieved read bandwidth is
 * bytes / kernel time. */
cf_status cf_stream_read_async(const void *src, uint64_t bytes, uint32_t *sink, void *stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* CHROMOFOLD_MEASURE_H */
