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

#ifdef __cplusplus
} /* extern "C" */

#include <vector>
/* reference src/cuda/suffix_array.cu:42 (C++ linkage, host vectors, allocates and synchronises) */
void cf_gpu_suffix_array(const std::vector<int> &s, std::vector<int> &out);
#endif

#endif /* CHROMOFOLD_INDEX_H */
