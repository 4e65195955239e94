// qw_internal.hpp — the rANS codec's half of cf_qw_matmul_async (qw_rans.hip), called by qw_matmul.hip after the
// descriptor checks shared by both codecs.
#pragma once

#include <hip/hip_runtime.h>

#include "chromofold/chromofold_qw.h"

namespace cfqw {

// Codec-specific descriptor checks of a CF_QW_CODEC_RANS matrix (host only, no device access).
cf_status rans_validate(const cf_qw_matrix *w);

// y[b, :] for b < batch on `s` (the descriptor already validated).
cf_status rans_matmul(const cf_qw_matrix *w, const uint16_t *x, float *y, uint32_t batch, hipStream_t s);

}  // namespace cfqw
