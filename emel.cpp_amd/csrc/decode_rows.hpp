// Per-row chunked prefill through the decode kernel (attn_decode.hip), used
// for the head size the MFMA prefill kernel does not take (512).
#pragma once

#include <hip/hip_runtime.h>

#include "emelk.h"
#include "pool_layout.hpp"

namespace emelk {

emel_error_type decode_rows(const pool_layout &L, const void *k_pool, const void *v_pool,
                            int32_t layer, const float *q, float *out, int32_t n_seq, int32_t n_q,
                            const int32_t *q_start, const uint16_t *block_tables,
                            int32_t table_stride, float scale, hipStream_t st);

}  // namespace emelk
