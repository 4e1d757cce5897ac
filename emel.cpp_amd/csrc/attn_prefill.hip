// Chunked-prefill attention (MFMA) — not built yet: the entry point fails
// loudly so no caller can mistake it for a working path.
#include "emelk.h"

extern "C" emel_error_type emelk_attn_prefill_chunk(const emelk_kv_geometry *, const void *,
                                                    const void *, int32_t, const float *, float *,
                                                    int32_t, int32_t, const int32_t *,
                                                    const uint16_t *, int32_t, float, void *) {
  return EMELK_ERR_BACKEND;
}
