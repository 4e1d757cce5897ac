// q8_0 block quantizer shared by the append kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>

#include "device_common.hpp"

namespace emelk::dev {

// One 32-value block as quantize_row_q8_0_strided
// (kernel/detail.hpp:804-824) bit for bit: d = amax/127 with IEEE division,
// inv_d = 1/d (0 when d == 0), q = clamp(roundf(x*inv_d), -127, 127), the
// scale stored as fp16(d) RNE.  hipcc keeps fp32 division correctly rounded
// unless fast-math is requested, and no flag here requests it.
__device__ __forceinline__ void quantize_block32(const float *__restrict__ x, int8_t *qs_out,
                                                 uint16_t &d_out) {
  float v[32];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float4_t f = reinterpret_cast<const float4_t *>(x)[j];
    v[4 * j + 0] = f.x;
    v[4 * j + 1] = f.y;
    v[4 * j + 2] = f.z;
    v[4 * j + 3] = f.w;
  }
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(v[j]));
  const float d = amax / 127.0f;
  const float inv_d = d != 0.0f ? 1.0f / d : 0.0f;
  d_out = f32_to_f16_bits(d);
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    const float prod = v[j] * inv_d;
    int q = static_cast<int>(roundf(prod));
    q = q < -127 ? -127 : (q > 127 ? 127 : q);
    qs_out[j] = static_cast<int8_t>(q);
  }
}

}  // namespace emelk::dev
