// TEST INFRASTRUCTURE ONLY — never part of the product path.
//
// Thin extern "C" shim over the reference's own std-only kernel header,
// compiled where it lies (-I /root/reference/src -I /root/reference/include)
// into oracle/_ref/libemelref.so.  It lets the tests and the golden-vector
// generator pin this repository's C restatement (oracle/oracle.c) against the
// reference's arithmetic bit for bit.  Nothing here is copied: every function
// forwards to the reference header.
//
// Reference functions reached (paths relative to /root/reference):
//   quant::fp32_to_fp16 / fp16_to_fp32        src/emel/kernel/detail.hpp:350-392
//   quantize_row_q8_0_strided                 src/emel/kernel/detail.hpp:804-824
//   dequantize_row_q8_0                       src/emel/kernel/detail.hpp:679-690
//   dot_product_f32_f16_scores                src/emel/kernel/detail.hpp:2211-2245
//   dot_product_ggml_f16_scores(float,float)  src/emel/kernel/detail.hpp:2085-2152
//   exp_and_sum_ggml_f32                      src/emel/kernel/detail.hpp:2055-2083
//   round_fp16_weight                         src/emel/kernel/detail.hpp:4258-4260
//   run_flash_attn_ext_active_kv_with_workspace_unchecked
//                                             src/emel/kernel/detail.hpp:5238-5291
#include <cstdint>
#include <cstring>
#include <memory>

#include "emel/kernel/events.hpp"

namespace kd = emel::kernel::detail;
namespace ke = emel::kernel::event;

extern "C" {

uint16_t ref_fp32_to_fp16(float v) { return kd::quant::fp32_to_fp16(v); }
float ref_fp16_to_fp32(uint16_t h) { return kd::quant::fp16_to_fp32(h); }

// FNV-1a fold of fp32_to_fp16 over the bit patterns [lo, hi) (exhaustive sweep).
uint64_t ref_fp32_to_fp16_sweep(uint64_t lo, uint64_t hi) {
  uint64_t acc = 0;
  for (uint64_t b = lo; b < hi; ++b) {
    const uint32_t bits = static_cast<uint32_t>(b);
    float f;
    std::memcpy(&f, &bits, 4);
    acc = (acc ^ kd::quant::fp32_to_fp16(f)) * 1099511628211ull;
  }
  return acc;
}

void ref_quantize_row_q8_0(const float *x, uint64_t stride, void *y, int64_t k) {
  kd::quant::quantize_row_q8_0_strided(x, stride, static_cast<kd::quant::block_q8_0 *>(y), k);
}

void ref_dequantize_row_q8_0(const void *x, float *y, int64_t k) {
  kd::quant::dequantize_row_q8_0(static_cast<const kd::quant::block_q8_0 *>(x), y, k);
}

uint64_t ref_sizeof_block_q8_0() { return sizeof(kd::quant::block_q8_0); }

float ref_dot_f32_f16(const float *lhs, const uint16_t *rhs, uint64_t n) {
  return kd::dot_product_f32_f16_scores(lhs, rhs, n);
}

float ref_dot_f32_f32_f16r(const float *lhs, const float *rhs, uint64_t n) {
  return kd::dot_product_ggml_f16_scores(lhs, rhs, n);
}

double ref_exp_and_sum(const float *src, float *dst, uint64_t n, float max_value) {
  return kd::exp_and_sum_ggml_f32(src, dst, n, max_value);
}

float ref_round_fp16_weight(float v) { return kd::round_fp16_weight(v); }

// Scalar flash decode (f16 accumulator) over a head-major f16 K/V buffer:
// k/v are [n_head_kv][kv_stride_tokens][head_dim]; q and out are
// [n_head][head_dim].
int ref_flash_attn_f16acc(const float *q, const uint16_t *k, const uint16_t *v,
                          uint64_t head_dim, uint64_t n_head, uint64_t n_head_kv,
                          uint64_t kv_tokens, uint64_t kv_stride_tokens,
                          float scale, uint32_t masked_total_tokens, float *out) {
  ke::op_flash_attn_ext request{};
  request.src0.data = q;
  request.src0.type = ke::dtype::f32;
  request.src0.ne = {head_dim, 1, n_head, 1};
  request.src0.nb = {4, 4 * head_dim, 4 * head_dim, 4 * head_dim * n_head};
  request.src1.data = k;
  request.src1.type = ke::dtype::f16;
  request.src1.ne = {head_dim, kv_tokens, n_head_kv, 1};
  request.src1.nb = {2, 2 * head_dim, 2 * head_dim * kv_stride_tokens,
                     2 * head_dim * kv_stride_tokens * n_head_kv};
  request.src2 = request.src1;
  request.src2.data = v;
  request.dst.data = out;
  request.dst.type = ke::dtype::f32;
  request.dst.ne = {head_dim, 1, n_head, 1};
  request.dst.nb = {4, 4 * head_dim, 4 * head_dim, 4 * head_dim * n_head};
  std::memcpy(request.op_params.data(), &scale, sizeof(scale));
  std::memcpy(request.op_params.data() + sizeof(scale), &masked_total_tokens,
              sizeof(masked_total_tokens));
  request.op_params_size = sizeof(scale) + sizeof(masked_total_tokens);
  auto workspace = std::make_unique<kd::flash_attn_workspace>();
  if (!kd::can_run_flash_attn_ext_with_workspace(request, *workspace)) {
    return 0;
  }
  kd::run_flash_attn_ext_active_kv_with_workspace_unchecked(request, *workspace);
  return 1;
}

}  // extern "C"
