// The step before append, fused into one launch: optional head-wise RMS
// norm of q and k, optional RMS norm of v, RoPE of q and k, and the append
// of k and v into the paged pool (f16 or q8_0).  Restates the part of
// compute_layer_attention_residual between the Q/K/V projections and
// store_attention_kv_cache (text/generator/detail.hpp:3806-3825) and the same
// steps of the chunked-prefill row loop (detail.hpp:4335-4360).
//
// Every product and sum is evaluated unfused in the reference's order
// (floating-point contraction is off for this whole file), and division and
// square root are the correctly rounded IEEE ones (hipcc's default
// -fhip-fp32-correctly-rounded-divide-sqrt; __fsqrt_rn would be the native,
// 1-ulp v_sqrt_f32), so the results are bit-exact against that arithmetic.  cos/sin come from a
// table built on the host with the reference's recurrence.
//
// Launch: one workgroup of 4 waves per (token, group of 4 rows), where the
// rows of a token are its n_head q heads, n_head_kv k heads and n_head_kv v
// heads.  A wave stages its row of head_dim floats in its own slice of LDS,
// so it needs no workgroup barrier, and requests the row together with the
// token's position.  This is a few KB per token: latency, not bandwidth,
// bounds it.
#include <hip/hip_runtime.h>

#include <cmath>
#include <new>
#include <vector>

#include "device_common.hpp"
#include "emelk.h"
#include "pool_layout.hpp"
#include "q8_device.hpp"

#pragma clang fp contract(off)

struct emelk_rope_table {
  emelk_rope_params params;
  int32_t head_dim = 0;
  int32_t pair_count = 0;
  int32_t x1_base = 0;
  int32_t max_positions = 0;
  float2 *dev = nullptr;  // [max_positions][pair_count] (cos, sin)
};

namespace emelk {
namespace {

using namespace emelk::dev;

constexpr int k_rows_per_wg = 4;
// rope_append_rows_kernel: rows per wave, and the launch size (rows) from
// which it replaces rope_append_kernel
#ifndef EMELK_ROPE_RPW
#define EMELK_ROPE_RPW 4
#endif
constexpr int k_rows_per_wave = EMELK_ROPE_RPW;
constexpr int64_t k_rows_kernel_min = 1 << 16;
constexpr int k_max_dim = 512;

struct rope_append_args {
  pool_layout L;
  uint8_t *k_pool;
  uint8_t *v_pool;
  int32_t layer;
  const float *q_in;
  float *q_out;
  const float *k_rows;
  const float *v_rows;
  int32_t n_seq;
  int32_t n_tokens;
  const int32_t *positions;
  const uint16_t *tables;
  int32_t table_stride;
  const float2 *rope;
  int32_t rope_positions;
  int32_t pair_count;
  int32_t x0_stride;
  int32_t x1_stride;
  int32_t x1_base;
  const float *q_norm;
  const float *k_norm;
  int32_t v_rms;
  float eps;
};

__global__ __launch_bounds__(k_rows_per_wg *k_wave) void rope_append_kernel(rope_append_args A) {
  __shared__ __align__(16) float s_row[k_rows_per_wg][k_max_dim];  // float4 reads (q8_0)
  __shared__ float s_scale[k_rows_per_wg];

  const pool_layout &L = A.L;
  const int32_t D = L.head_dim;
  const int32_t s = blockIdx.x / A.n_tokens;
  const int32_t t = blockIdx.x % A.n_tokens;
  const int32_t wave = threadIdx.x / k_wave;
  const int32_t lane = threadIdx.x % k_wave;
  const int32_t row = blockIdx.y * k_rows_per_wg + wave;
  const int32_t n_rows = L.n_head + 2 * L.n_head_kv;
  const bool have = row < n_rows;
  const int32_t kind = row < L.n_head ? 0 : (row < L.n_head + L.n_head_kv ? 1 : 2);
  const int32_t head = kind == 0 ? row : (kind == 1 ? row - L.n_head : row - L.n_head - L.n_head_kv);
  const uint64_t tok = static_cast<uint64_t>(s) * A.n_tokens + t;
  // The row is requested together with the position (two floats per lane
  // per 128 dims), before the token's validity is known.
  constexpr int NC = k_max_dim / (2 * k_wave);
  float2 x[NC];
  if (have) {
    const float *src =
        kind == 0 ? A.q_in + (tok * L.n_head + head) * static_cast<uint64_t>(D)
                  : (kind == 1 ? A.k_rows : A.v_rows) + (tok * L.n_head_kv + head) * static_cast<uint64_t>(D);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int32_t d = 2 * (lane + c * k_wave);
      if (d < D) x[c] = *reinterpret_cast<const float2 *>(src + d);
    }
  }
  const int32_t pos = A.positions[s] + t;
  // An invalid token (no position, outside the rope table, past the table
  // row or on an invalid page) writes nothing, q included.
  if (pos < 0) return;
  if (A.pair_count > 0 && pos >= A.rope_positions) return;
  // the (cos, sin) of the lane's pairs, requested with the page
  constexpr int NP = k_max_dim / (2 * k_wave);
  float2 cs[NP];
  if (have && kind < 2) {
#pragma unroll
    for (int c = 0; c < NP; ++c) {
      const int32_t pr = lane + c * k_wave;
      if (pr < A.pair_count) cs[c] = A.rope[static_cast<uint64_t>(pos) * A.pair_count + pr];
    }
  }
  const int32_t lb = pos / L.block_tokens;
  if (lb >= A.table_stride) return;
  const uint32_t page = A.tables[static_cast<uint64_t>(s) * A.table_stride + lb];
  if (page >= static_cast<uint32_t>(L.max_blocks)) return;
  const int32_t slot = pos % L.block_tokens;
  if (!have) return;  // uniform per wave; nothing below synchronises across waves
  // Each wave stages only its own row (and its s_scale), so ordering its
  // own LDS operations is all the synchronisation needed.
  auto wave_sync = []() {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
  };
  float *buf = s_row[wave];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int32_t d = 2 * (lane + c * k_wave);
    if (d < D) *reinterpret_cast<float2 *>(buf + d) = x[c];
  }
  wave_sync();

  // Norm scale, computed by one lane in the reference's summation order.
  const float *wt = kind == 0 ? A.q_norm : (kind == 1 ? A.k_norm : nullptr);
  const bool head_norm = kind < 2 && wt != nullptr;
  const bool v_norm = kind == 2 && A.v_rms != 0;
  if (lane == 0 && head_norm) {
    // apply_headwise_rms_norm (detail.hpp:1073-1082)
    float ss = 0.0f;
    for (int32_t d = 0; d < D; ++d) ss += buf[d] * buf[d];
    s_scale[wave] = 1.0f / sqrtf(ss / static_cast<float>(D) + A.eps);
  }
  if (v_norm) {  // uniform per wave
    // apply_rms_norm_in_place (detail.hpp:1098-1106) over the token's whole
    // v, summed in its order: the wave loads 64 values per coalesced load
    // (8 chunks ahead) and every lane adds the squares one by one, each
    // taken from its lane with readlane
    const float *v = A.v_rows + tok * L.n_head_kv * static_cast<uint64_t>(D);
    const int32_t n = L.n_head_kv * D;
    constexpr int kC = 8;
    double ss = 0.0;
    for (int32_t c0 = 0; c0 < n; c0 += kC * k_wave) {
      float sq[kC];
#pragma unroll
      for (int u = 0; u < kC; ++u) {
        const int32_t i = c0 + u * k_wave + lane;
        const float x = i < n ? v[i] : 0.0f;
        sq[u] = x * x;
      }
#pragma unroll
      for (int u = 0; u < kC; ++u) {
        const int32_t left = n - (c0 + u * k_wave);
        if (left <= 0) break;  // uniform
        const double dq = static_cast<double>(sq[u]);
        if (left >= k_wave) {  // a full chunk: lane indices known at compile time
#pragma unroll
          for (int j = 0; j < k_wave; ++j) {
            const int lo = __builtin_amdgcn_readlane(static_cast<int>(__builtin_bit_cast(uint64_t, dq)), j);
            const int hi = __builtin_amdgcn_readlane(static_cast<int>(__builtin_bit_cast(uint64_t, dq) >> 32), j);
            ss += __builtin_bit_cast(double, (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) |
                                                 static_cast<uint32_t>(lo));
          }
        } else {
          for (int32_t j = 0; j < left; ++j) {
            ss += static_cast<double>(__builtin_bit_cast(
                float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sq[u]), j)));
          }
        }
      }
    }
    const float mean = static_cast<float>(ss / static_cast<double>(n));
    if (lane == 0) s_scale[wave] = 1.0f / sqrtf(mean + A.eps);
  }
  if (head_norm || v_norm) {
    wave_sync();
    const float sc = s_scale[wave];
    if (head_norm) {
      for (int32_t d = lane; d < D; d += k_wave) buf[d] *= sc * wt[d];
    } else {
      for (int32_t d = lane; d < D; d += k_wave) buf[d] *= sc;
    }
    wave_sync();
  }

  // apply_rope_pairing (detail.hpp:2905-2936): lane p rotates pairs p,
  // p + 64, ... (pairs never overlap, so the order does not matter)
  if (kind < 2 && A.pair_count > 0) {
#pragma unroll
    for (int c = 0; c < NP; ++c) {
      const int32_t pr = lane + c * k_wave;
      if (pr >= A.pair_count) break;
      const int32_t d0 = pr * A.x0_stride;
      const int32_t d1 = pr * A.x1_stride + A.x1_base;
      const float x0 = buf[d0];
      const float x1 = buf[d1];
      buf[d0] = x0 * cs[c].x - x1 * cs[c].y;
      buf[d1] = x0 * cs[c].y + x1 * cs[c].x;
    }
    wave_sync();
  }

  if (kind == 0) {
    float *dst = A.q_out + (tok * L.n_head + head) * static_cast<uint64_t>(D);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int32_t d = 2 * (lane + c * k_wave);
      if (d < D) *reinterpret_cast<float2 *>(dst + d) = *reinterpret_cast<const float2 *>(buf + d);
    }
    return;
  }
  uint8_t *region = (kind == 1 ? A.k_pool : A.v_pool) +
                    L.region_offset(A.layer, static_cast<int32_t>(page), head);
  if (L.kv_type == EMELK_KV_F16) {
    // store_fp16_rounded_cache (detail.hpp:3050-3055): RNE per value
    uint32_t *dst = reinterpret_cast<uint32_t *>(region + static_cast<uint64_t>(slot) * D * 2u);
    for (int32_t j = lane; j < D / 2; j += k_wave) dst[j] = as_u32(pack_half2(buf[2 * j], buf[2 * j + 1]));
  } else {
    const int32_t blocks = D / 32;
    if (lane < blocks) {
      int8_t qs[32];
      uint16_t dq;
      quantize_block32(buf + 32 * lane, qs, dq);
      uint4_t *dst = reinterpret_cast<uint4_t *>(region + static_cast<uint64_t>(slot) * D +
                                                 static_cast<uint64_t>(lane) * 32u);
      dst[0] = __builtin_bit_cast(uint4_t, *reinterpret_cast<int8_t(*)[16]>(qs));
      dst[1] = __builtin_bit_cast(uint4_t, *reinterpret_cast<int8_t(*)[16]>(qs + 16));
      reinterpret_cast<uint16_t *>(region + L.scale_plane())[static_cast<uint64_t>(slot) * blocks +
                                                             lane] = dq;
    }
  }
}

// Large launches (a prefill chunk): each wave takes RPW consecutive
// (token, row) pairs, token-major, and requests all of their rows and
// positions, then all of their pages and (cos, sin), before it stages any
// row, so a wave keeps RPW rows in flight instead of one.  Every loop over
// the rows is unrolled (the per-row registers stay registers), and the
// arithmetic per row is that of rope_append_kernel.
// REG: adjacent pairs (d, d + 1), no norms, f16 pool: a lane's two floats
// are exactly its pair, so the row never leaves registers.
template <int D, int RPW, bool REG>
__global__ __launch_bounds__(k_rows_per_wg *k_wave) void rope_append_rows_kernel(rope_append_args A) {
  __shared__ __align__(16) float s_row[k_rows_per_wg][D];  // float4 reads (q8_0)
  __shared__ float s_scale[k_rows_per_wg];
  constexpr int NC = D / (2 * k_wave) > 0 ? D / (2 * k_wave) : 1;  // float2 per lane per row
  const pool_layout &L = A.L;
  const int32_t wave = __builtin_amdgcn_readfirstlane(static_cast<int32_t>(threadIdx.x / k_wave));
  const int32_t lane = threadIdx.x % k_wave;
  const uint32_t n_rows = static_cast<uint32_t>(L.n_head + 2 * L.n_head_kv);
  const uint32_t n_tok = static_cast<uint32_t>(A.n_tokens);
  const uint32_t total = static_cast<uint32_t>(A.n_seq) * n_tok * n_rows;  // < 2^31 (host check)
  const uint32_t base = (blockIdx.x * k_rows_per_wg + static_cast<uint32_t>(wave)) * RPW;
  float *buf = s_row[wave];
  auto wave_sync = []() {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
  };

  uint32_t tok[RPW], seq[RPW];
  int32_t kind[RPW], head[RPW], pos[RPW];
  uint32_t page[RPW];
  bool ok[RPW];
  float2 x[RPW][NC], cs[RPW][NC];
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const uint32_t gr = base + i < total ? base + i : total - 1;  // past the end: a valid address
    tok[i] = gr / n_rows;
    const int32_t row = static_cast<int32_t>(gr - tok[i] * n_rows);
    kind[i] = row < L.n_head ? 0 : (row < L.n_head + L.n_head_kv ? 1 : 2);
    head[i] = kind[i] == 0 ? row : (kind[i] == 1 ? row - L.n_head : row - L.n_head - L.n_head_kv);
    const float *src = kind[i] == 0
                           ? A.q_in + (static_cast<uint64_t>(tok[i]) * L.n_head + head[i]) * D
                           : (kind[i] == 1 ? A.k_rows : A.v_rows) +
                                 (static_cast<uint64_t>(tok[i]) * L.n_head_kv + head[i]) * D;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int32_t d = 2 * (lane + c * k_wave);
      if (d < D) x[i][c] = *reinterpret_cast<const float2 *>(src + d);
    }
    seq[i] = tok[i] / n_tok;
    pos[i] = A.positions[seq[i]] + static_cast<int32_t>(tok[i] - seq[i] * n_tok);
  }
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    // An invalid token (no position, outside the rope table, past the table
    // row or on an invalid page) writes nothing, q included.
    bool v = base + i < total && pos[i] >= 0 &&
             (A.pair_count == 0 || pos[i] < A.rope_positions);
    const int32_t lb = v ? pos[i] / L.block_tokens : 0;
    v = v && lb < A.table_stride;
    page[i] = v ? static_cast<uint32_t>(A.tables[static_cast<uint64_t>(seq[i]) * A.table_stride + lb])
                : 0xFFFFFFFFu;
    ok[i] = page[i] < static_cast<uint32_t>(L.max_blocks);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int32_t pr = lane + c * k_wave;
      if (v && kind[i] < 2 && pr < A.pair_count) {
        cs[i][c] = A.rope[static_cast<uint64_t>(pos[i]) * A.pair_count + pr];
      }
    }
  }
  if constexpr (REG) {
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      if (!ok[i]) continue;  // uniform
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int32_t pr = lane + c * k_wave;  // the lane's pair: dims 2 pr, 2 pr + 1
        if (2 * pr >= D) continue;
        float2 y = x[i][c];
        if (kind[i] < 2 && pr < A.pair_count) {  // apply_rope_pairing, same expressions
          const float x0 = y.x, x1 = y.y;
          y.x = x0 * cs[i][c].x - x1 * cs[i][c].y;
          y.y = x0 * cs[i][c].y + x1 * cs[i][c].x;
        }
        if (kind[i] == 0) {
          *reinterpret_cast<float2 *>(A.q_out + (static_cast<uint64_t>(tok[i]) * L.n_head + head[i]) * D +
                                      2 * pr) = y;
        } else {
          const int32_t slot = pos[i] % L.block_tokens;
          uint8_t *region = (kind[i] == 1 ? A.k_pool : A.v_pool) +
                            L.region_offset(A.layer, static_cast<int32_t>(page[i]), head[i]);
          reinterpret_cast<uint32_t *>(region + static_cast<uint64_t>(slot) * D * 2u)[pr] =
              as_u32(pack_half2(y.x, y.y));
        }
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    if (ok[i]) {  // uniform
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int32_t d = 2 * (lane + c * k_wave);
        if (d < D) *reinterpret_cast<float2 *>(buf + d) = x[i][c];
      }
      wave_sync();
      const float *wt = kind[i] == 0 ? A.q_norm : (kind[i] == 1 ? A.k_norm : nullptr);
      const bool head_norm = kind[i] < 2 && wt != nullptr;
      const bool v_norm = kind[i] == 2 && A.v_rms != 0;
      if (lane == 0 && head_norm) {
        // apply_headwise_rms_norm (detail.hpp:1073-1082)
        float ss = 0.0f;
        for (int32_t d = 0; d < D; ++d) ss += buf[d] * buf[d];
        s_scale[wave] = 1.0f / sqrtf(ss / static_cast<float>(D) + A.eps);
      }
      if (v_norm) {
        // apply_rms_norm_in_place (detail.hpp:1098-1106), in the order of
        // rope_append_kernel: one fp64 chain over the token's whole v
        const float *vv = A.v_rows + static_cast<uint64_t>(tok[i]) * L.n_head_kv * D;
        const int32_t n = L.n_head_kv * D;
        double ss = 0.0;
        for (int32_t c0 = 0; c0 < n; c0 += k_wave) {
          const int32_t j = c0 + lane;
          const float xv = j < n ? vv[j] : 0.0f;
          const float sq = xv * xv;
          const int32_t left = n - c0 < k_wave ? n - c0 : k_wave;
          for (int32_t l = 0; l < left; ++l) {
            ss += static_cast<double>(
                __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sq), l)));
          }
        }
        const float mean = static_cast<float>(ss / static_cast<double>(n));
        if (lane == 0) s_scale[wave] = 1.0f / sqrtf(mean + A.eps);
      }
      if (head_norm || v_norm) {
        wave_sync();
        const float sc = s_scale[wave];
        if (head_norm) {
          for (int32_t d = lane; d < D; d += k_wave) buf[d] *= sc * wt[d];
        } else {
          for (int32_t d = lane; d < D; d += k_wave) buf[d] *= sc;
        }
        wave_sync();
      }
      // apply_rope_pairing (detail.hpp:2905-2936)
      if (kind[i] < 2 && A.pair_count > 0) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const int32_t pr = lane + c * k_wave;
          if (pr < A.pair_count) {
            const int32_t d0 = pr * A.x0_stride;
            const int32_t d1 = pr * A.x1_stride + A.x1_base;
            const float x0 = buf[d0];
            const float x1 = buf[d1];
            buf[d0] = x0 * cs[i][c].x - x1 * cs[i][c].y;
            buf[d1] = x0 * cs[i][c].y + x1 * cs[i][c].x;
          }
        }
        wave_sync();
      }
      if (kind[i] == 0) {
        float *dst = A.q_out + (static_cast<uint64_t>(tok[i]) * L.n_head + head[i]) * D;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const int32_t d = 2 * (lane + c * k_wave);
          if (d < D) *reinterpret_cast<float2 *>(dst + d) = *reinterpret_cast<const float2 *>(buf + d);
        }
      } else {
        const int32_t slot = pos[i] % L.block_tokens;
        uint8_t *region = (kind[i] == 1 ? A.k_pool : A.v_pool) +
                          L.region_offset(A.layer, static_cast<int32_t>(page[i]), head[i]);
        if (L.kv_type == EMELK_KV_F16) {
          // store_fp16_rounded_cache (detail.hpp:3050-3055): RNE per value
          uint32_t *dst = reinterpret_cast<uint32_t *>(region + static_cast<uint64_t>(slot) * D * 2u);
          for (int32_t j = lane; j < D / 2; j += k_wave) dst[j] = as_u32(pack_half2(buf[2 * j], buf[2 * j + 1]));
        } else {
          constexpr int32_t blocks = D / 32;
          if (lane < blocks) {
            int8_t qs[32];
            uint16_t dq;
            quantize_block32(buf + 32 * lane, qs, dq);
            uint4_t *dst = reinterpret_cast<uint4_t *>(region + static_cast<uint64_t>(slot) * D +
                                                       static_cast<uint64_t>(lane) * 32u);
            dst[0] = __builtin_bit_cast(uint4_t, *reinterpret_cast<int8_t(*)[16]>(qs));
            dst[1] = __builtin_bit_cast(uint4_t, *reinterpret_cast<int8_t(*)[16]>(qs + 16));
            reinterpret_cast<uint16_t *>(region + L.scale_plane())[static_cast<uint64_t>(slot) * blocks +
                                                                   lane] = dq;
          }
        }
      }
      wave_sync();  // the next row reuses buf
    }
  }
}

// Checks a pairing: every pair inside the head and no dim used twice.
bool pairing_ok(const emelk_rope_params &p, int32_t head_dim, int32_t pair_count, int32_t x1_base) {
  if (p.x0_stride < 0 || p.x1_stride < 0 || x1_base < 0) return false;
  std::vector<char> used(static_cast<size_t>(head_dim), 0);
  for (int32_t i = 0; i < pair_count; ++i) {
    const int64_t d0 = static_cast<int64_t>(i) * p.x0_stride;
    const int64_t d1 = static_cast<int64_t>(i) * p.x1_stride + x1_base;
    if (d0 >= head_dim || d1 >= head_dim || d0 == d1) return false;
    if (used[static_cast<size_t>(d0)] || used[static_cast<size_t>(d1)]) return false;
    used[static_cast<size_t>(d0)] = 1;
    used[static_cast<size_t>(d1)] = 1;
  }
  return true;
}

}  // namespace
}  // namespace emelk

extern "C" emel_error_type emelk_rope_table_create(const emelk_rope_params *params,
                                                   int32_t head_dim, int32_t max_positions,
                                                   void *stream, emelk_rope_table **table_out) {
  if (table_out == nullptr) return EMELK_ERR_INVALID_REQUEST;
  *table_out = nullptr;
  if (params == nullptr || head_dim <= 0 || head_dim > emelk::k_max_dim || max_positions <= 0 ||
      !(params->freq_base > 0.0f) || !std::isfinite(params->freq_base)) {
    return EMELK_ERR_INVALID_REQUEST;
  }
  const int32_t rot_dim = params->n_rot < head_dim ? params->n_rot : head_dim;
  // apply_rope_pairing leaves the vector unchanged when rot_dim <= 1
  const int32_t pair_count = rot_dim > 1 ? rot_dim / 2 : 0;
  const int64_t x1_base_wide = static_cast<int64_t>(params->x1_offset) +
                               static_cast<int64_t>(params->x1_half_rot_offset) * pair_count;
  if (x1_base_wide < 0 || x1_base_wide > head_dim) return EMELK_ERR_INVALID_REQUEST;
  const int32_t x1_base = static_cast<int32_t>(x1_base_wide);
  if (!emelk::pairing_ok(*params, head_dim, pair_count, x1_base)) return EMELK_ERR_INVALID_REQUEST;
  const uint64_t entries = static_cast<uint64_t>(max_positions) * static_cast<uint64_t>(pair_count);
  if (entries > (uint64_t{1} << 29)) return EMELK_ERR_INVALID_REQUEST;  // 4 GiB of (cos, sin)

  auto *tb = new (std::nothrow) emelk_rope_table();
  if (tb == nullptr) return EMELK_ERR_OUT_OF_MEMORY;
  tb->params = *params;
  tb->head_dim = head_dim;
  tb->pair_count = pair_count;
  tb->x1_base = x1_base;
  tb->max_positions = max_positions;
  if (entries > 0) {
    std::vector<float2> host;
    try {
      host.resize(entries);
    } catch (...) {
      delete tb;
      return EMELK_ERR_OUT_OF_MEMORY;
    }
    // the per-call recurrence of apply_rope_pairing (detail.hpp:2915-2934)
    const float theta_scale = ::powf(params->freq_base, -2.0f / static_cast<float>(rot_dim));
    for (int32_t p = 0; p < max_positions; ++p) {
      float theta = static_cast<float>(p);
      float2 *row = host.data() + static_cast<uint64_t>(p) * pair_count;
      for (int32_t i = 0; i < pair_count; ++i) {
        row[i] = make_float2(::cosf(theta), ::sinf(theta));
        theta *= theta_scale;
      }
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (hipMalloc(reinterpret_cast<void **>(&tb->dev), entries * sizeof(float2)) != hipSuccess) {
      delete tb;
      return EMELK_ERR_OUT_OF_MEMORY;
    }
    if (hipMemcpyAsync(tb->dev, host.data(), entries * sizeof(float2), hipMemcpyHostToDevice, st) !=
            hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess) {
      emelk_rope_table_destroy(tb);
      return EMELK_ERR_BACKEND;
    }
  }
  *table_out = tb;
  return EMELK_ERR_NONE;
}

extern "C" void emelk_rope_table_destroy(emelk_rope_table *table) {
  if (table == nullptr) return;
  if (table->dev != nullptr) {
    (void)hipDeviceSynchronize();
    (void)hipFree(table->dev);
  }
  delete table;
}

extern "C" int32_t emelk_rope_table_positions(const emelk_rope_table *table) {
  return table == nullptr ? 0 : table->max_positions;
}

extern "C" emel_error_type emelk_kv_qkv_rope_append(
    const emelk_kv_geometry *g, void *k_pool, void *v_pool, int32_t layer, const float *q_in,
    float *q_out, const float *k_rows, const float *v_rows, int32_t n_seq, int32_t n_tokens,
    const int32_t *positions, const uint16_t *block_tables, int32_t table_stride,
    const emelk_rope_table *rope, const float *q_norm, const float *k_norm, int32_t v_rms,
    float rms_epsilon, void *stream) {
  emelk::pool_layout L;
  if (emelk::make_pool_layout(g, L) != EMELK_ERR_NONE || k_pool == nullptr || v_pool == nullptr ||
      q_in == nullptr || q_out == nullptr || k_rows == nullptr || v_rows == nullptr ||
      positions == nullptr || block_tables == nullptr || rope == nullptr || layer < 0 ||
      layer >= L.n_layer || n_seq < 0 || n_tokens < 0 || table_stride <= 0 ||
      rope->head_dim != L.head_dim || !std::isfinite(rms_epsilon) ||
      static_cast<int64_t>(n_seq) * n_tokens > 0x7FFFFFFF) {
    return EMELK_ERR_INVALID_REQUEST;
  }
  if (n_seq == 0 || n_tokens == 0) return EMELK_ERR_NONE;
  emelk::rope_append_args A;
  A.L = L;
  A.k_pool = static_cast<uint8_t *>(k_pool);
  A.v_pool = static_cast<uint8_t *>(v_pool);
  A.layer = layer;
  A.q_in = q_in;
  A.q_out = q_out;
  A.k_rows = k_rows;
  A.v_rows = v_rows;
  A.n_seq = n_seq;
  A.n_tokens = n_tokens;
  A.positions = positions;
  A.tables = block_tables;
  A.table_stride = table_stride;
  A.rope = rope->dev;
  A.rope_positions = rope->max_positions;
  A.pair_count = rope->pair_count;
  A.x0_stride = rope->params.x0_stride;
  A.x1_stride = rope->params.x1_stride;
  A.x1_base = rope->x1_base;
  A.q_norm = q_norm;
  A.k_norm = k_norm;
  A.v_rms = v_rms;
  A.eps = rms_epsilon;
  const int32_t n_rows = L.n_head + 2 * L.n_head_kv;
  const int64_t rows = static_cast<int64_t>(n_seq) * n_tokens * n_rows;
  const dim3 block(emelk::k_rows_per_wg * emelk::k_wave);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (rows >= emelk::k_rows_kernel_min && rows < 0x7FFFFFFF) {
    constexpr int RPW = emelk::k_rows_per_wave;
    constexpr int64_t per_wg = emelk::k_rows_per_wg * RPW;
    const dim3 grid(static_cast<uint32_t>((rows + per_wg - 1) / per_wg));
    const bool reg = L.kv_type == EMELK_KV_F16 && q_norm == nullptr && k_norm == nullptr &&
                     v_rms == 0 && A.x0_stride == 2 && A.x1_stride == 2 && A.x1_base == 1;
    if (reg) {
      switch (L.head_dim) {
        case 64: hipLaunchKernelGGL((emelk::rope_append_rows_kernel<64, RPW, true>), grid, block, 0, st, A); break;
        case 128: hipLaunchKernelGGL((emelk::rope_append_rows_kernel<128, RPW, true>), grid, block, 0, st, A); break;
        case 256: hipLaunchKernelGGL((emelk::rope_append_rows_kernel<256, RPW, true>), grid, block, 0, st, A); break;
        default: hipLaunchKernelGGL((emelk::rope_append_rows_kernel<512, RPW, true>), grid, block, 0, st, A); break;
      }
    } else {
      switch (L.head_dim) {
        case 64: hipLaunchKernelGGL((emelk::rope_append_rows_kernel<64, RPW, false>), grid, block, 0, st, A); break;
        case 128: hipLaunchKernelGGL((emelk::rope_append_rows_kernel<128, RPW, false>), grid, block, 0, st, A); break;
        case 256: hipLaunchKernelGGL((emelk::rope_append_rows_kernel<256, RPW, false>), grid, block, 0, st, A); break;
        default: hipLaunchKernelGGL((emelk::rope_append_rows_kernel<512, RPW, false>), grid, block, 0, st, A); break;
      }
    }
  } else {
    const dim3 grid(static_cast<uint32_t>(n_seq * n_tokens),
                    static_cast<uint32_t>((n_rows + emelk::k_rows_per_wg - 1) / emelk::k_rows_per_wg));
    hipLaunchKernelGGL(emelk::rope_append_kernel, grid, block, 0, st, A);
  }
  return hipGetLastError() == hipSuccess ? EMELK_ERR_NONE : EMELK_ERR_BACKEND;
}
