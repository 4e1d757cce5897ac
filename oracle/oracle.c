/*
 * TEST INFRASTRUCTURE — CPU oracle for the KV-cache hot path.
 *
 * This file is the checker, never the product: only tests/, the smoke check and
 * bench.py's cpu_baseline leg load liboracle.so.  It restates, in plain C, the
 * reference CPU arithmetic of stateforward/emel.cpp for each function below
 * (file:line relative to the reference checkout).  Build flags: -O3, no
 * fast-math, -ffp-contract=off, so every float operation rounds as written.
 *
 * Pinning (how each function is checked against something other than itself):
 *   orc_fp32_to_fp16 / orc_fp16_to_fp32
 *       exhaustive sweep of all 2^32 inputs vs the reference header compiled
 *       into oracle/_ref (checksum fixture), plus the reference's own known
 *       answers (detail_tests.cpp:1085-1118).
 *   orc_quantize_row_q8_0 / orc_dequantize_row_q8_0
 *       golden blocks from the compiled reference quantizer (outliers, .5 ties,
 *       all-zero block), plus the reference known answer detail_tests.cpp:1309-1324.
 *   orc_physical_kv_position / orc_store_kv_*
 *       closed form and the reference cases detail_tests.cpp:2460-2641
 *       (reversed two-block map).
 *   orc_compute_attention_f16
 *       helpers pinned against the compiled reference (dot products, exp-sum,
 *       fp16 weight rounding); the composition is checked against the fp64
 *       ideal (orc_attention_f64) and a brute-force one-token case where the
 *       output must equal fp16(v) exactly.
 *   orc_compute_attention_q8_0
 *       same composition over dequantize_row_q8_0 values; pinned by the same
 *       ideal-attention and one-token checks (the reference has no q8_0 KV
 *       route, so the route itself is this repository's definition).
 *   orc_flash_attn_f16acc
 *       bit-exact vs the compiled reference scalar flash route.
 *   orc_attention_f64
 *       one-token (output = v), uniform-score (output = mean of v) and
 *       two-token closed forms.
 *   orc_rope_pairing
 *       position 0 is the identity; every pair keeps its norm; the result
 *       matches a float64 rotation by the float32 theta recurrence within
 *       a few ulp; the normal and neox pairings touch exactly the dims the
 *       reference tests expect (detail_tests.cpp:974-1030); dims past
 *       n_rot are untouched.
 *   orc_headwise_rms_norm / orc_rms_norm_in_place
 *       float64 closed form within a few ulp; unit weights and a constant
 *       vector give rms 1; rejected shapes return 0 as the reference does.
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

static inline uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* IEEE binary32 -> binary16, round to nearest even; NaN -> sign|0x7E00.
 * Restates quant::fp32_to_fp16 (src/emel/kernel/detail.hpp:372-392) by the
 * textbook integer method rather than the reference's float-bias trick. */
uint16_t orc_fp32_to_fp16(float value) {
  const uint32_t x = f2u(value);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return sign | 0x7e00u;          /* NaN */
  if (ax >= 0x477ff000u) return sign | 0x7c00u;         /* |v| >= 65520 -> inf */
  if (ax < 0x38800000u) {                               /* below 2^-14: subnormal */
    if (ax <= 0x33000000u) return sign;                 /* <= 2^-25 rounds to 0 */
    const uint32_t e = ax >> 23;
    const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    const uint32_t shift = 126u - e;                    /* 14..24 */
    uint32_t r = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (r & 1u))) ++r;
    return sign | (uint16_t)r;
  }
  const uint32_t e16 = (ax >> 23) - 112u;
  const uint32_t m = ax & 0x7fffffu;
  uint32_t r = (e16 << 10) | (m >> 13);
  const uint32_t rem = m & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
  return sign | (uint16_t)r;
}

/* binary16 -> binary32, exact.  Restates quant::fp16_to_fp32
 * (src/emel/kernel/detail.hpp:350-370). */
float orc_fp16_to_fp32(uint16_t h) {
  const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  const uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
  const uint32_t m = (uint32_t)h & 0x3ffu;
  if (e == 0x1fu) return u2f(sign | 0x7f800000u | (m << 13));
  if (e != 0) return u2f(sign | ((e + 112u) << 23) | (m << 13));
  if (m == 0) return u2f(sign);
  /* subnormal: m * 2^-24 is exact in fp32 */
  const float mag = (float)m * 5.9604644775390625e-08f;
  return u2f(sign | f2u(mag));
}

uint64_t orc_fp32_to_fp16_sweep(uint64_t lo, uint64_t hi) {
  uint64_t acc = 0;
  for (uint64_t b = lo; b < hi; ++b) {
    acc = (acc ^ orc_fp32_to_fp16(u2f((uint32_t)b))) * 1099511628211ull;
  }
  return acc;
}

static inline float fp16r(float v) { return orc_fp16_to_fp32(orc_fp32_to_fp16(v)); }

void orc_fp32_to_fp16_row(const float *src, uint16_t *dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = orc_fp32_to_fp16(src[i]);
}
void orc_fp16_to_fp32_row(const uint16_t *src, float *dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = orc_fp16_to_fp32(src[i]);
}

/* q8_0 quantizer.  Restates quantize_row_q8_0_strided
 * (src/emel/kernel/detail.hpp:804-824): per 32 values d = amax/127 (IEEE
 * division), inv_d = d != 0 ? 1/d : 0, q = clamp(round-half-away(x*inv_d),
 * -127, 127), scale stored as fp16(d). */
void orc_quantize_row_q8_0(const float *x, uint64_t stride, orc_block_q8_0 *y, int64_t k) {
  const int64_t nb = k / ORC_QK8_0;
  for (int64_t i = 0; i < nb; ++i) {
    const float *blk = x + (uint64_t)i * ORC_QK8_0 * stride;
    float amax = 0.0f;
    for (int j = 0; j < ORC_QK8_0; ++j) {
      const float a = fabsf(blk[(uint64_t)j * stride]);
      if (a > amax) amax = a;
    }
    const float d = amax / 127.0f;
    const float inv_d = d != 0.0f ? 1.0f / d : 0.0f;
    y[i].d = orc_fp32_to_fp16(d);
    for (int j = 0; j < ORC_QK8_0; ++j) {
      int q = (int)roundf(blk[(uint64_t)j * stride] * inv_d);
      if (q < -127) q = -127;
      if (q > 127) q = 127;
      y[i].qs[j] = (int8_t)q;
    }
  }
}

/* dequantize_row_q8_0 (src/emel/kernel/detail.hpp:679-690): y = f32(d) * q. */
void orc_dequantize_row_q8_0(const orc_block_q8_0 *x, float *y, int64_t k) {
  const int64_t nb = k / ORC_QK8_0;
  for (int64_t i = 0; i < nb; ++i) {
    const float d = orc_fp16_to_fp32(x[i].d);
    for (int j = 0; j < ORC_QK8_0; ++j) y[i * ORC_QK8_0 + j] = d * (float)x[i].qs[j];
  }
}

/* physical_kv_position (src/emel/text/generator/detail.hpp:2976-2982). */
int64_t orc_physical_kv_position(const uint16_t *blocks, int32_t bt, int32_t pos) {
  return (int64_t)blocks[pos / bt] * bt + (pos % bt);
}

/* store_attention_kv_cache, token-major half (detail.hpp:3294-3312):
 * fp32 -> fp16 RNE at layer_cache_offset(position). */
void orc_store_kv_f16(uint16_t *key_cache, uint16_t *value_cache, int32_t kv_dim,
                      const uint16_t *blocks, int32_t bt, int32_t position,
                      const float *k_row, const float *v_row) {
  const int64_t off = orc_physical_kv_position(blocks, bt, position) * kv_dim;
  orc_fp32_to_fp16_row(k_row, key_cache + off, kv_dim);
  orc_fp32_to_fp16_row(v_row, value_cache + off, kv_dim);
}

/* Same placement with the row quantized by quantize_row_q8_0_strided
 * (stride 1) instead of rounded to fp16. */
void orc_store_kv_q8_0(orc_block_q8_0 *key_cache, orc_block_q8_0 *value_cache, int32_t kv_dim,
                       const uint16_t *blocks, int32_t bt, int32_t position,
                       const float *k_row, const float *v_row) {
  const int64_t nblk = kv_dim / ORC_QK8_0;
  const int64_t off = orc_physical_kv_position(blocks, bt, position) * nblk;
  orc_quantize_row_q8_0(k_row, 1, key_cache + off, kv_dim);
  orc_quantize_row_q8_0(v_row, 1, value_cache + off, kv_dim);
}

/* dot_product_f32_f16_scores, scalar route (kernel/detail.hpp:2211-2245):
 * float(sum double(fp16r(lhs_i)) * double(f16 rhs_i)). */
float orc_dot_f32_f16(const float *lhs, const uint16_t *rhs, int64_t n) {
  double acc = 0.0;
  for (int64_t i = 0; i < n; ++i) acc += (double)fp16r(lhs[i]) * (double)orc_fp16_to_fp32(rhs[i]);
  return (float)acc;
}

/* dot_product_ggml_f16_scores(float, float), scalar route
 * (kernel/detail.hpp:2085-2152): both operands rounded to fp16. */
float orc_dot_f32_f32_f16r(const float *lhs, const float *rhs, int64_t n) {
  double acc = 0.0;
  for (int64_t i = 0; i < n; ++i) acc += (double)fp16r(lhs[i]) * (double)fp16r(rhs[i]);
  return (float)acc;
}

/* exp_and_sum_ggml_f32, scalar route (kernel/detail.hpp:2055-2083). */
double orc_exp_and_sum(const float *src, float *dst, int64_t n, float max_value) {
  double sum = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    const float e = expf(src[i] - max_value);
    dst[i] = e;
    sum += (double)e;
  }
  return sum;
}

/* round_fp16_weight (kernel/detail.hpp:4254-4260). */
float orc_round_fp16_weight(float v) { return fp16r(v); }

/* Shared body of compute_attention (detail.hpp:3153-3230) with
 * round_q_for_nonflash (2898-2903) and fill_masked_softmax_probs_ggml
 * (3123-3151).  load_row(p, kv_head, dst) yields the float K or V values of
 * position p.  Scores: float(sum_d double(fp16r(q_d)) * double(k_d)) * inv_scale
 * (dot_product_f32_f16_scores, kernel/detail.hpp:2211-2245); softmax over
 * n_ctx columns with -inf padding, expf and a double sum
 * (exp_and_sum_ggml_f32, 2055-2083); p = e * float(1/sum) rounded to fp16
 * (round_fp16_weight, 4258); out_d = float(sum_p double(fp16r(v)) *
 * double(fp16r(p16))) (dot_product_ggml_f16_scores(float,float), 2085-2152). */
typedef void (*orc_row_loader)(const void *cache, const uint16_t *blocks, int32_t bt,
                               int32_t kv_dim, int32_t pos, int32_t kv_head,
                               int32_t head_dim, float *dst);

static void load_f16_row(const void *cache, const uint16_t *blocks, int32_t bt, int32_t kv_dim,
                         int32_t pos, int32_t kv_head, int32_t head_dim, float *dst) {
  const uint16_t *c = (const uint16_t *)cache;
  const int64_t off = orc_physical_kv_position(blocks, bt, pos) * kv_dim + (int64_t)kv_head * head_dim;
  for (int32_t d = 0; d < head_dim; ++d) dst[d] = orc_fp16_to_fp32(c[off + d]);
}

static void load_q8_0_row(const void *cache, const uint16_t *blocks, int32_t bt, int32_t kv_dim,
                          int32_t pos, int32_t kv_head, int32_t head_dim, float *dst) {
  const orc_block_q8_0 *c = (const orc_block_q8_0 *)cache;
  const int64_t nblk = kv_dim / ORC_QK8_0;
  const int64_t off = orc_physical_kv_position(blocks, bt, pos) * nblk +
                      ((int64_t)kv_head * head_dim) / ORC_QK8_0;
  orc_dequantize_row_q8_0(c + off, dst, head_dim);
}

static int compute_attention_generic(const float *q, const void *key_cache, const void *value_cache,
                                     orc_row_loader load, int round_v, const uint16_t *blocks,
                                     int32_t bt,
                                     int32_t n_head, int32_t n_head_kv, int32_t head_dim,
                                     int32_t position_limit, int32_t n_ctx, float inv_scale,
                                     float *out, float *scratch) {
  if (position_limit <= 0 || position_limit > n_ctx || n_head_kv <= 0 || n_head % n_head_kv) {
    return 0;
  }
  const int32_t n_rep = n_head / n_head_kv;
  const int32_t kv_dim = n_head_kv * head_dim;
  float *scores = scratch;
  float *probs = scratch + n_ctx;
  float *rounded = scratch + 2 * (int64_t)n_ctx;
  float *qr = (float *)malloc(sizeof(float) * (size_t)head_dim * 2);
  float *vrow = qr + head_dim;
  for (int32_t head = 0; head < n_head; ++head) {
    const int32_t kv_head = head / n_rep;
    const float *qh = q + (int64_t)head * head_dim;
    for (int32_t d = 0; d < head_dim; ++d) qr[d] = fp16r(qh[d]);   /* round_q_for_nonflash */
    for (int32_t p = 0; p < position_limit; ++p) {
      load(key_cache, blocks, bt, kv_dim, p, kv_head, head_dim, vrow);
      double acc = 0.0;   /* dot_product_f32_f16_scores on the loaded row */
      for (int32_t d = 0; d < head_dim; ++d) acc += (double)fp16r(qr[d]) * (double)vrow[d];
      scores[p] = (float)acc * inv_scale;
    }
    for (int32_t p = position_limit; p < n_ctx; ++p) scores[p] = -INFINITY;

    float mx = -INFINITY;
    for (int32_t p = 0; p < n_ctx; ++p) mx = scores[p] > mx ? scores[p] : mx;
    const double sum = orc_exp_and_sum(scores, probs, n_ctx, mx);
    const float inv_sum = sum == 0.0 ? 0.0f : (float)(1.0 / sum);
    for (int32_t p = 0; p < n_ctx; ++p) {
      probs[p] = probs[p] * inv_sum;
      rounded[p] = orc_round_fp16_weight(probs[p]);
    }

    /* out_d: the reference walks dim-major over a gathered value column; the
     * per-dim double sum runs over positions in ascending order, as here. */
    double *accv = (double *)calloc((size_t)head_dim, sizeof(double));
    for (int32_t p = 0; p < position_limit; ++p) {
      load(value_cache, blocks, bt, kv_dim, p, kv_head, head_dim, vrow);
      const double w = (double)fp16r(rounded[p]);
      for (int32_t d = 0; d < head_dim; ++d) {
        accv[d] += (double)(round_v ? fp16r(vrow[d]) : vrow[d]) * w;
      }
    }
    /* padded columns contribute fp16r(0) * p = +0.0 to each sum: no-op */
    for (int32_t d = 0; d < head_dim; ++d) out[(int64_t)head * head_dim + d] = (float)accv[d];
    free(accv);
  }
  free(qr);
  return 1;
}

int orc_compute_attention_f16(const float *q, const uint16_t *key_cache,
                              const uint16_t *value_cache, const uint16_t *blocks,
                              int32_t bt, int32_t n_head, int32_t n_head_kv,
                              int32_t head_dim, int32_t position_limit, int32_t n_ctx,
                              float inv_scale, float *out, float *scratch) {
  return compute_attention_generic(q, key_cache, value_cache, load_f16_row, 1, blocks, bt, n_head,
                                   n_head_kv, head_dim, position_limit, n_ctx, inv_scale, out,
                                   scratch);
}

/* q8_0 cache: identical arithmetic, with the K/V values produced by
 * dequantize_row_q8_0.  The reference's PV dot rounds its value operand to
 * fp16 (dot_product_ggml_f16_scores) because its cache holds fp16 values, for
 * which that rounding is the identity; dequantized q8_0 values (d * q, up to
 * 19 significant bits) are not fp16 values, so here they enter the double
 * sum unrounded — the only rounding kept is the reference's own (q and the
 * normalised probabilities to fp16). */
int orc_compute_attention_q8_0(const float *q, const orc_block_q8_0 *key_cache,
                               const orc_block_q8_0 *value_cache, const uint16_t *blocks,
                               int32_t bt, int32_t n_head, int32_t n_head_kv,
                               int32_t head_dim, int32_t position_limit, int32_t n_ctx,
                               float inv_scale, float *out, float *scratch) {
  return compute_attention_generic(q, key_cache, value_cache, load_q8_0_row, 0, blocks, bt, n_head,
                                   n_head_kv, head_dim, position_limit, n_ctx, inv_scale, out,
                                   scratch);
}

/* Flash decode with an f16 accumulator: restates
 * run_flash_attn_ext_active_kv_with_workspace_unchecked
 * (src/emel/kernel/detail.hpp:5238-5291) with dot_product_f16_f16_scores
 * (2154-2209), scale_f16_buffer_scalar (4312-4320) and axpy_f16_buffer_scalar
 * (4322-4333). */
int orc_flash_attn_f16acc(const float *q, const uint16_t *k, const uint16_t *v, int32_t head_dim,
                          int32_t n_head, int32_t n_head_kv, int32_t kv_tokens,
                          int64_t kv_stride_tokens, float scale, float *out) {
  if (head_dim <= 0 || n_head_kv <= 0 || n_head % n_head_kv || kv_tokens <= 0) return 0;
  const int32_t n_rep = n_head / n_head_kv;
  uint16_t *q16 = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)head_dim * 2);
  uint16_t *acc = q16 + head_dim;
  for (int32_t head = 0; head < n_head; ++head) {
    const int32_t kv_head = head / n_rep;
    const uint16_t *kh = k + (int64_t)kv_head * kv_stride_tokens * head_dim;
    const uint16_t *vh = v + (int64_t)kv_head * kv_stride_tokens * head_dim;
    for (int32_t d = 0; d < head_dim; ++d) {
      q16[d] = orc_fp32_to_fp16(q[(int64_t)head * head_dim + d]);
      acc[d] = 0;
    }
    float score_sum = 0.0f;
    float max_score = -INFINITY;
    for (int32_t t = 0; t < kv_tokens; ++t) {
      const uint16_t *kt = kh + (int64_t)t * head_dim;
      const uint16_t *vt = vh + (int64_t)t * head_dim;
      double dot = 0.0;
      for (int32_t d = 0; d < head_dim; ++d) {
        dot += (double)orc_fp16_to_fp32(q16[d]) * (double)orc_fp16_to_fp32(kt[d]);
      }
      const float score = (float)dot * scale;
      const float old_max = max_score;
      float max_scale = 1.0f;
      float value_scale = 1.0f;
      if (score > max_score) {
        max_score = score;
        max_scale = expf(old_max - max_score);
        const float rs = fp16r(max_scale);
        for (int32_t d = 0; d < head_dim; ++d) {
          acc[d] = orc_fp32_to_fp16(fp16r(orc_fp16_to_fp32(acc[d]) * rs));
        }
      } else {
        value_scale = expf(score - max_score);
      }
      const float ra = fp16r(value_scale);
      for (int32_t d = 0; d < head_dim; ++d) {
        const float prod = orc_fp16_to_fp32(vt[d]) * ra;
        acc[d] = orc_fp32_to_fp16(fp16r(orc_fp16_to_fp32(acc[d]) + prod));
      }
      score_sum = score_sum * max_scale + value_scale;
    }
    float *o = out + (int64_t)head * head_dim;
    if (score_sum == 0.0f) {
      for (int32_t d = 0; d < head_dim; ++d) o[d] = 0.0f;
    } else {
      const float inv = 1.0f / score_sum;
      for (int32_t d = 0; d < head_dim; ++d) o[d] = orc_fp16_to_fp32(acc[d]) * inv;
    }
  }
  free(q16);
  return 1;
}

/* Double-precision reference attention (softmax(q.k * s) . v), the "ideal"
 * against which both the reference routes and the GPU kernels are measured. */
void orc_attention_f64(const float *q, const float *k, const float *v, int32_t n_head,
                       int32_t n_head_kv, int32_t head_dim, int32_t kv_tokens, double inv_scale,
                       float *out) {
  const int32_t n_rep = n_head / n_head_kv;
  const int64_t kv_dim = (int64_t)n_head_kv * head_dim;
  double *s = (double *)malloc(sizeof(double) * ((size_t)kv_tokens + (size_t)head_dim));
  double *o = s + kv_tokens;
  for (int32_t head = 0; head < n_head; ++head) {
    const int32_t kvh = head / n_rep;
    double mx = -INFINITY;
    for (int32_t t = 0; t < kv_tokens; ++t) {
      double acc = 0.0;
      for (int32_t d = 0; d < head_dim; ++d) {
        acc += (double)q[(int64_t)head * head_dim + d] * (double)k[t * kv_dim + kvh * head_dim + d];
      }
      s[t] = acc * inv_scale;
      if (s[t] > mx) mx = s[t];
    }
    double sum = 0.0;
    for (int32_t t = 0; t < kv_tokens; ++t) {
      s[t] = exp(s[t] - mx);
      sum += s[t];
    }
    for (int32_t d = 0; d < head_dim; ++d) o[d] = 0.0;
    for (int32_t t = 0; t < kv_tokens; ++t) {
      const double w = s[t] / sum;
      for (int32_t d = 0; d < head_dim; ++d) o[d] += w * (double)v[t * kv_dim + kvh * head_dim + d];
    }
    for (int32_t d = 0; d < head_dim; ++d) out[(int64_t)head * head_dim + d] = (float)o[d];
  }
  free(s);
}

/* ---- batched CPU baseline driver (one thread per sequence lane) ---------- */

/* Rows of attention over paged caches, spread over threads: row i uses
 * block-table row row_table[i] (identity when NULL) and attends to
 * [0, limits[i]); its softmax spans n_ctx positions (limits[i] when n_ctx
 * <= 0).  kind 0: f16 caches (orc_compute_attention_f16), 1: q8_0
 * (orc_compute_attention_q8_0).  Threads take rows in order from a shared
 * counter, so long and short rows balance.  Returns the wall seconds of
 * the compute alone. */
typedef struct {
  int32_t kind;
  const float *q;
  const void *key_cache, *value_cache;
  const uint16_t *block_tables;
  const int32_t *row_table, *limits;
  int32_t table_stride, n_rows, bt, n_head, n_head_kv, head_dim, n_ctx;
  float inv_scale;
  float *out;
  int32_t next; /* shared row counter */
} orc_rows_job;

static void *rows_worker(void *arg) {
  orc_rows_job *j = (orc_rows_job *)arg;
  int32_t max_ctx = j->n_ctx;
  for (int32_t i = 0; i < j->n_rows; ++i) max_ctx = j->limits[i] > max_ctx ? j->limits[i] : max_ctx;
  float *scratch = (float *)malloc(sizeof(float) * 4 * (size_t)(max_ctx > 0 ? max_ctx : 1));
  const int64_t qd = (int64_t)j->n_head * j->head_dim;
  for (;;) {
    const int32_t i = __atomic_fetch_add(&j->next, 1, __ATOMIC_RELAXED);
    if (i >= j->n_rows) break;
    const int32_t t = j->row_table != NULL ? j->row_table[i] : i;
    const int32_t lim = j->limits[i];
    const int32_t n_ctx = j->n_ctx > 0 ? j->n_ctx : lim;
    const uint16_t *blocks = j->block_tables + (int64_t)t * j->table_stride;
    if (j->kind == 0) {
      orc_compute_attention_f16(j->q + i * qd, (const uint16_t *)j->key_cache,
                                (const uint16_t *)j->value_cache, blocks, j->bt, j->n_head,
                                j->n_head_kv, j->head_dim, lim, n_ctx, j->inv_scale,
                                j->out + i * qd, scratch);
    } else {
      orc_compute_attention_q8_0(j->q + i * qd, (const orc_block_q8_0 *)j->key_cache,
                                 (const orc_block_q8_0 *)j->value_cache, blocks, j->bt, j->n_head,
                                 j->n_head_kv, j->head_dim, lim, n_ctx, j->inv_scale,
                                 j->out + i * qd, scratch);
    }
  }
  free(scratch);
  return NULL;
}

double orc_attention_rows(int32_t kind, const float *q, const void *key_cache,
                          const void *value_cache, const uint16_t *block_tables,
                          int32_t table_stride, const int32_t *row_table,
                          const int32_t *limits, int32_t n_rows, int32_t bt, int32_t n_head,
                          int32_t n_head_kv, int32_t head_dim, int32_t n_ctx, float inv_scale,
                          float *out, int32_t n_threads) {
  if (n_threads < 1) n_threads = 1;
  if (n_threads > n_rows) n_threads = n_rows > 0 ? n_rows : 1;
  pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)n_threads);
  orc_rows_job job = {kind, q, key_cache, value_cache, block_tables, row_table, limits,
                      table_stride, n_rows, bt, n_head, n_head_kv, head_dim, n_ctx, inv_scale,
                      out, 0};
  struct timespec t0, t1;
  clock_gettime(CLOCK_MONOTONIC, &t0);
  for (int32_t i = 0; i < n_threads; ++i) pthread_create(&th[i], NULL, rows_worker, &job);
  for (int32_t i = 0; i < n_threads; ++i) pthread_join(th[i], NULL);
  clock_gettime(CLOCK_MONOTONIC, &t1);
  free(th);
  return (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
}

/* The f16 batch of one decode step: sequence s uses table row s and
 * attends to [0, position_limits[s]) with an n_ctx-wide softmax. */
double orc_decode_batch_f16(const float *q, const uint16_t *key_cache, const uint16_t *value_cache,
                            const uint16_t *block_tables, int32_t table_stride,
                            const int32_t *position_limits, int32_t n_seq, int32_t bt,
                            int32_t n_head, int32_t n_head_kv, int32_t head_dim, int32_t n_ctx,
                            float inv_scale, float *out, int32_t n_threads) {
  return orc_attention_rows(0, q, key_cache, value_cache, block_tables, table_stride, NULL,
                            position_limits, n_seq, bt, n_head, n_head_kv, head_dim, n_ctx,
                            inv_scale, out, n_threads);
}

/* ---- the step before append --------------------------------------------- */

void orc_rope_pairing(float *vec, int32_t x0_stride, int32_t x1_stride, int32_t x1_offset,
                      int32_t x1_half_rot_offset, int32_t head_count, int32_t head_dim,
                      int32_t n_rot, int32_t position, float freq_base) {
  const int32_t rot_dim = n_rot < head_dim ? n_rot : head_dim;
  if (head_count <= 0 || head_dim <= 1 || rot_dim <= 1) return;
  const float theta_scale = powf(freq_base, -2.0f / (float)rot_dim);
  const int32_t pair_count = rot_dim / 2;
  const int32_t x1_base = x1_offset + x1_half_rot_offset * pair_count;
  for (int32_t head = 0; head < head_count; ++head) {
    float *h = vec + (size_t)head * (size_t)head_dim;
    float theta = (float)position;
    for (int32_t pair = 0; pair < pair_count; ++pair) {
      const float c = cosf(theta);
      const float s = sinf(theta);
      const int32_t d0 = pair * x0_stride;
      const int32_t d1 = pair * x1_stride + x1_base;
      const float x0 = h[d0];
      const float x1 = h[d1];
      h[d0] = x0 * c - x1 * s;
      h[d1] = x0 * s + x1 * c;
      theta *= theta_scale;
    }
  }
}

int orc_headwise_rms_norm(float *vec, const float *weights, int32_t head_count, int32_t head_dim,
                          float epsilon) {
  if (head_count <= 0 || head_dim <= 0) return 0;
  for (int32_t head = 0; head < head_count; ++head) {
    float *h = vec + (size_t)head * (size_t)head_dim;
    float square_sum = 0.0f;
    for (int32_t d = 0; d < head_dim; ++d) square_sum += h[d] * h[d];
    const float inv_rms = 1.0f / sqrtf(square_sum / (float)head_dim + epsilon);
    for (int32_t d = 0; d < head_dim; ++d) h[d] *= inv_rms * weights[d];
  }
  return 1;
}

int orc_rms_norm_in_place(float *vec, int64_t n, float epsilon) {
  if (n <= 0) return 0;
  double square_sum = 0.0;
  for (int64_t i = 0; i < n; ++i) square_sum += (double)(vec[i] * vec[i]);
  const float mean = (float)(square_sum / (double)n);
  const float scale = 1.0f / sqrtf(mean + epsilon);
  for (int64_t i = 0; i < n; ++i) vec[i] *= scale;
  return 1;
}
