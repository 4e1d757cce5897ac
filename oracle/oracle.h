/*
 * TEST INFRASTRUCTURE — the CPU oracle for the KV-cache hot path.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this library, and only as the checker (or as the timed CPU baseline).  The
 * product path (emel.cpp_amd/) never links or calls it.
 *
 * Each function is a plain-C restatement of the reference CPU arithmetic it
 * cites (paths relative to the reference checkout, stateforward/emel.cpp).
 * Pinning status of every function is listed in oracle.c's header.
 */
#ifndef EMELK_ORACLE_H
#define EMELK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF q8_0 block: 32 int8 values and an f16 scale (34 bytes, packed). */
#define ORC_QK8_0 32
typedef struct __attribute__((packed)) {
  uint16_t d;
  int8_t qs[ORC_QK8_0];
} orc_block_q8_0;

uint16_t orc_fp32_to_fp16(float value);
float orc_fp16_to_fp32(uint16_t bits);
uint64_t orc_fp32_to_fp16_sweep(uint64_t lo, uint64_t hi);
void orc_fp32_to_fp16_row(const float *src, uint16_t *dst, int64_t n);
void orc_fp16_to_fp32_row(const uint16_t *src, float *dst, int64_t n);

void orc_quantize_row_q8_0(const float *x, uint64_t stride, orc_block_q8_0 *y, int64_t k);
void orc_dequantize_row_q8_0(const orc_block_q8_0 *x, float *y, int64_t k);

float orc_dot_f32_f16(const float *lhs, const uint16_t *rhs, int64_t n);
float orc_dot_f32_f32_f16r(const float *lhs, const float *rhs, int64_t n);
double orc_exp_and_sum(const float *src, float *dst, int64_t n, float max_value);
float orc_round_fp16_weight(float v);

int64_t orc_physical_kv_position(const uint16_t *blocks, int32_t block_tokens, int32_t position);

/* apply_rope_pairing (text/generator/detail.hpp:2905-2936) on head_count
 * consecutive heads of head_dim floats, in place. */
void orc_rope_pairing(float *vec, int32_t x0_stride, int32_t x1_stride, int32_t x1_offset,
                      int32_t x1_half_rot_offset, int32_t head_count, int32_t head_dim,
                      int32_t n_rot, int32_t position, float freq_base);
/* apply_headwise_rms_norm (detail.hpp:1060-1090), in place; returns 0 on a
 * rejected shape (as the reference returns false). */
int orc_headwise_rms_norm(float *vec, const float *weights, int32_t head_count, int32_t head_dim,
                          float epsilon);
/* apply_rms_norm_in_place (detail.hpp:1092-1111), in place. */
int orc_rms_norm_in_place(float *vec, int64_t n, float epsilon);

/* Append one token row (fp32) for one layer into a token-major paged cache. */
void orc_store_kv_f16(uint16_t *key_cache, uint16_t *value_cache, int32_t kv_dim,
                      const uint16_t *blocks, int32_t block_tokens, int32_t position,
                      const float *k_row, const float *v_row);
void orc_store_kv_q8_0(orc_block_q8_0 *key_cache, orc_block_q8_0 *value_cache, int32_t kv_dim,
                       const uint16_t *blocks, int32_t block_tokens, int32_t position,
                       const float *k_row, const float *v_row);

/*
 * Paged decode attention over one layer, the reference's nonflash route.
 * key_cache/value_cache: token-major [physical position][kv_dim] (kv_dim =
 * n_head_kv*head_dim).  q/out: [n_head][head_dim].  scratch: >= 4*n_ctx floats.
 * inv_scale is the score multiplier (the reference uses 1/sqrt(head_dim)).
 */
int orc_compute_attention_f16(const float *q, const uint16_t *key_cache,
                              const uint16_t *value_cache, const uint16_t *blocks,
                              int32_t block_tokens, int32_t n_head, int32_t n_head_kv,
                              int32_t head_dim, int32_t position_limit, int32_t n_ctx,
                              float inv_scale, float *out, float *scratch);
int orc_compute_attention_q8_0(const float *q, const orc_block_q8_0 *key_cache,
                               const orc_block_q8_0 *value_cache, const uint16_t *blocks,
                               int32_t block_tokens, int32_t n_head, int32_t n_head_kv,
                               int32_t head_dim, int32_t position_limit, int32_t n_ctx,
                               float inv_scale, float *out, float *scratch);

/* Contiguous flash decode with the f16 accumulator (reference flash route).
 * k/v: head-major [n_head_kv][kv_stride_tokens][head_dim]. */
int orc_flash_attn_f16acc(const float *q, const uint16_t *k, const uint16_t *v,
                          int32_t head_dim, int32_t n_head, int32_t n_head_kv,
                          int32_t kv_tokens, int64_t kv_stride_tokens, float scale,
                          float *out);

/* fp64 "ideal" attention on the stored values (k/v already dequantized to
 * float, token-major logical [kv_tokens][n_head_kv*head_dim]); q unrounded. */
void orc_attention_f64(const float *q, const float *k, const float *v, int32_t n_head,
                       int32_t n_head_kv, int32_t head_dim, int32_t kv_tokens,
                       double inv_scale, float *out);

/*
 * Batched paged decode over a whole batch for one layer, the CPU baseline
 * driver: sequences spread over up to n_threads threads.  Layout as
 * orc_compute_attention_f16; block tables are [n_seq][table_stride].
 * position_limits[s] = tokens to attend for sequence s.  Returns wall seconds.
 */
double orc_decode_batch_f16(const float *q, const uint16_t *key_cache,
                            const uint16_t *value_cache, const uint16_t *block_tables,
                            int32_t table_stride, const int32_t *position_limits,
                            int32_t n_seq, int32_t block_tokens, int32_t n_head,
                            int32_t n_head_kv, int32_t head_dim, int32_t n_ctx,
                            float inv_scale, float *out, int32_t n_threads);

/*
 * Rows of attention for the CPU baseline, spread over up to n_threads
 * threads (a shared row counter balances rows of different lengths).  Row i
 * takes q row i, block-table row row_table[i] (row i when row_table is
 * NULL) and attends to [0, limits[i]) with an n_ctx-wide softmax (limits[i]
 * when n_ctx <= 0).  kind 0: f16 caches, 1: q8_0 caches (orc_block_q8_0
 * rows).  Returns wall seconds.
 */
double orc_attention_rows(int32_t kind, const float *q, const void *key_cache,
                          const void *value_cache, const uint16_t *block_tables,
                          int32_t table_stride, const int32_t *row_table,
                          const int32_t *limits, int32_t n_rows, int32_t block_tokens,
                          int32_t n_head, int32_t n_head_kv, int32_t head_dim, int32_t n_ctx,
                          float inv_scale, float *out, int32_t n_threads);

#ifdef __cplusplus
}
#endif

#endif
