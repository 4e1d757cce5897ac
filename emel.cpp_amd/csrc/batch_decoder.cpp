// Multi-sequence step executor over the C ABI.
//
// The reference generator runs one sequence (k_sequence_id = 0,
// text/generator/context.hpp:33): per token it sends allocate_slots with the
// copy_kv_cache_block callback (text/generator/actions.hpp:460-474), takes the
// memory view (capture_view, actions.hpp:270-281) and computes every layer
// with that sequence's block table (kv_addressing_from_request,
// detail.hpp:1010-1014).  This executor does the same for a batch of
// sequences: one allocate_slots per sequence (all or nothing over the
// batch), one block-table export for all of them, one upload, and per layer
// the fused norm + RoPE + append followed by decode (one token per
// sequence) or chunked-prefill attention (several).  It is a client of the
// public entry points only.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstring>
#include <new>

#include "emelk.h"

struct emelk_batch_decoder {
  emelk_kv_geometry g{};
  emelk_kv_actor *actor = nullptr;
  emelk_kv_cache *cache = nullptr;
  const emelk_rope_table *rope = nullptr;
  hipStream_t stream = nullptr;
  int32_t max_batch = 0;
  int32_t max_kv_len = 0;
  int32_t stride = 0;  // block-table row length (pages)

  // device
  uint16_t *d_tables = nullptr;  // [max_batch][stride]
  int32_t *d_pos = nullptr;      // [max_batch] first new position
  int32_t *d_kv_len = nullptr;   // [max_batch] position + n_tokens
  void *d_ws = nullptr;
  uint64_t ws_bytes = 0;

  // pinned staging, two sets used alternately; each set's upload event
  // tells when the copy engine is done reading it
  struct staging {
    uint16_t *tables = nullptr;
    int32_t *pos = nullptr;
    int32_t *kv_len = nullptr;
    hipEvent_t uploaded = nullptr;
    bool pending = false;
  } st[2];
  int32_t next_st = 0;

  // current step
  int32_t n_seq = 0;
  int32_t n_tokens = 0;
  int32_t step_max_kv = 0;
  bool step_open = false;
  bool fixed_plan = false;  // plan attention for max_kv_len, not the step's longest
};

namespace {

emel_error_type hip_ok(hipError_t e) { return e == hipSuccess ? EMELK_ERR_NONE : EMELK_ERR_BACKEND; }

}  // namespace

extern "C" emel_error_type emelk_batch_decoder_create(const emelk_kv_geometry *g,
                                                      emelk_kv_actor *actor, emelk_kv_cache *cache,
                                                      const emelk_rope_table *rope,
                                                      int32_t max_batch, int32_t max_kv_len,
                                                      void *stream, emelk_batch_decoder **out) {
  if (out == nullptr) return EMELK_ERR_INVALID_REQUEST;
  *out = nullptr;
  uint64_t pool_bytes = 0;
  if (g == nullptr || actor == nullptr || cache == nullptr || rope == nullptr || max_batch <= 0 ||
      max_batch > EMELK_MAX_SEQUENCES || max_kv_len <= 0 ||
      emelk_kv_pool_bytes(g, &pool_bytes) != EMELK_ERR_NONE ||
      emelk_rope_table_positions(rope) < max_kv_len) {
    return EMELK_ERR_INVALID_REQUEST;
  }
  // page copies of the tail split run on the cache's stream; the decoder's
  // kernels must be ordered after them (and the copies after earlier appends)
  if (stream != emelk_kv_cache_stream(cache)) return EMELK_ERR_INVALID_REQUEST;
  const int32_t stride = (max_kv_len + g->block_tokens - 1) / g->block_tokens;
  if (stride > EMELK_MAX_BLOCKS_PER_SEQUENCE) return EMELK_ERR_INVALID_REQUEST;
  uint64_t ws = 0;
  if (emelk_attn_decode_workspace_size(g, max_batch, max_kv_len, &ws) != EMELK_ERR_NONE) {
    return EMELK_ERR_INVALID_REQUEST;
  }
  auto *d = new (std::nothrow) emelk_batch_decoder();
  if (d == nullptr) return EMELK_ERR_OUT_OF_MEMORY;
  d->g = *g;
  d->actor = actor;
  d->cache = cache;
  d->rope = rope;
  d->stream = static_cast<hipStream_t>(stream);
  d->max_batch = max_batch;
  d->max_kv_len = max_kv_len;
  d->stride = stride;
  d->ws_bytes = ws;
  const size_t tb = static_cast<size_t>(max_batch) * stride * sizeof(uint16_t);
  const size_t ib = static_cast<size_t>(max_batch) * sizeof(int32_t);
  bool ok = hipMalloc(reinterpret_cast<void **>(&d->d_tables), tb) == hipSuccess &&
            hipMalloc(reinterpret_cast<void **>(&d->d_pos), ib) == hipSuccess &&
            hipMalloc(reinterpret_cast<void **>(&d->d_kv_len), ib) == hipSuccess &&
            hipMalloc(&d->d_ws, ws) == hipSuccess;
  for (auto &s : d->st) {
    ok = ok && hipHostMalloc(reinterpret_cast<void **>(&s.tables), tb, hipHostMallocDefault) == hipSuccess &&
         hipHostMalloc(reinterpret_cast<void **>(&s.pos), ib, hipHostMallocDefault) == hipSuccess &&
         hipHostMalloc(reinterpret_cast<void **>(&s.kv_len), ib, hipHostMallocDefault) == hipSuccess &&
         hipEventCreateWithFlags(&s.uploaded, hipEventDisableTiming) == hipSuccess;
  }
  if (!ok) {
    emelk_batch_decoder_destroy(d);
    return EMELK_ERR_OUT_OF_MEMORY;
  }
  *out = d;
  return EMELK_ERR_NONE;
}

extern "C" void emelk_batch_decoder_destroy(emelk_batch_decoder *d) {
  if (d == nullptr) return;
  if (d->stream != nullptr) (void)hipStreamSynchronize(d->stream);
  else (void)hipDeviceSynchronize();
  if (d->d_tables) (void)hipFree(d->d_tables);
  if (d->d_pos) (void)hipFree(d->d_pos);
  if (d->d_kv_len) (void)hipFree(d->d_kv_len);
  if (d->d_ws) (void)hipFree(d->d_ws);
  for (auto &s : d->st) {
    if (s.tables) (void)hipHostFree(s.tables);
    if (s.pos) (void)hipHostFree(s.pos);
    if (s.kv_len) (void)hipHostFree(s.kv_len);
    if (s.uploaded) (void)hipEventDestroy(s.uploaded);
  }
  delete d;
}

extern "C" emel_error_type emelk_batch_decoder_begin_step(emelk_batch_decoder *d,
                                                          const int32_t *seq_ids, int32_t n_seq,
                                                          int32_t n_tokens,
                                                          int32_t *positions_out) {
  if (d == nullptr || seq_ids == nullptr || n_seq <= 0 || n_seq > d->max_batch || n_tokens <= 0) {
    return EMELK_ERR_INVALID_REQUEST;
  }
  for (int32_t i = 0; i < n_seq; ++i) {
    for (int32_t j = 0; j < i; ++j) {
      if (seq_ids[i] == seq_ids[j]) return EMELK_ERR_INVALID_REQUEST;  // one row per sequence
    }
  }
  auto &s = d->st[d->next_st];
  if (s.pending) {  // the copy engine may still read this staging set
    if (hipEventSynchronize(s.uploaded) != hipSuccess) return EMELK_ERR_BACKEND;
    s.pending = false;
  }
  int32_t max_kv = 0;
  for (int32_t i = 0; i < n_seq; ++i) {
    const int32_t len = emelk_kv_sequence_length(d->actor, seq_ids[i]);
    if (len < 0) return EMELK_ERR_INVALID_REQUEST;
    s.pos[i] = len;
    s.kv_len[i] = s.pos[i] + n_tokens;
    if (s.kv_len[i] > d->max_kv_len) return EMELK_ERR_INVALID_REQUEST;
    max_kv = std::max(max_kv, s.kv_len[i]);
  }
  // allocate_slots per sequence, all or nothing: a refusal rolls back the
  // sequences already extended in this step
  for (int32_t i = 0; i < n_seq; ++i) {
    int32_t err = 0;
    emelk_event_allocate_slots ev{seq_ids[i], n_tokens, nullptr, &err, emelk_kv_cache_copy_block,
                                  d->cache};
    if (!emelk_kv_allocate_slots(d->actor, &ev)) {
      for (int32_t j = 0; j < i; ++j) {
        int32_t rerr = 0;
        emelk_event_rollback_slots rb{seq_ids[j], n_tokens, nullptr, &rerr};
        (void)emelk_kv_rollback_slots(d->actor, &rb);
      }
      return err != 0 ? static_cast<emel_error_type>(err) : EMELK_ERR_INTERNAL;
    }
  }
  emel_error_type e = emelk_kv_export_block_tables(d->actor, seq_ids, n_seq, s.tables, d->stride);
  if (e != EMELK_ERR_NONE) return e;
  const size_t tb = static_cast<size_t>(n_seq) * d->stride * sizeof(uint16_t);
  const size_t ib = static_cast<size_t>(n_seq) * sizeof(int32_t);
  e = hip_ok(hipMemcpyAsync(d->d_tables, s.tables, tb, hipMemcpyHostToDevice, d->stream));
  if (e == EMELK_ERR_NONE) e = hip_ok(hipMemcpyAsync(d->d_pos, s.pos, ib, hipMemcpyHostToDevice, d->stream));
  if (e == EMELK_ERR_NONE) {
    e = hip_ok(hipMemcpyAsync(d->d_kv_len, s.kv_len, ib, hipMemcpyHostToDevice, d->stream));
  }
  if (e == EMELK_ERR_NONE) e = hip_ok(hipEventRecord(s.uploaded, d->stream));
  if (e != EMELK_ERR_NONE) return e;
  s.pending = true;
  if (positions_out != nullptr) std::memcpy(positions_out, s.pos, ib);
  d->next_st ^= 1;
  d->n_seq = n_seq;
  d->n_tokens = n_tokens;
  d->step_max_kv = max_kv;
  d->step_open = true;
  return EMELK_ERR_NONE;
}

extern "C" emel_error_type emelk_batch_decoder_layer(emelk_batch_decoder *d, int32_t layer,
                                                     const float *q_in, float *q_roped,
                                                     const float *k_rows, const float *v_rows,
                                                     const float *q_norm, const float *k_norm,
                                                     int32_t v_rms, float rms_epsilon, float scale,
                                                     float *out) {
  if (d == nullptr || !d->step_open || out == nullptr || q_roped == nullptr) {
    return EMELK_ERR_INVALID_REQUEST;
  }
  void *kp = emelk_kv_cache_k_pool(d->cache);
  void *vp = emelk_kv_cache_v_pool(d->cache);
  emel_error_type e = emelk_kv_qkv_rope_append(
      &d->g, kp, vp, layer, q_in, q_roped, k_rows, v_rows, d->n_seq, d->n_tokens, d->d_pos,
      d->d_tables, d->stride, d->rope, q_norm, k_norm, v_rms, rms_epsilon, d->stream);
  if (e != EMELK_ERR_NONE) return e;
  if (d->n_tokens == 1) {
    const int32_t plan_len = d->fixed_plan ? d->max_kv_len : d->step_max_kv;
    return emelk_attn_decode(&d->g, kp, vp, layer, q_roped, out, d->n_seq, d->d_kv_len, plan_len,
                             d->d_tables, d->stride, scale, d->d_ws, d->ws_bytes, d->stream);
  }
  return emelk_attn_prefill_chunk(&d->g, kp, vp, layer, q_roped, out, d->n_seq, d->n_tokens,
                                  d->d_pos, d->d_tables, d->stride, scale, d->stream);
}

extern "C" emel_error_type emelk_batch_decoder_set_fixed_plan(emelk_batch_decoder *d, int32_t on) {
  if (d == nullptr) return EMELK_ERR_INVALID_REQUEST;
  d->fixed_plan = on != 0;
  return EMELK_ERR_NONE;
}
