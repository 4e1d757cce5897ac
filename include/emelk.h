/*
 * emelk — MI355X (gfx950) KV-cache hot path for stateforward/emel.cpp.
 *
 * C ABI: plain pointers and sizes only.  Device pointers are HIP device
 * addresses; `stream` is a hipStream_t passed as void* (NULL = the default
 * stream).  Every entry point returns emel_error_type
 * (reference include/emel/emel.h:11) with the memory/kv bit values of
 * src/emel/memory/kv/errors.hpp:7-14, or `bool` where the reference event API
 * returns bool.  Kernel entry points only enqueue work; they never
 * synchronise the stream.
 *
 * Paths in citations are relative to the reference checkout.
 */
#ifndef EMELK_H
#define EMELK_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint32_t emel_error_type; /* include/emel/emel.h:11 */

/* src/emel/memory/kv/errors.hpp:7-14 */
enum {
  EMELK_ERR_NONE = 0u,
  EMELK_ERR_INVALID_REQUEST = 1u << 0,
  EMELK_ERR_BACKEND = 1u << 1,
  EMELK_ERR_INTERNAL = 1u << 2,
  EMELK_ERR_OUT_OF_MEMORY = 1u << 3,
  EMELK_ERR_UNTRACKED = 1u << 4,
};

/* Geometry contract, src/emel/memory/view.hpp:10-19. */
#define EMELK_MAX_SEQUENCES 256
#define EMELK_MAX_BLOCKS_PER_SEQUENCE 4096
#define EMELK_MAX_BLOCKS 32768
#define EMELK_DEFAULT_BLOCK_TOKENS 16
#define EMELK_INVALID_KV_BLOCK 0xFFFFu

/* ------------------------------------------------------------------------ */
/* Host KV block-map actor (src/emel/memory/kv/sm.hpp:364-507).             */
/* Event structs are layout-identical to src/emel/memory/events.hpp:9-62.   */
/* ------------------------------------------------------------------------ */

typedef struct emelk_event_reserve { /* events.hpp:9-14 */
  int32_t max_sequences;
  int32_t max_blocks;
  int32_t block_tokens;
  int32_t *error_out;
} emelk_event_reserve;

typedef struct emelk_event_allocate_sequence { /* events.hpp:16-19 */
  int32_t seq_id;
  int32_t *error_out;
} emelk_event_allocate_sequence;

/* allocate_slots::copy_block_fn, events.hpp:22-26 */
typedef bool (*emelk_copy_block_fn)(int32_t src_block, int32_t dst_block, int32_t block_tokens,
                                    void *user_data, int32_t *error_out);

typedef struct emelk_event_allocate_slots { /* events.hpp:21-34 */
  int32_t seq_id;
  int32_t token_count;
  int32_t *block_count_out;
  int32_t *error_out;
  emelk_copy_block_fn copy_block;
  void *copy_block_user_data;
} emelk_event_allocate_slots;

typedef bool (*emelk_copy_state_fn)(int32_t src_slot, int32_t dst_slot, void *user_data,
                                    int32_t *error_out);

typedef struct emelk_event_branch_sequence { /* events.hpp:36-45 */
  int32_t parent_seq_id;
  int32_t child_seq_id;
  emelk_copy_state_fn copy_state;
  void *copy_state_user_data;
  int32_t *error_out;
} emelk_event_branch_sequence;

typedef struct emelk_event_free_sequence { /* events.hpp:47-50 */
  int32_t seq_id;
  int32_t *error_out;
} emelk_event_free_sequence;

typedef struct emelk_event_rollback_slots { /* events.hpp:52-57 */
  int32_t seq_id;
  int32_t token_count;
  int32_t *block_count_out;
  int32_t *error_out;
} emelk_event_rollback_slots;

/* view::snapshot, src/emel/memory/view.hpp:59-117 (same member order). */
typedef struct emelk_view_snapshot {
  int32_t max_sequences;
  int32_t block_tokens;
  uint8_t sequence_active[EMELK_MAX_SEQUENCES];
  int32_t sequence_length_values[EMELK_MAX_SEQUENCES];
  int32_t sequence_kv_block_count[EMELK_MAX_SEQUENCES];
  uint16_t sequence_kv_blocks[EMELK_MAX_SEQUENCES][EMELK_MAX_BLOCKS_PER_SEQUENCE];
  int32_t sequence_recurrent_slot[EMELK_MAX_SEQUENCES];
} emelk_view_snapshot;

typedef struct emelk_event_capture_view { /* events.hpp:59-62 */
  emelk_view_snapshot *snapshot_out;
  int32_t *error_out;
} emelk_event_capture_view;

/* New events (no counterpart in the reference, which never evicts or
 * compacts; built on its copy_block mechanism, kv/actions.hpp:218-242). */
typedef struct emelk_event_evict_blocks {
  int32_t seq_id;
  const int32_t *logical_blocks; /* distinct logical block indices of seq_id */
  int32_t block_count;
  int32_t *tokens_removed_out;
  int32_t *error_out;
} emelk_event_evict_blocks;

typedef struct emelk_event_compact {
  int32_t *moves_out;      /* host [max_moves][2] = (src_block, dst_block) */
  int32_t max_moves;
  int32_t *move_count_out;
  int32_t *error_out;
} emelk_event_compact;

/* kv_binding, src/emel/memory/hybrid/context.hpp:21-30.  The reference's
 * dispatch functions take `const event&`, which the platform C++ ABI passes
 * as a pointer, so a filled emelk_kv_binding can be copied bit for bit into
 * emel::memory::hybrid::kv_binding. */
typedef struct emelk_kv_binding {
  void *actor;
  bool (*dispatch_reserve)(void *, const emelk_event_reserve *);
  bool (*dispatch_allocate_sequence)(void *, const emelk_event_allocate_sequence *);
  bool (*dispatch_allocate_slots)(void *, const emelk_event_allocate_slots *);
  bool (*dispatch_branch_sequence)(void *, const emelk_event_branch_sequence *);
  bool (*dispatch_free_sequence)(void *, const emelk_event_free_sequence *);
  bool (*dispatch_rollback_slots)(void *, const emelk_event_rollback_slots *);
  bool (*dispatch_capture_view)(void *, const emelk_event_capture_view *);
} emelk_kv_binding;

typedef struct emelk_kv_actor emelk_kv_actor;

/* Construct / destroy (the reference sm is default-constructed, sm.hpp:370). */
emelk_kv_actor *emelk_kv_actor_create(void);
void emelk_kv_actor_destroy(emelk_kv_actor *actor);

/* kv::sm::process_event overloads, src/emel/memory/kv/sm.hpp:372-465. */
bool emelk_kv_reserve(emelk_kv_actor *actor, const emelk_event_reserve *ev);
bool emelk_kv_allocate_sequence(emelk_kv_actor *actor, const emelk_event_allocate_sequence *ev);
bool emelk_kv_allocate_slots(emelk_kv_actor *actor, const emelk_event_allocate_slots *ev);
bool emelk_kv_branch_sequence(emelk_kv_actor *actor, const emelk_event_branch_sequence *ev);
bool emelk_kv_free_sequence(emelk_kv_actor *actor, const emelk_event_free_sequence *ev);
bool emelk_kv_rollback_slots(emelk_kv_actor *actor, const emelk_event_rollback_slots *ev);
bool emelk_kv_capture_view(emelk_kv_actor *actor, const emelk_event_capture_view *ev);
/* kv::sm::view() (sm.hpp:480-499): cached snapshot, refreshed when dirty. */
const emelk_view_snapshot *emelk_kv_view(emelk_kv_actor *actor);
/* snapshot::lookup_kv_block (view.hpp:87-109) on the cached view. */
int32_t emelk_kv_lookup_kv_block(emelk_kv_actor *actor, int32_t seq_id, int32_t pos);

bool emelk_kv_evict_blocks(emelk_kv_actor *actor, const emelk_event_evict_blocks *ev);
bool emelk_kv_compact(emelk_kv_actor *actor, const emelk_event_compact *ev);

/* hybrid::bind_kv_actor (hybrid/context.hpp:77-89). */
void emelk_kv_bind(emelk_kv_actor *actor, emelk_kv_binding *binding_out);

/* Copies the block rows of seq_ids[0..n_seq) into a host table
 * [n_seq][table_stride] (entries past a sequence's block count are
 * EMELK_INVALID_KV_BLOCK).  Replaces the per-decode snapshot walk of
 * kv_addressing_from_request (text/generator/detail.hpp:1010-1014). */
emel_error_type emelk_kv_export_block_tables(emelk_kv_actor *actor, const int32_t *seq_ids,
                                             int32_t n_seq, uint16_t *table_out,
                                             int32_t table_stride);

/* Test and bench hook: replaces the free stack's pop order.  order[0] is
 * popped first; it must be a permutation of the currently free block ids.
 * Used to install the seeded random page permutations of the workloads
 * through the real allocate_slots path. */
emel_error_type emelk_kv_set_free_order(emelk_kv_actor *actor, const uint16_t *order,
                                        int32_t count);

/* Refcount of a physical block (kv/detail.hpp:46-97 block_pool). */
int32_t emelk_kv_block_refs(emelk_kv_actor *actor, int32_t block_id);
int32_t emelk_kv_free_count(emelk_kv_actor *actor);
/* Token count of an active sequence (snapshot::sequence_length_values,
 * view.hpp:59-117, without rebuilding the snapshot); -1 if inactive or
 * out of range. */
int32_t emelk_kv_sequence_length(emelk_kv_actor *actor, int32_t seq_id);

/* ------------------------------------------------------------------------ */
/* Device page pool and kernels (gfx950).                                   */
/* ------------------------------------------------------------------------ */

enum { EMELK_KV_F16 = 1, EMELK_KV_Q8_0 = 8 };

typedef struct emelk_kv_geometry {
  int32_t n_layer;
  int32_t n_head;      /* query heads */
  int32_t n_head_kv;   /* key/value heads (GQA: n_head % n_head_kv == 0) */
  int32_t head_dim;    /* 64, 128, 256 or 512 (q8_0 at 512: prefill runs row by row) */
  int32_t block_tokens;/* tokens per page */
  int32_t max_blocks;  /* pages in the pool */
  int32_t kv_type;     /* EMELK_KV_F16 or EMELK_KV_Q8_0 */
} emelk_kv_geometry;

/* Bytes of one pool (K or V; both have the same size).  Layout:
 *   f16 : [layer][page][kv_head][block_tokens][head_dim] halves
 *   q8_0: [layer][page][kv_head] regions of block_tokens*head_dim int8 values
 *         followed by block_tokens*head_dim/32 f16 scales (GGUF q8_0 content,
 *         split into value and scale planes per page and head). */
emel_error_type emelk_kv_pool_bytes(const emelk_kv_geometry *g, uint64_t *bytes_out);

/* store_attention_kv_cache (text/generator/detail.hpp:3294-3332) for a batch:
 * k_rows/v_rows are fp32 [n_seq][n_tokens][n_head_kv*head_dim]; token t of
 * sequence s lands at logical position positions[s] + t through
 * block_tables[s*table_stride + pos/block_tokens].  f16 pools: RNE rounding
 * (quant::fp32_to_fp16, kernel/detail.hpp:372-392).  q8_0 pools: per 32
 * values quantize_row_q8_0_strided (kernel/detail.hpp:804-824). */
emel_error_type emelk_kv_append(const emelk_kv_geometry *g, void *k_pool, void *v_pool,
                                int32_t layer, const float *k_rows, const float *v_rows,
                                int32_t n_seq, int32_t n_tokens, const int32_t *positions,
                                const uint16_t *block_tables, int32_t table_stride, void *stream);

/* Block-table gather: logical tokens [0, lengths[s]) of layer `layer` into
 * dense head-major outputs [n_seq][n_head_kv][out_tokens][...]: f16 rows of
 * head_dim halves, or GGUF block_q8_0 rows (head_dim/32 blocks of 34 bytes,
 * kernel/detail.hpp:226-229).  Addressing is physical_kv_position +
 * flash_layer_cache_head_position_offset (text/generator/detail.hpp:2976-3048). */
emel_error_type emelk_kv_gather(const emelk_kv_geometry *g, const void *k_pool,
                                const void *v_pool, int32_t layer, int32_t n_seq,
                                const int32_t *lengths, const uint16_t *block_tables,
                                int32_t table_stride, void *k_out, void *v_out,
                                int32_t out_tokens, void *stream);

/* Batched page copy for every layer, K and V: moves is device int32
 * [n_moves][2] = (src_block, dst_block).  copy_attention_kv_block
 * (text/generator/detail.hpp:3334-3417) applied to many pages in one launch.
 * Sources and destinations must be disjoint sets (eviction compaction and the
 * copy-on-write tail split both satisfy this). */
emel_error_type emelk_kv_copy_blocks(const emelk_kv_geometry *g, void *k_pool, void *v_pool,
                                     const int32_t *moves, int32_t n_moves, void *stream);

/* Split-K flash-decode GQA attention for one layer; replaces compute_attention
 * (text/generator/detail.hpp:3153-3230) and the flash route
 * (kernel/detail.hpp:5238-5291).  q: fp32 [n_seq][n_head][head_dim] (rounded
 * to fp16 on load, as round_q_for_nonflash does); out: fp32, same shape.
 * kv_lens: device int32 [n_seq], tokens to attend (position + 1), each in
 * [1, max_kv_len].  scale multiplies q.k.  workspace: device scratch of
 * emelk_attn_decode_workspace_size bytes.
 * emelk_attn_decode_workspace_size(n_seq, max_kv_len) is enough for every
 * call with at most n_seq sequences and max_kv_len at most max_kv_len (the
 * split count rises as the batch shrinks, so the exact need of one call is
 * not monotone in n_seq); emelk_attn_decode_plan reports the host split
 * plan (tokens_per_split, n_splits per sequence) and the exact workspace need
 * of one call with these arguments.  For 2 to 64 sequences the device
 * rebalances the splits over the actual lengths (never more splits than
 * n_seq * n_splits, each at most tokens_per_split tokens), so the summation
 * order of a sequence depends on the batch's lengths; results are
 * deterministic for the same inputs.  The reference has no counterpart: its
 * CPU route needs no partials. */
emel_error_type emelk_attn_decode_workspace_size(const emelk_kv_geometry *g, int32_t n_seq,
                                                 int32_t max_kv_len, uint64_t *bytes_out);
emel_error_type emelk_attn_decode_plan(const emelk_kv_geometry *g, int32_t n_seq,
                                       int32_t max_kv_len, int32_t *tokens_per_split,
                                       int32_t *n_splits, uint64_t *bytes_out);
emel_error_type emelk_attn_decode(const emelk_kv_geometry *g, const void *k_pool,
                                  const void *v_pool, int32_t layer, const float *q, float *out,
                                  int32_t n_seq, const int32_t *kv_lens, int32_t max_kv_len,
                                  const uint16_t *block_tables, int32_t table_stride, float scale,
                                  void *workspace, uint64_t workspace_bytes, void *stream);
/* One decode step's store + attend in one launch, as
 * compute_layer_attention_residual does per token (store_attention_kv_cache
 * then compute_attention, text/generator/detail.hpp:3806-3840): for each
 * sequence the token at position kv_lens[s] - 1, rows k_rows/v_rows fp32
 * [n_seq][n_head_kv * head_dim], is written into the pools exactly as
 * emelk_kv_append writes it (f16, or q8_0 quantized on the fly; skipped on
 * an invalid page) and attended together with the kv_lens[s] - 1 tokens
 * before it.  Same result as emelk_kv_append(positions = kv_lens - 1,
 * n_tokens = 1) followed by emelk_attn_decode, up to summation order. */
emel_error_type emelk_attn_decode_append(const emelk_kv_geometry *g, void *k_pool, void *v_pool,
                                         int32_t layer, const float *k_rows, const float *v_rows,
                                         const float *q, float *out, int32_t n_seq,
                                         const int32_t *kv_lens, int32_t max_kv_len,
                                         const uint16_t *block_tables, int32_t table_stride,
                                         float scale, void *workspace, uint64_t workspace_bytes,
                                         void *stream);

/* Decode on contiguous caches: the flash route's request
 * (make_flash_attn_request, text/generator/detail.hpp:3232-3292, taken for
 * an identity block map, generator/guards.hpp:890-906), whose K and V caches
 * are head-major [layer][kv_head][capacity][head_dim].  Sequence s holds
 * token t at page s * (seq_stride_tokens / block_tokens) + t / block_tokens,
 * row t % block_tokens, of the pools' usual layout; no block table is read.
 * With block_tokens = capacity and max_blocks = 1 (one page per layer,
 * holding every KV head's capacity rows) the pools are exactly the flash
 * caches, and n_seq = 1, seq_stride_tokens = capacity.  With k_rows and
 * v_rows non-NULL the step's token (position kv_lens[s] - 1) is stored first,
 * as emelk_attn_decode_append does; both NULL: attend only.  Same results as
 * emelk_attn_decode / _append with the equivalent identity tables.
 * seq_stride_tokens must be a multiple of block_tokens and at least
 * max_kv_len, and n_seq * seq_stride_tokens / block_tokens at most
 * max_blocks.  Workspace as for emelk_attn_decode. */
emel_error_type emelk_attn_decode_contiguous(const emelk_kv_geometry *g, void *k_pool,
                                             void *v_pool, int32_t layer, const float *k_rows,
                                             const float *v_rows, const float *q, float *out,
                                             int32_t n_seq, const int32_t *kv_lens,
                                             int32_t max_kv_len, int32_t seq_stride_tokens,
                                             float scale, void *workspace,
                                             uint64_t workspace_bytes, void *stream);

/* Allocation-free decode.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same results as
 * emelk_attn_decode (k_rows == v_rows == NULL) or emelk_attn_decode_append
 * (both non-NULL), with the split partials in a static device array of
 * EMELK_DECODE_STATIC_SCRATCH_BYTES per GPU instead of a caller workspace;
 * it calls no allocating routine.  A call whose exact need
 * (emelk_attn_decode_plan's bytes_out) exceeds that size returns
 * EMELK_ERR_OUT_OF_MEMORY before touching the device.  Every call on one
 * GPU uses that GPU's one array: calls that overlap on one GPU (other
 * streams, other threads) race.  The stream must belong to the current
 * device (a stream of another device returns EMELK_ERR_INVALID_REQUEST). */
#define EMELK_DECODE_STATIC_SCRATCH_BYTES (16u << 20)
emel_error_type emelk_attn_decode_noalloc(const emelk_kv_geometry *g, void *k_pool, void *v_pool,
                                          int32_t layer, const float *k_rows, const float *v_rows,
                                          const float *q, float *out, int32_t n_seq,
                                          const int32_t *kv_lens, int32_t max_kv_len,
                                          const uint16_t *block_tables, int32_t table_stride,
                                          float scale, void *stream);

/* Chunked-prefill attention for one layer: q fp32
 * [n_seq][n_q][n_head][head_dim]; row r of sequence s attends causally to
 * logical positions [0, q_start[s] + r] (the chunk must already be appended).
 * Replaces the per-row store + attend loop of run_prefill
 * (text/generator/detail.hpp:4297-4372).  A negative q_start[s] makes every
 * row of sequence s attend to nothing: its rows are written as zeros, on
 * every route.  head_dim 64 and 128 run on MFMA,
 * f16 and q8_0 pools alike (q8_0 K values enter the score MFMAs exactly, as
 * two fp16 parts, values of magnitude 65520 or more excepted, and q8_0 V
 * values the same way in the P.V MFMAs, with P as two fp16 parts), and so do
 * head_dim 256 and, on f16 pools, 512.  q8_0 at head_dim 512 runs row by
 * row through the decode kernel (n_seq * n_q <= 65535, and a row's
 * context, table_stride * block_tokens tokens at most, must fit 1022
 * pages). */
emel_error_type emelk_attn_prefill_chunk(const emelk_kv_geometry *g, const void *k_pool,
                                         const void *v_pool, int32_t layer, const float *q,
                                         float *out, int32_t n_seq, int32_t n_q,
                                         const int32_t *q_start, const uint16_t *block_tables,
                                         int32_t table_stride, float scale, void *stream);

/* RoPE parameters: the reference's rope_pairing (text/generator/detail.hpp:39-50;
 * normal = {2, 2, 1, 0}, neox = {1, 1, 0, 1}) plus n_rot and the frequency base
 * of apply_rope_pairing (detail.hpp:2905-2936).  Pair p rotates dims
 * p*x0_stride and p*x1_stride + x1_offset + x1_half_rot_offset*(rot_dim/2),
 * rot_dim = min(n_rot, head_dim). */
typedef struct emelk_rope_params {
  int32_t n_rot;
  int32_t x0_stride;
  int32_t x1_stride;
  int32_t x1_offset;
  int32_t x1_half_rot_offset;
  float freq_base;
} emelk_rope_params;

/* Device table of (cos, sin) per (position, pair) for positions
 * [0, max_positions), computed once on the host exactly as
 * apply_rope_pairing does per call: theta = float(position), then
 * theta *= powf(freq_base, -2/rot_dim) after each pair, cosf/sinf of each
 * theta.  Pairings whose pairs overlap or leave the head are rejected.
 * The table is hipMalloc'd and uploaded on `stream` (synchronously). */
typedef struct emelk_rope_table emelk_rope_table;
emel_error_type emelk_rope_table_create(const emelk_rope_params *params, int32_t head_dim,
                                        int32_t max_positions, void *stream,
                                        emelk_rope_table **table_out);
void emelk_rope_table_destroy(emelk_rope_table *table);
/* Positions covered by the table (0 for NULL). */
int32_t emelk_rope_table_positions(const emelk_rope_table *table);

/* The step before append, fused: for every token of every sequence, the
 * steps of compute_layer_attention_residual (text/generator/detail.hpp:3806-3825)
 * and of the chunked-prefill row loop (detail.hpp:4335-4360) between the
 * Q/K/V projections and store_attention_kv_cache:
 *   q_norm/k_norm (optional, [head_dim]): apply_headwise_rms_norm
 *     (detail.hpp:1060-1090) on every head of q / k;
 *   v_rms != 0: apply_rms_norm_in_place (detail.hpp:1092-1111) on the whole
 *     v vector of the token;
 *   RoPE (apply_rope_pairing) on q and k at position positions[s] + t;
 *   q_out (fp32, may alias q_in) receives q; k and v are appended to the
 *   pools as emelk_kv_append does.
 * q_in/q_out: fp32 [n_seq][n_tokens][n_head][head_dim]; k_rows/v_rows:
 * fp32 [n_seq][n_tokens][n_head_kv][head_dim].  Tokens whose position is
 * outside the rope table, the block table or the pool are skipped (nothing
 * written).  Products and sums are evaluated unfused, in the reference's
 * order, so results are bit-exact against that arithmetic. */
emel_error_type emelk_kv_qkv_rope_append(const emelk_kv_geometry *g, void *k_pool, void *v_pool,
                                         int32_t layer, const float *q_in, float *q_out,
                                         const float *k_rows, const float *v_rows,
                                         int32_t n_seq, int32_t n_tokens,
                                         const int32_t *positions, const uint16_t *block_tables,
                                         int32_t table_stride, const emelk_rope_table *rope,
                                         const float *q_norm, const float *k_norm, int32_t v_rms,
                                         float rms_epsilon, void *stream);

/* Device KV owner: allocates both pools (hipMalloc) and serves as the
 * allocate_slots copy_block callback target (text/generator/context.hpp:36-50). */
typedef struct emelk_kv_cache emelk_kv_cache;
emel_error_type emelk_kv_cache_create(const emelk_kv_geometry *g, void *stream,
                                      emelk_kv_cache **cache_out);
void emelk_kv_cache_destroy(emelk_kv_cache *cache);
void *emelk_kv_cache_k_pool(emelk_kv_cache *cache);
void *emelk_kv_cache_v_pool(emelk_kv_cache *cache);
/* The stream the cache was created with (its page copies run there). */
void *emelk_kv_cache_stream(const emelk_kv_cache *cache);
/* emelk_copy_block_fn: user_data is an emelk_kv_cache*.  Enqueues the copy of
 * one page (all layers, K and V) on the cache's stream. */
bool emelk_kv_cache_copy_block(int32_t src_block, int32_t dst_block, int32_t block_tokens,
                               void *user_data, int32_t *error_out);
/* capture_view into device memory (kv/sm.hpp:448-465, memory/view.hpp:59-117):
 * the actor's snapshot is copied to view_dev (sizeof(emelk_view_snapshot),
 * 2.1 MB) on the cache's stream, after the page copies already enqueued
 * there.  Device consumers read it in place: sequence_kv_blocks is a block
 * table with rows by sequence id and table_stride
 * EMELK_MAX_BLOCKS_PER_SEQUENCE, and sequence_length_values holds kv_lens,
 * so sequences 0..n-1 decode straight from the view.  (A decode step that
 * needs only some rows moves fewer bytes with emelk_kv_export_block_tables.) */
emel_error_type emelk_kv_cache_upload_view(emelk_kv_cache *cache, emelk_kv_actor *actor,
                                           emelk_view_snapshot *view_dev);

/* Multi-sequence step executor: the reference generator's per-token flow
 * (allocate_slots with copy_kv_cache_block, text/generator/actions.hpp:460-474;
 * capture_view, actions.hpp:270-281; per-layer compute on the sequence's
 * block table, detail.hpp:1010-1014 and 3745-3840) for a batch of sequences
 * instead of the single k_sequence_id = 0 (text/generator/context.hpp:33).
 * It uses the actor, the device cache and the rope table it is given (all
 * must outlive it) and allocates its own block-table, position and
 * workspace buffers for up to max_batch sequences of up to max_kv_len
 * tokens.  `stream` must be the stream the cache was created with, so page
 * copies and kernels stay ordered. */
typedef struct emelk_batch_decoder emelk_batch_decoder;
emel_error_type emelk_batch_decoder_create(const emelk_kv_geometry *g, emelk_kv_actor *actor,
                                           emelk_kv_cache *cache, const emelk_rope_table *rope,
                                           int32_t max_batch, int32_t max_kv_len, void *stream,
                                           emelk_batch_decoder **decoder_out);
void emelk_batch_decoder_destroy(emelk_batch_decoder *decoder);
/* Extends each listed sequence by n_tokens (allocate_slots; a shared tail
 * page is split on the device through emelk_kv_cache_copy_block).  All or
 * nothing: if one sequence is refused, the ones already extended are rolled
 * back and its error is returned.  Uploads the block tables and positions on
 * the stream; positions_out (host, optional) receives each sequence's first
 * new position. */
emel_error_type emelk_batch_decoder_begin_step(emelk_batch_decoder *decoder,
                                               const int32_t *seq_ids, int32_t n_seq,
                                               int32_t n_tokens, int32_t *positions_out);
/* One layer of the open step: emelk_kv_qkv_rope_append, then attention over
 * every sequence's history including the new tokens (emelk_attn_decode when
 * n_tokens == 1, emelk_attn_prefill_chunk otherwise).  q_in/q_roped/out:
 * [n_seq][n_tokens][n_head][head_dim] fp32 (q_roped may alias q_in);
 * k_rows/v_rows: [n_seq][n_tokens][n_head_kv][head_dim] fp32. */
/* Graph-stable launches (no counterpart in the reference, whose generator
 * runs on the CPU): when on, each layer's attention is planned for the
 * decoder's max_kv_len instead of the step's longest sequence, so a layer
 * call's launches depend only on n_seq and n_tokens.  A captured graph of
 * the layer calls then stays valid for later steps of the same shape
 * (begin_step runs outside the graph and refreshes the device tables,
 * positions and lengths the kernels read).  Off by default: the step's own
 * length gives better split sizes while contexts are short. */
emel_error_type emelk_batch_decoder_set_fixed_plan(emelk_batch_decoder *decoder, int32_t on);
emel_error_type emelk_batch_decoder_layer(emelk_batch_decoder *decoder, int32_t layer,
                                          const float *q_in, float *q_roped, const float *k_rows,
                                          const float *v_rows, const float *q_norm,
                                          const float *k_norm, int32_t v_rms, float rms_epsilon,
                                          float scale, float *out);

/* ---- Batch planner (host) ----------------------------------------------
 * Splits a batch of tokens into steps, as emel::batch::planner::sm does
 * (src/emel/batch/planner/sm.hpp:20-146, detail.hpp:129-359,
 * modes/{simple,equal,sequential}/actions.hpp): `simple` cuts the tokens
 * into chunks of the step size; `sequential` grows each step along tokens
 * whose sequence set is a subset of the current one; `equal` takes the same
 * number of tokens from every sequence of a group of non-overlapping
 * sequences (consecutive primary ids when equal_sequential).  An equal step
 * is the shape emelk_batch_decoder_begin_step takes; see
 * emelk_plan_step_sequences. */
#define EMELK_PLAN_MAX_STEPS 4096 /* batch/planner/context.hpp:7 */
#define EMELK_PLAN_SEQ_WORDS 4    /* 256 sequences: context.hpp:8-9 */

typedef enum emelk_plan_mode {
  EMELK_PLAN_SIMPLE = 0,
  EMELK_PLAN_EQUAL = 1,
  EMELK_PLAN_SEQUENTIAL = 2
} emelk_plan_mode;

/* Planner error bits (batch/planner/errors.hpp:6-25). */
#define EMELK_PLAN_ERR_INVALID_REQUEST (1u << 0)
#define EMELK_PLAN_ERR_INVALID_TOKEN_DATA (1u << 1)
#define EMELK_PLAN_ERR_INVALID_STEP_SIZE (1u << 2)
#define EMELK_PLAN_ERR_INVALID_SEQUENCE_METADATA (1u << 3)
#define EMELK_PLAN_ERR_INVALID_SEQUENCE_ID (1u << 4)
#define EMELK_PLAN_ERR_INVALID_SEQUENCE_MASK (1u << 5)
#define EMELK_PLAN_ERR_MULTIPLE_BITS_IN_MASK (1u << 6)
#define EMELK_PLAN_ERR_INVALID_MODE (1u << 8)
#define EMELK_PLAN_ERR_OUTPUT_PLAN_FULL (1u << 9)
#define EMELK_PLAN_ERR_OUTPUT_INDICES_FULL (1u << 10)
#define EMELK_PLAN_ERR_OUTPUT_STEPS_FULL (1u << 11)
#define EMELK_PLAN_ERR_PLANNING_PROGRESS_STALLED (1u << 12)
#define EMELK_PLAN_ERR_ALGORITHM_FAILED (1u << 13)
#define EMELK_PLAN_ERR_INTERNAL_ERROR (1u << 15)

/* event::plan_request (batch/planner/events.hpp:24-42) without the
 * callbacks.  seq_masks: n_tokens rows of seq_mask_words uint64 words (bit s
 * = sequence s); seq_primary_ids: one sequence id per token; with neither,
 * every token is on sequence 0.  The reference's default seq_mask_words is
 * 1 and equal_sequential true. */
typedef struct emelk_plan_request {
  const int32_t *token_ids;
  int32_t n_tokens;
  int32_t n_steps;  /* step size; <= 0 means n_tokens */
  int32_t mode;     /* emelk_plan_mode */
  const uint64_t *seq_masks;
  int32_t seq_masks_count;
  const int32_t *seq_primary_ids;
  int32_t seq_primary_ids_count;
  int32_t equal_sequential;
  int32_t seq_mask_words;
  const int8_t *output_mask;
  int32_t output_mask_count;
  int32_t output_all;
} emelk_plan_request;

/* events::plan_done (events.hpp:64-73): step s holds the token indices
 * step_token_indices[step_token_offsets[s] .. step_token_offsets[s+1]) and
 * has step_sizes[s] of them.  Counts are zero after a refused request. */
typedef struct emelk_plan_result {
  int32_t step_count;
  int32_t total_outputs;
  int32_t token_indices_count;
  int32_t step_sizes[EMELK_PLAN_MAX_STEPS];
  int32_t step_token_indices[EMELK_PLAN_MAX_STEPS];
  int32_t step_token_offsets[EMELK_PLAN_MAX_STEPS + 1];
} emelk_plan_result;

/* The planner's process_event: true iff a plan was produced; *error_out
 * (optional) receives the error bits (0 on success).  Replaces
 * Planner::process_event (batch/planner/sm.hpp:130-136). */
bool emelk_batch_plan(const emelk_plan_request *request, emelk_plan_result *result,
                      uint32_t *error_out);
/* One mode's planner with the step size given (modes::*::sm with
 * plan_scratch::effective_step_size set by the caller), without the outer
 * input validation and step-size normalisation. */
bool emelk_batch_plan_mode(const emelk_plan_request *request, int32_t effective_step_size,
                           emelk_plan_result *result, uint32_t *error_out);
/* The decoder shape of plan step `step`: its tokens must form runs of one
 * sequence each, all runs of equal length (what `equal` produces, and any
 * single-sequence step).  Writes the run sequences in order to seq_ids_out
 * (capacity EMELK_MAX_SEQUENCES) and the run length to *n_tokens_out. */
emel_error_type emelk_plan_step_sequences(const emelk_plan_request *request,
                                          const emelk_plan_result *result, int32_t step,
                                          int32_t *seq_ids_out, int32_t *n_seq_out,
                                          int32_t *n_tokens_out);

/* Library version and the device the kernels were built for. */
const char *emelk_build_info(void);

#ifdef __cplusplus
}
#endif

#endif /* EMELK_H */
