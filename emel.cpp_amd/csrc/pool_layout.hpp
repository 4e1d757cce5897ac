// Device page-pool layout shared by every kernel.
//
// One pool per K and per V.  A page holds `block_tokens` consecutive logical
// positions of one sequence for every KV head of one layer; pages of a layer
// are contiguous, layers are contiguous:
//
//   f16 : region(layer, page, kv_head) = block_tokens x head_dim halves,
//         row t (token within page) at t*head_dim.
//   q8_0: region(layer, page, kv_head) = block_tokens*head_dim int8 values
//         (row-major, as f16) followed by block_tokens*head_dim/32 f16 scales
//         (scale of token t, 32-value block j at t*head_dim/32 + j).
//
// Head-major inside a page keeps every (page, head) a single contiguous run
// (8 KiB at head_dim 128, 32-token pages) so the decode kernel streams it
// with 16-byte loads, and a page move is one contiguous copy per layer.
// The reference keeps two layouts (token-major key_cache and head-major
// flash_key_cache, text/generator/detail.hpp:2984-3048); this one pool
// serves both of its access patterns.
#pragma once

#include <stdint.h>

#include "emelk.h"

namespace emelk {

struct pool_layout {
  int32_t n_layer = 0;
  int32_t n_head = 0;
  int32_t n_head_kv = 0;
  int32_t head_dim = 0;
  int32_t block_tokens = 0;
  int32_t max_blocks = 0;
  int32_t kv_type = 0;
  uint64_t region_bytes = 0;  // one (layer, page, kv_head)
  uint64_t page_bytes = 0;    // one (layer, page): n_head_kv regions
  uint64_t layer_bytes = 0;   // one layer: max_blocks pages
  uint64_t pool_bytes = 0;

  __host__ __device__ uint64_t region_offset(int32_t layer, int32_t page, int32_t kvh) const {
    return (static_cast<uint64_t>(layer) * static_cast<uint64_t>(max_blocks) +
            static_cast<uint64_t>(page)) *
               page_bytes +
           static_cast<uint64_t>(kvh) * region_bytes;
  }
  // q8_0: byte offset of the scale plane inside a region.
  __host__ __device__ uint64_t scale_plane() const {
    return static_cast<uint64_t>(block_tokens) * static_cast<uint64_t>(head_dim);
  }
};

// Validates the geometry and fills the derived sizes.  Returns an emel error.
inline emel_error_type make_pool_layout(const emelk_kv_geometry *g, pool_layout &out) {
  if (g == nullptr) return EMELK_ERR_INVALID_REQUEST;
  const bool type_ok = g->kv_type == EMELK_KV_F16 || g->kv_type == EMELK_KV_Q8_0;
  if (!type_ok || g->n_layer <= 0 || g->n_head <= 0 || g->n_head_kv <= 0 ||
      g->n_head % g->n_head_kv != 0 || (g->head_dim != 64 && g->head_dim != 128 && g->head_dim != 256 && g->head_dim != 512) ||
      g->block_tokens <= 0 || g->max_blocks <= 0 || g->max_blocks > EMELK_MAX_BLOCKS) {
    return EMELK_ERR_INVALID_REQUEST;
  }
  const int32_t group = g->n_head / g->n_head_kv;
  if (group != 1 && group != 2 && group != 4 && group != 8) return EMELK_ERR_INVALID_REQUEST;
  const uint64_t vals = static_cast<uint64_t>(g->block_tokens) * static_cast<uint64_t>(g->head_dim);
  if (g->kv_type == EMELK_KV_Q8_0 && (vals % 256u) != 0) return EMELK_ERR_INVALID_REQUEST;
  out.n_layer = g->n_layer;
  out.n_head = g->n_head;
  out.n_head_kv = g->n_head_kv;
  out.head_dim = g->head_dim;
  out.block_tokens = g->block_tokens;
  out.max_blocks = g->max_blocks;
  out.kv_type = g->kv_type;
  out.region_bytes = g->kv_type == EMELK_KV_F16 ? vals * 2u : vals + vals / 16u;
  out.page_bytes = out.region_bytes * static_cast<uint64_t>(g->n_head_kv);
  out.layer_bytes = out.page_bytes * static_cast<uint64_t>(g->max_blocks);
  out.pool_bytes = out.layer_bytes * static_cast<uint64_t>(g->n_layer);
  return EMELK_ERR_NONE;
}

}  // namespace emelk
