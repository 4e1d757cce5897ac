// Host KV block-map actor: the logical->physical page map, per-page refcounts
// and the LIFO free stack of stateforward/emel.cpp's memory::kv::sm, with the
// same event API and the same observable results (block ids, error bits,
// out-params, state left unchanged on failure).  It never touches K/V bytes:
// physical storage belongs to the device page pool (kv_cache.hip), reached
// through the copy_block callback exactly as the reference reaches
// copy_attention_kv_block.
//
// Reference (paths relative to the reference checkout):
//   context            src/emel/memory/kv/context.hpp:10-24
//   actions            src/emel/memory/kv/actions.hpp:23-544
//   guards             src/emel/memory/kv/guards.hpp:19-280
//   transition table   src/emel/memory/kv/sm.hpp:57-362
//   typed wrappers     src/emel/memory/kv/sm.hpp:364-507
//
// The reference drives these through a Stateforward.SML transition table.
// Here each event is one run-to-completion member function whose guard order
// and error mapping follow the table row by row; the table itself is not
// reproduced because nothing observable depends on it.
#pragma once

#include <array>
#include <cstdint>
#include <memory>

#include "emelk.h"

namespace emelk::kv {

inline constexpr int32_t k_max_sequences = EMELK_MAX_SEQUENCES;
inline constexpr int32_t k_max_blocks = EMELK_MAX_BLOCKS;
inline constexpr int32_t k_max_blocks_per_sequence = EMELK_MAX_BLOCKS_PER_SEQUENCE;
inline constexpr int32_t k_default_block_tokens = EMELK_DEFAULT_BLOCK_TOKENS;

// view::blocks_for_tokens (src/emel/memory/view.hpp:30-42): 0 for
// non-positive inputs.
constexpr int32_t blocks_for_tokens(int32_t block_tokens, int32_t token_count) noexcept {
  if (block_tokens <= 0 || token_count <= 0) return 0;
  return static_cast<int32_t>((static_cast<int64_t>(token_count) + block_tokens - 1) /
                              block_tokens);
}

// view::positions_capacity_for (view.hpp:47-57): -1 on int32 overflow.
constexpr int32_t positions_capacity_for(int32_t block_tokens, int32_t token_count) noexcept {
  if (block_tokens <= 0) return 0;
  const int64_t cap =
      static_cast<int64_t>(blocks_for_tokens(block_tokens, token_count)) * block_tokens;
  return cap > INT32_MAX ? -1 : static_cast<int32_t>(cap);
}

struct state {
  int32_t max_sequences = k_max_sequences;
  int32_t max_blocks = k_max_blocks;
  int32_t block_tokens = k_default_block_tokens;
  std::array<uint16_t, k_max_blocks> refs = {};
  std::array<bool, k_max_sequences> active = {};
  std::array<int32_t, k_max_sequences> length = {};
  std::array<int32_t, k_max_sequences> block_count = {};
  std::array<std::array<uint16_t, k_max_blocks_per_sequence>, k_max_sequences> blocks = {};
  std::array<uint16_t, k_max_blocks> free_stack = {};
  int32_t free_count = 0;
};

class actor {
 public:
  actor();

  bool process_event(const emelk_event_reserve &ev);
  bool process_event(const emelk_event_allocate_sequence &ev);
  bool process_event(const emelk_event_allocate_slots &ev);
  bool process_event(const emelk_event_branch_sequence &ev);
  bool process_event(const emelk_event_free_sequence &ev);
  bool process_event(const emelk_event_rollback_slots &ev);
  bool process_event(const emelk_event_capture_view &ev);
  bool process_event(const emelk_event_evict_blocks &ev);
  bool process_event(const emelk_event_compact &ev);

  const emelk_view_snapshot &view() noexcept;

  emel_error_type export_block_tables(const int32_t *seq_ids, int32_t n_seq, uint16_t *out,
                                      int32_t stride) const noexcept;
  emel_error_type set_free_order(const uint16_t *order, int32_t count) noexcept;
  int32_t refs(int32_t block) const noexcept;
  int32_t free_count() const noexcept { return st_->free_count; }

  // Direct access for white-box tests of the effect functions (the
  // reference tests do the same with action::context).
  state &raw() noexcept { return *st_; }

  // effect_allocate_slots_impl<split> (kv/actions.hpp:246-341); returns
  // accepted and writes the physical block count.
  bool effect_allocate_slots(int32_t seq_id, int32_t token_count, bool split_shared_tail,
                             int32_t &block_count_out) noexcept;

 private:
  void reset_runtime() noexcept;
  void fill_snapshot(emelk_view_snapshot &out) const noexcept;
  bool valid_seq(int32_t seq_id) const noexcept {
    return seq_id >= 0 && seq_id < st_->max_sequences;
  }
  bool link(int32_t block) noexcept;
  bool unlink(int32_t block) noexcept;
  int32_t shared_tail_split_needed(int32_t seq, int32_t old_length,
                                   int32_t old_blocks) const noexcept;

  std::unique_ptr<state> st_;
  std::unique_ptr<emelk_view_snapshot> snapshot_;
  bool snapshot_dirty_ = true;
};

}  // namespace emelk::kv
