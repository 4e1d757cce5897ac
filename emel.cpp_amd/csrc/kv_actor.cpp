// Host KV block-map actor; see kv_actor.hpp for the contract and citations.
#include "kv_actor.hpp"

#include <algorithm>
#include <cstring>
#include <vector>

namespace emelk::kv {

namespace {

constexpr int32_t k_none = static_cast<int32_t>(EMELK_ERR_NONE);
constexpr int32_t k_invalid = static_cast<int32_t>(EMELK_ERR_INVALID_REQUEST);
constexpr int32_t k_backend = static_cast<int32_t>(EMELK_ERR_BACKEND);
constexpr int32_t k_oom = static_cast<int32_t>(EMELK_ERR_OUT_OF_MEMORY);

// memory::detail::bind_or_sink (src/emel/memory/detail.hpp:24-28).
struct out_slot {
  int32_t sink = 0;
  int32_t *ptr;
  explicit out_slot(int32_t *p) : ptr(p != nullptr ? p : &sink) {}
  void set(int32_t v) { *ptr = v; }
};

// view::resolved_or_default (view.hpp:23-26).
constexpr int32_t resolved_or_default(int32_t value, int32_t fallback) {
  return value > 0 ? value : fallback;
}

}  // namespace

actor::actor()
    : st_(std::make_unique<state>()), snapshot_(std::make_unique<emelk_view_snapshot>()) {
  std::memset(snapshot_.get(), 0, sizeof(emelk_view_snapshot));
  snapshot_->block_tokens = k_default_block_tokens;
}

// reset_runtime (kv/actions.hpp:23-39): the stack top holds block 0 so fresh
// allocations pop ascending ids.
void actor::reset_runtime() noexcept {
  state &s = *st_;
  s.active.fill(false);
  s.length.fill(0);
  s.block_count.fill(0);
  for (auto &row : s.blocks) row.fill(0);
  s.refs.fill(0);
  s.free_count = s.max_blocks;
  for (int32_t i = 0; i < s.max_blocks; ++i) {
    s.free_stack[static_cast<size_t>(i)] = static_cast<uint16_t>(s.max_blocks - 1 - i);
  }
}

bool actor::link(int32_t block) noexcept {
  if (block < 0 || block >= k_max_blocks || st_->refs[static_cast<size_t>(block)] == UINT16_MAX) {
    return false;
  }
  ++st_->refs[static_cast<size_t>(block)];
  return true;
}

bool actor::unlink(int32_t block) noexcept {
  if (block < 0 || block >= k_max_blocks || st_->refs[static_cast<size_t>(block)] == 0) {
    return false;
  }
  --st_->refs[static_cast<size_t>(block)];
  return true;
}

int32_t actor::refs(int32_t block) const noexcept {
  if (block < 0 || block >= k_max_blocks) return -1;
  return st_->refs[static_cast<size_t>(block)];
}

// guard_shared_partial_tail_split_needed (kv/guards.hpp:19-30).
int32_t actor::shared_tail_split_needed(int32_t seq, int32_t old_length,
                                        int32_t old_blocks) const noexcept {
  const state &s = *st_;
  const bool partial = old_length > 0 && (old_length % s.block_tokens) != 0 && old_blocks > 0;
  if (!partial) return 0;
  const uint16_t tail = s.blocks[static_cast<size_t>(seq)][static_cast<size_t>(old_blocks - 1)];
  return s.refs[tail] > 1 ? 1 : 0;
}

// ---- reserve (sm.hpp:64-80; guards.hpp:34-47; actions.hpp:155-171) -------
bool actor::process_event(const emelk_event_reserve &ev) {
  out_slot err(ev.error_out);
  err.set(k_none);
  snapshot_dirty_ = true;
  const int32_t max_seq = ev.max_sequences > 0 ? ev.max_sequences : k_max_sequences;
  const int32_t max_blk = ev.max_blocks > 0 ? ev.max_blocks : k_max_blocks;
  const int32_t bt = ev.block_tokens > 0 ? ev.block_tokens : k_default_block_tokens;
  if (!(max_seq > 0 && max_seq <= k_max_sequences && max_blk > 0 && max_blk <= k_max_blocks &&
        bt > 0)) {
    err.set(k_invalid);
    return false;
  }
  st_->max_sequences = resolved_or_default(ev.max_sequences, k_max_sequences);
  st_->max_blocks = resolved_or_default(ev.max_blocks, k_max_blocks);
  st_->block_tokens = resolved_or_default(ev.block_tokens, k_default_block_tokens);
  reset_runtime();
  return true;
}

// ---- allocate_sequence (sm.hpp:83-99; actions.hpp:173-185) ---------------
bool actor::process_event(const emelk_event_allocate_sequence &ev) {
  out_slot err(ev.error_out);
  err.set(k_none);
  snapshot_dirty_ = true;
  if (!valid_seq(ev.seq_id)) {
    err.set(k_invalid);
    return false;
  }
  const size_t i = static_cast<size_t>(ev.seq_id);
  const bool was_active = st_->active[i];
  st_->active[i] = true;
  if (!was_active) {
    st_->length[i] = 0;
    st_->block_count[i] = 0;
  }
  return true;
}

// ---- allocate_slots effect (actions.hpp:246-341) -------------------------
// All-or-nothing: when any needed link/unlink is impossible nothing changes.
bool actor::effect_allocate_slots(int32_t seq_id, int32_t token_count, bool split,
                                  int32_t &block_count_out) noexcept {
  state &s = *st_;
  const size_t seq = static_cast<size_t>(seq_id);
  const int32_t old_length = s.length[seq];
  const int32_t new_length = old_length + token_count;
  const int32_t existing = s.block_count[seq];
  const int32_t old_blocks = blocks_for_tokens(s.block_tokens, old_length);
  const int32_t new_blocks = blocks_for_tokens(s.block_tokens, new_length);
  const int32_t needed = new_blocks - old_blocks;
  const int32_t tail = split ? 1 : 0;
  const int32_t physical = needed + tail;
  const int32_t top = s.free_count;
  block_count_out = 0;

  auto linkable = [&](int32_t b) {
    return b >= 0 && b < k_max_blocks && s.refs[static_cast<size_t>(b)] < UINT16_MAX;
  };
  auto unlinkable = [&](int32_t b) {
    return b >= 0 && b < k_max_blocks && s.refs[static_cast<size_t>(b)] > 0;
  };
  auto stack_at = [&](int32_t idx) -> int32_t {
    return (idx >= 0 && idx < k_max_blocks) ? s.free_stack[static_cast<size_t>(idx)] : -1;
  };

  int32_t tail_index = 0;
  int32_t old_tail = 0;
  int32_t new_tail = 0;
  int32_t can_link = 0;
  int32_t can_unlink = 0;
  if (split) {
    tail_index = old_blocks - 1;
    old_tail = s.blocks[seq][static_cast<size_t>(tail_index)];
    new_tail = stack_at(top - 1);
    can_link += linkable(new_tail) ? 1 : 0;
    can_unlink += unlinkable(old_tail) ? 1 : 0;
  }
  for (int32_t i = 0; i < needed; ++i) can_link += linkable(stack_at(top - 1 - tail - i)) ? 1 : 0;
  if (can_link != physical || can_unlink != tail) return false;

  int32_t linked = 0;
  int32_t unlinked = 0;
  if (split) {
    linked += link(new_tail) ? 1 : 0;
    unlinked += unlink(old_tail) ? 1 : 0;
  }
  for (int32_t i = 0; i < needed; ++i) linked += link(stack_at(top - 1 - tail - i)) ? 1 : 0;
  if (linked != physical || unlinked != tail) return false;

  if (split) s.blocks[seq][static_cast<size_t>(tail_index)] = static_cast<uint16_t>(new_tail);
  for (int32_t i = 0; i < needed; ++i) {
    s.blocks[seq][static_cast<size_t>(existing + i)] =
        static_cast<uint16_t>(stack_at(top - 1 - tail - i));
  }
  s.free_count = top - physical;
  s.block_count[seq] = new_blocks;
  s.length[seq] = new_length;
  block_count_out = physical;
  return true;
}

// ---- allocate_slots (sm.hpp:102-164; guards.hpp:69-191) ------------------
bool actor::process_event(const emelk_event_allocate_slots &ev) {
  out_slot err(ev.error_out);
  out_slot count(ev.block_count_out);
  err.set(k_none);
  count.set(0);
  snapshot_dirty_ = true;
  state &s = *st_;

  // shape: valid id, positive count, active sequence -> invalid_request
  if (!(valid_seq(ev.seq_id) && ev.token_count > 0 && s.block_tokens > 0 &&
        s.active[static_cast<size_t>(ev.seq_id)])) {
    err.set(k_invalid);
    return false;
  }
  const size_t seq = static_cast<size_t>(ev.seq_id);
  // length: new length must stay a positive int32 -> invalid_request
  const int64_t wide = static_cast<int64_t>(s.length[seq]) + ev.token_count;
  if (!(wide > 0 && wide <= INT32_MAX)) {
    err.set(k_invalid);
    return false;
  }
  const int32_t old_length = s.length[seq];
  const int32_t new_length = static_cast<int32_t>(wide);
  const int32_t existing = s.block_count[seq];
  const int32_t old_blocks = blocks_for_tokens(s.block_tokens, old_length);
  const int32_t new_blocks = blocks_for_tokens(s.block_tokens, new_length);
  // block layout: map must cover the current length -> backend_error
  if (!(existing >= old_blocks && new_blocks >= old_blocks)) {
    err.set(k_backend);
    return false;
  }
  // capacity -> out_of_memory
  const int32_t needed = new_blocks - old_blocks;
  const int32_t split = shared_tail_split_needed(ev.seq_id, old_length, old_blocks);
  if (!(existing + needed <= k_max_blocks_per_sequence && s.free_count >= needed + split)) {
    err.set(k_oom);
    return false;
  }
  if (split != 0) {
    if (ev.copy_block == nullptr) {  // tail copy missing -> invalid_request
      err.set(k_invalid);
      return false;
    }
    // effect_copy_shared_tail_block (actions.hpp:218-242): copy the shared
    // partial tail into the block about to be popped, before the map changes.
    const int32_t old_tail = s.blocks[seq][static_cast<size_t>(old_blocks - 1)];
    const int32_t new_tail = s.free_stack[static_cast<size_t>(s.free_count - 1)];
    int32_t copy_error = k_none;
    const bool copy_accepted =
        ev.copy_block(old_tail, new_tail, s.block_tokens, ev.copy_block_user_data, &copy_error);
    if (!(copy_accepted && copy_error == k_none)) {
      err.set(copy_error != k_none ? copy_error : k_backend);
      return false;
    }
  }
  int32_t physical = 0;
  if (!effect_allocate_slots(ev.seq_id, ev.token_count, split != 0, physical)) {
    err.set(k_backend);  // operation_failed_without_error
    return false;
  }
  count.set(physical);
  return true;
}

// ---- branch_sequence (sm.hpp:167-181; guards.hpp:193-206; actions.hpp:357-381)
bool actor::process_event(const emelk_event_branch_sequence &ev) {
  out_slot err(ev.error_out);
  err.set(k_none);
  snapshot_dirty_ = true;
  state &s = *st_;
  if (!valid_seq(ev.parent_seq_id) || !valid_seq(ev.child_seq_id) ||
      ev.parent_seq_id == ev.child_seq_id || !s.active[static_cast<size_t>(ev.parent_seq_id)] ||
      s.active[static_cast<size_t>(ev.child_seq_id)]) {
    err.set(k_invalid);
    return false;
  }
  const size_t parent = static_cast<size_t>(ev.parent_seq_id);
  const size_t child = static_cast<size_t>(ev.child_seq_id);
  const int32_t parent_blocks = s.block_count[parent];
  int32_t linked = 0;
  // As in the reference, links that succeed before a failing one stay linked.
  for (int32_t i = 0; i < parent_blocks; ++i) {
    const uint16_t b = s.blocks[parent][static_cast<size_t>(i)];
    s.blocks[child][static_cast<size_t>(i)] = b;
    linked += link(b) ? 1 : 0;
  }
  const bool all = linked == parent_blocks;
  s.active[child] = all;
  if (all) {
    s.length[child] = s.length[parent];
    s.block_count[child] = parent_blocks;
    return true;
  }
  err.set(k_backend);
  return false;
}

// ---- free_sequence (sm.hpp:184-197; actions.hpp:383-420) -----------------
bool actor::process_event(const emelk_event_free_sequence &ev) {
  out_slot err(ev.error_out);
  err.set(k_none);
  snapshot_dirty_ = true;
  state &s = *st_;
  if (!valid_seq(ev.seq_id)) {
    err.set(k_invalid);
    return false;
  }
  const size_t seq = static_cast<size_t>(ev.seq_id);
  if (!s.active[seq]) return true;  // freeing an inactive sequence is a no-op
  const int32_t n = s.block_count[seq];
  int32_t unlinked = 0;
  for (int32_t i = 0; i < n; ++i) unlinked += unlink(s.blocks[seq][static_cast<size_t>(i)]) ? 1 : 0;
  if (unlinked != n) {
    err.set(k_backend);
    return false;
  }
  // Recycle refcount-0 blocks, last logical block first, so the next pops
  // return them in ascending logical order.
  for (int32_t i = n - 1; i >= 0; --i) {
    const uint16_t b = s.blocks[seq][static_cast<size_t>(i)];
    if (s.refs[b] == 0 && s.free_count < k_max_blocks) {
      s.free_stack[static_cast<size_t>(s.free_count++)] = b;
    }
  }
  s.active[seq] = false;
  s.length[seq] = 0;
  s.block_count[seq] = 0;
  return true;
}

// ---- rollback_slots (sm.hpp:200-214; guards.hpp:229-236; actions.hpp:422-464)
bool actor::process_event(const emelk_event_rollback_slots &ev) {
  out_slot err(ev.error_out);
  out_slot count(ev.block_count_out);
  err.set(k_none);
  count.set(0);
  snapshot_dirty_ = true;
  state &s = *st_;
  if (!(valid_seq(ev.seq_id) && ev.token_count > 0 && s.block_tokens > 0 &&
        s.active[static_cast<size_t>(ev.seq_id)])) {
    err.set(k_invalid);
    return false;
  }
  const size_t seq = static_cast<size_t>(ev.seq_id);
  const int32_t cur = s.length[seq];
  const int32_t new_length = std::max(0, cur - ev.token_count);
  const int32_t existing = s.block_count[seq];
  const int32_t new_blocks = blocks_for_tokens(s.block_tokens, new_length);
  const bool plan_valid = cur >= 0 && new_blocks <= existing;
  const int32_t remove = plan_valid ? existing - new_blocks : 0;
  int32_t unlinked = 0;
  for (int32_t i = 0; i < remove; ++i) {
    unlinked += unlink(s.blocks[seq][static_cast<size_t>(existing - 1 - i)]) ? 1 : 0;
  }
  if (!(plan_valid && unlinked == remove)) {
    err.set(k_backend);
    return false;
  }
  for (int32_t i = 0; i < remove; ++i) {
    const uint16_t b = s.blocks[seq][static_cast<size_t>(existing - 1 - i)];
    if (s.refs[b] == 0 && s.free_count < k_max_blocks) {
      s.free_stack[static_cast<size_t>(s.free_count++)] = b;
    }
  }
  s.block_count[seq] = new_blocks;
  s.length[seq] = new_length;
  count.set(remove);
  return true;
}

// ---- capture_view (sm.hpp:217-231; actions.hpp:41-59, 466-472) -----------
void actor::fill_snapshot(emelk_view_snapshot &out) const noexcept {
  const state &s = *st_;
  std::memset(&out, 0, sizeof(out));
  out.max_sequences = s.max_sequences;
  out.block_tokens = s.block_tokens;
  for (int32_t q = 0; q < s.max_sequences; ++q) {
    const size_t i = static_cast<size_t>(q);
    const bool a = s.active[i];
    out.sequence_active[i] = a ? 1 : 0;
    out.sequence_recurrent_slot[i] = -1;
    out.sequence_length_values[i] = a ? s.length[i] : 0;
    const int32_t n = a ? s.block_count[i] : 0;
    out.sequence_kv_block_count[i] = n;
    if (n > 0) std::memcpy(out.sequence_kv_blocks[i], s.blocks[i].data(), sizeof(uint16_t) * n);
  }
}

bool actor::process_event(const emelk_event_capture_view &ev) {
  out_slot err(ev.error_out);
  err.set(k_none);
  if (ev.snapshot_out == nullptr) {
    err.set(k_invalid);
    return false;
  }
  fill_snapshot(*ev.snapshot_out);
  if (ev.snapshot_out == snapshot_.get()) snapshot_dirty_ = false;
  return true;
}

// kv::sm::view (sm.hpp:480-499).
const emelk_view_snapshot &actor::view() noexcept {
  if (snapshot_dirty_) {
    fill_snapshot(*snapshot_);
    snapshot_dirty_ = false;
  }
  return *snapshot_;
}

// ---- evict_blocks (new) --------------------------------------------------
// Drops whole logical blocks from one sequence: the survivors close ranks in
// logical order, the length shrinks by the tokens the dropped blocks held,
// each dropped block is unlinked and recycled when its refcount reaches 0
// (recycle order as free_sequence: last listed first).  All-or-nothing.
bool actor::process_event(const emelk_event_evict_blocks &ev) {
  out_slot err(ev.error_out);
  out_slot removed(ev.tokens_removed_out);
  err.set(k_none);
  removed.set(0);
  snapshot_dirty_ = true;
  state &s = *st_;
  if (!(valid_seq(ev.seq_id) && s.active[static_cast<size_t>(ev.seq_id)] &&
        ev.block_count > 0 && ev.logical_blocks != nullptr)) {
    err.set(k_invalid);
    return false;
  }
  const size_t seq = static_cast<size_t>(ev.seq_id);
  const int32_t n = s.block_count[seq];
  std::vector<uint8_t> drop(static_cast<size_t>(std::max(n, 0)), 0);
  for (int32_t i = 0; i < ev.block_count; ++i) {
    const int32_t lb = ev.logical_blocks[i];
    if (lb < 0 || lb >= n || drop[static_cast<size_t>(lb)]) {
      err.set(k_invalid);
      return false;
    }
    drop[static_cast<size_t>(lb)] = 1;
  }
  for (int32_t i = 0; i < ev.block_count; ++i) {
    if (s.refs[s.blocks[seq][static_cast<size_t>(ev.logical_blocks[i])]] == 0) {
      err.set(k_backend);
      return false;
    }
  }
  const int32_t len = s.length[seq];
  int32_t tokens = 0;
  for (int32_t i = 0; i < ev.block_count; ++i) {
    const int32_t lb = ev.logical_blocks[i];
    tokens += std::max(0, std::min(s.block_tokens, len - lb * s.block_tokens));
    unlink(s.blocks[seq][static_cast<size_t>(lb)]);
  }
  for (int32_t i = ev.block_count - 1; i >= 0; --i) {
    const uint16_t b = s.blocks[seq][static_cast<size_t>(ev.logical_blocks[i])];
    if (s.refs[b] == 0 && s.free_count < k_max_blocks) {
      s.free_stack[static_cast<size_t>(s.free_count++)] = b;
    }
  }
  int32_t w = 0;
  for (int32_t i = 0; i < n; ++i) {
    if (!drop[static_cast<size_t>(i)]) s.blocks[seq][static_cast<size_t>(w++)] = s.blocks[seq][static_cast<size_t>(i)];
  }
  s.block_count[seq] = w;
  s.length[seq] = len - tokens;
  removed.set(tokens);
  return true;
}

// ---- compact (new) -------------------------------------------------------
// Renumbers live blocks (refcount > 0) onto [0, n_live): every live block at
// or above n_live moves, in ascending order, into the lowest free id below
// n_live.  Sources and destinations are therefore disjoint and the device
// copies may all run at once.  Block maps and refcounts are renumbered and
// the free stack is rebuilt so later pops return n_live, n_live+1, ...
bool actor::process_event(const emelk_event_compact &ev) {
  out_slot err(ev.error_out);
  out_slot count(ev.move_count_out);
  err.set(k_none);
  count.set(0);
  snapshot_dirty_ = true;
  state &s = *st_;
  int32_t n_live = 0;
  for (int32_t b = 0; b < s.max_blocks; ++b) n_live += s.refs[static_cast<size_t>(b)] > 0 ? 1 : 0;
  std::vector<int32_t> holes;
  std::vector<int32_t> movers;
  for (int32_t b = 0; b < n_live; ++b) {
    if (s.refs[static_cast<size_t>(b)] == 0) holes.push_back(b);
  }
  for (int32_t b = n_live; b < s.max_blocks; ++b) {
    if (s.refs[static_cast<size_t>(b)] > 0) movers.push_back(b);
  }
  const int32_t moves = static_cast<int32_t>(movers.size());
  if (moves != static_cast<int32_t>(holes.size())) {
    err.set(k_backend);
    return false;
  }
  if (moves > 0 && (ev.moves_out == nullptr || ev.max_moves < moves)) {
    err.set(k_invalid);
    return false;
  }
  std::vector<uint16_t> remap(static_cast<size_t>(s.max_blocks));
  for (int32_t b = 0; b < s.max_blocks; ++b) remap[static_cast<size_t>(b)] = static_cast<uint16_t>(b);
  for (int32_t i = 0; i < moves; ++i) {
    remap[static_cast<size_t>(movers[i])] = static_cast<uint16_t>(holes[i]);
    ev.moves_out[2 * i] = movers[i];
    ev.moves_out[2 * i + 1] = holes[i];
    s.refs[static_cast<size_t>(holes[i])] = s.refs[static_cast<size_t>(movers[i])];
    s.refs[static_cast<size_t>(movers[i])] = 0;
  }
  for (int32_t q = 0; q < s.max_sequences; ++q) {
    const size_t i = static_cast<size_t>(q);
    if (!s.active[i]) continue;
    for (int32_t k = 0; k < s.block_count[i]; ++k) {
      uint16_t &b = s.blocks[i][static_cast<size_t>(k)];
      if (b < s.max_blocks) b = remap[b];
    }
  }
  s.free_count = s.max_blocks - n_live;
  for (int32_t i = 0; i < s.free_count; ++i) {
    s.free_stack[static_cast<size_t>(i)] = static_cast<uint16_t>(s.max_blocks - 1 - i);
  }
  count.set(moves);
  return true;
}

emel_error_type actor::export_block_tables(const int32_t *seq_ids, int32_t n_seq, uint16_t *out,
                                           int32_t stride) const noexcept {
  const state &s = *st_;
  if (seq_ids == nullptr || out == nullptr || n_seq < 0 || stride <= 0) {
    return EMELK_ERR_INVALID_REQUEST;
  }
  for (int32_t r = 0; r < n_seq; ++r) {
    const int32_t q = seq_ids[r];
    if (!valid_seq(q) || !s.active[static_cast<size_t>(q)]) return EMELK_ERR_INVALID_REQUEST;
    if (s.block_count[static_cast<size_t>(q)] > stride) return EMELK_ERR_INVALID_REQUEST;
  }
  for (int32_t r = 0; r < n_seq; ++r) {
    const size_t q = static_cast<size_t>(seq_ids[r]);
    uint16_t *row = out + static_cast<size_t>(r) * static_cast<size_t>(stride);
    const int32_t n = s.block_count[q];
    std::memcpy(row, s.blocks[q].data(), sizeof(uint16_t) * static_cast<size_t>(n));
    std::fill(row + n, row + stride, static_cast<uint16_t>(EMELK_INVALID_KV_BLOCK));
  }
  return EMELK_ERR_NONE;
}

emel_error_type actor::set_free_order(const uint16_t *order, int32_t count) noexcept {
  state &s = *st_;
  if (order == nullptr || count != s.free_count) return EMELK_ERR_INVALID_REQUEST;
  std::vector<uint8_t> seen(static_cast<size_t>(k_max_blocks), 0);
  for (int32_t i = 0; i < count; ++i) seen[s.free_stack[static_cast<size_t>(i)]] = 1;
  std::vector<uint8_t> used(static_cast<size_t>(k_max_blocks), 0);
  for (int32_t i = 0; i < count; ++i) {
    const uint16_t b = order[i];
    if (b >= k_max_blocks || !seen[b] || used[b]) return EMELK_ERR_INVALID_REQUEST;
    used[b] = 1;
  }
  for (int32_t i = 0; i < count; ++i) s.free_stack[static_cast<size_t>(count - 1 - i)] = order[i];
  return EMELK_ERR_NONE;
}

}  // namespace emelk::kv
