// extern "C" surface of the host KV actor (include/emelk.h).
#include <new>

#include "emelk.h"
#include "kv_actor.hpp"

struct emelk_kv_actor {
  emelk::kv::actor impl;
};

namespace {

template <class event_type>
bool dispatch(void *actor, const event_type *ev) {
  if (actor == nullptr || ev == nullptr) return false;
  return static_cast<emelk_kv_actor *>(actor)->impl.process_event(*ev);
}

template <class event_type>
bool guarded(emelk_kv_actor *actor, const event_type *ev) {
  if (actor == nullptr || ev == nullptr) return false;
  return actor->impl.process_event(*ev);
}

}  // namespace

extern "C" {

emelk_kv_actor *emelk_kv_actor_create(void) { return new (std::nothrow) emelk_kv_actor(); }

void emelk_kv_actor_destroy(emelk_kv_actor *actor) { delete actor; }

bool emelk_kv_reserve(emelk_kv_actor *a, const emelk_event_reserve *ev) { return guarded(a, ev); }
bool emelk_kv_allocate_sequence(emelk_kv_actor *a, const emelk_event_allocate_sequence *ev) {
  return guarded(a, ev);
}
bool emelk_kv_allocate_slots(emelk_kv_actor *a, const emelk_event_allocate_slots *ev) {
  return guarded(a, ev);
}
bool emelk_kv_branch_sequence(emelk_kv_actor *a, const emelk_event_branch_sequence *ev) {
  return guarded(a, ev);
}
bool emelk_kv_free_sequence(emelk_kv_actor *a, const emelk_event_free_sequence *ev) {
  return guarded(a, ev);
}
bool emelk_kv_rollback_slots(emelk_kv_actor *a, const emelk_event_rollback_slots *ev) {
  return guarded(a, ev);
}
bool emelk_kv_capture_view(emelk_kv_actor *a, const emelk_event_capture_view *ev) {
  return guarded(a, ev);
}
bool emelk_kv_evict_blocks(emelk_kv_actor *a, const emelk_event_evict_blocks *ev) {
  return guarded(a, ev);
}
bool emelk_kv_compact(emelk_kv_actor *a, const emelk_event_compact *ev) { return guarded(a, ev); }

const emelk_view_snapshot *emelk_kv_view(emelk_kv_actor *a) {
  return a == nullptr ? nullptr : &a->impl.view();
}

// snapshot::lookup_kv_block (src/emel/memory/view.hpp:87-109).
int32_t emelk_kv_lookup_kv_block(emelk_kv_actor *a, int32_t seq_id, int32_t pos) {
  if (a == nullptr) return -1;
  const emelk_view_snapshot &s = a->impl.view();
  if (seq_id < 0 || seq_id >= s.max_sequences || seq_id >= EMELK_MAX_SEQUENCES ||
      s.sequence_active[seq_id] == 0 || pos < 0 || s.block_tokens <= 0) {
    return -1;
  }
  if (pos >= s.sequence_length_values[seq_id]) return -1;
  const int32_t count = s.sequence_kv_block_count[seq_id];
  if (count <= 0 || count > EMELK_MAX_BLOCKS_PER_SEQUENCE) return -1;
  const int32_t lb = pos / s.block_tokens;
  if (lb >= count) return -1;
  const uint16_t b = s.sequence_kv_blocks[seq_id][lb];
  return b == EMELK_INVALID_KV_BLOCK ? -1 : static_cast<int32_t>(b);
}

void emelk_kv_bind(emelk_kv_actor *a, emelk_kv_binding *out) {
  if (out == nullptr) return;
  out->actor = a;
  out->dispatch_reserve = &dispatch<emelk_event_reserve>;
  out->dispatch_allocate_sequence = &dispatch<emelk_event_allocate_sequence>;
  out->dispatch_allocate_slots = &dispatch<emelk_event_allocate_slots>;
  out->dispatch_branch_sequence = &dispatch<emelk_event_branch_sequence>;
  out->dispatch_free_sequence = &dispatch<emelk_event_free_sequence>;
  out->dispatch_rollback_slots = &dispatch<emelk_event_rollback_slots>;
  out->dispatch_capture_view = &dispatch<emelk_event_capture_view>;
}

emel_error_type emelk_kv_export_block_tables(emelk_kv_actor *a, const int32_t *seq_ids,
                                             int32_t n_seq, uint16_t *table_out,
                                             int32_t table_stride) {
  if (a == nullptr) return EMELK_ERR_INVALID_REQUEST;
  return a->impl.export_block_tables(seq_ids, n_seq, table_out, table_stride);
}

emel_error_type emelk_kv_set_free_order(emelk_kv_actor *a, const uint16_t *order, int32_t count) {
  if (a == nullptr) return EMELK_ERR_INVALID_REQUEST;
  return a->impl.set_free_order(order, count);
}

int32_t emelk_kv_block_refs(emelk_kv_actor *a, int32_t block_id) {
  return a == nullptr ? -1 : a->impl.refs(block_id);
}

int32_t emelk_kv_sequence_length(emelk_kv_actor *a, int32_t seq_id) {
  if (a == nullptr) return -1;
  const auto &st = a->impl.raw();
  if (seq_id < 0 || seq_id >= st.max_sequences || !st.active[static_cast<size_t>(seq_id)]) return -1;
  return st.length[static_cast<size_t>(seq_id)];
}

int32_t emelk_kv_free_count(emelk_kv_actor *a) { return a == nullptr ? -1 : a->impl.free_count(); }

const char *emelk_build_info(void) { return "emelk gfx950 kv-cache hot path"; }

}  // extern "C"
