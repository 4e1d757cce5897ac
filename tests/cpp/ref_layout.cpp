// Pins the drop-in boundary against the reference's own headers.
//
// Compiled by tests/test_ref_layout.py only where the reference checkout is
// present: it includes src/emel/memory/events.hpp and view.hpp from there,
// and REF_KV_BINDING_HEADER, a header the test cuts out of
// src/emel/memory/hybrid/context.hpp (the dispatch typedefs and struct
// kv_binding, context.hpp:11-30; the rest of that file needs the SML
// library).  Every event struct, the snapshot and the binding must match
// include/emelk.h in size, alignment and member offsets; then a binding
// filled by emelk_kv_bind is copied into the reference's kv_binding and the
// actor is driven through the reference's own event types.
#include <cstddef>
#include <cstdio>
#include <cstring>
#include <type_traits>

#include "emel/memory/events.hpp"
#include "emel/memory/view.hpp"
#include "emelk.h"

namespace emel::memory::hybrid {
#include REF_KV_BINDING_HEADER
}

namespace ev = emel::memory::event;
namespace hy = emel::memory::hybrid;
namespace vw = emel::memory::view;

#define SAME_SIZE(R, E)                                                        \
  static_assert(sizeof(R) == sizeof(E), #R " size");                          \
  static_assert(alignof(R) == alignof(E), #R " alignment");                   \
  static_assert(std::is_standard_layout_v<R> && std::is_standard_layout_v<E>, \
                #R " standard layout")
#define SAME_AT(R, E, rf, ef) \
  static_assert(offsetof(R, rf) == offsetof(E, ef), #R "::" #rf " offset")
#define SAME_FIELD(R, E, f)                                                      \
  SAME_AT(R, E, f, f);                                                           \
  static_assert(sizeof(std::declval<R &>().f) == sizeof(std::declval<E &>().f), \
                #R "::" #f " size")

SAME_SIZE(ev::reserve, emelk_event_reserve);
SAME_FIELD(ev::reserve, emelk_event_reserve, max_sequences);
SAME_FIELD(ev::reserve, emelk_event_reserve, max_blocks);
SAME_FIELD(ev::reserve, emelk_event_reserve, block_tokens);
SAME_FIELD(ev::reserve, emelk_event_reserve, error_out);

SAME_SIZE(ev::allocate_sequence, emelk_event_allocate_sequence);
SAME_FIELD(ev::allocate_sequence, emelk_event_allocate_sequence, seq_id);
SAME_FIELD(ev::allocate_sequence, emelk_event_allocate_sequence, error_out);

SAME_SIZE(ev::allocate_slots, emelk_event_allocate_slots);
SAME_FIELD(ev::allocate_slots, emelk_event_allocate_slots, seq_id);
SAME_FIELD(ev::allocate_slots, emelk_event_allocate_slots, token_count);
SAME_FIELD(ev::allocate_slots, emelk_event_allocate_slots, block_count_out);
SAME_FIELD(ev::allocate_slots, emelk_event_allocate_slots, error_out);
SAME_FIELD(ev::allocate_slots, emelk_event_allocate_slots, copy_block);
SAME_FIELD(ev::allocate_slots, emelk_event_allocate_slots, copy_block_user_data);
static_assert(std::is_same_v<ev::allocate_slots::copy_block_fn, emelk_copy_block_fn>,
              "copy_block_fn signature");

SAME_SIZE(ev::branch_sequence, emelk_event_branch_sequence);
SAME_FIELD(ev::branch_sequence, emelk_event_branch_sequence, parent_seq_id);
SAME_FIELD(ev::branch_sequence, emelk_event_branch_sequence, child_seq_id);
SAME_FIELD(ev::branch_sequence, emelk_event_branch_sequence, copy_state);
SAME_FIELD(ev::branch_sequence, emelk_event_branch_sequence, copy_state_user_data);
SAME_FIELD(ev::branch_sequence, emelk_event_branch_sequence, error_out);
static_assert(std::is_same_v<ev::branch_sequence::copy_state_fn, emelk_copy_state_fn>,
              "copy_state_fn signature");

SAME_SIZE(ev::free_sequence, emelk_event_free_sequence);
SAME_FIELD(ev::free_sequence, emelk_event_free_sequence, seq_id);
SAME_FIELD(ev::free_sequence, emelk_event_free_sequence, error_out);

SAME_SIZE(ev::rollback_slots, emelk_event_rollback_slots);
SAME_FIELD(ev::rollback_slots, emelk_event_rollback_slots, seq_id);
SAME_FIELD(ev::rollback_slots, emelk_event_rollback_slots, token_count);
SAME_FIELD(ev::rollback_slots, emelk_event_rollback_slots, block_count_out);
SAME_FIELD(ev::rollback_slots, emelk_event_rollback_slots, error_out);

SAME_SIZE(ev::capture_view, emelk_event_capture_view);
SAME_FIELD(ev::capture_view, emelk_event_capture_view, snapshot_out);
SAME_FIELD(ev::capture_view, emelk_event_capture_view, error_out);

SAME_SIZE(vw::snapshot, emelk_view_snapshot);
SAME_FIELD(vw::snapshot, emelk_view_snapshot, max_sequences);
SAME_FIELD(vw::snapshot, emelk_view_snapshot, block_tokens);
SAME_FIELD(vw::snapshot, emelk_view_snapshot, sequence_active);
SAME_FIELD(vw::snapshot, emelk_view_snapshot, sequence_length_values);
SAME_FIELD(vw::snapshot, emelk_view_snapshot, sequence_kv_block_count);
SAME_FIELD(vw::snapshot, emelk_view_snapshot, sequence_kv_blocks);
SAME_FIELD(vw::snapshot, emelk_view_snapshot, sequence_recurrent_slot);
static_assert(vw::MAX_SEQUENCES == EMELK_MAX_SEQUENCES, "MAX_SEQUENCES");
static_assert(vw::MAX_BLOCKS_PER_SEQUENCE == EMELK_MAX_BLOCKS_PER_SEQUENCE,
              "MAX_BLOCKS_PER_SEQUENCE");
static_assert(vw::MAX_BLOCKS == EMELK_MAX_BLOCKS, "MAX_BLOCKS");
static_assert(vw::INVALID_KV_BLOCK == EMELK_INVALID_KV_BLOCK, "INVALID_KV_BLOCK");

SAME_SIZE(hy::kv_binding, emelk_kv_binding);
SAME_FIELD(hy::kv_binding, emelk_kv_binding, actor);
SAME_FIELD(hy::kv_binding, emelk_kv_binding, dispatch_reserve);
SAME_FIELD(hy::kv_binding, emelk_kv_binding, dispatch_allocate_sequence);
SAME_FIELD(hy::kv_binding, emelk_kv_binding, dispatch_allocate_slots);
SAME_FIELD(hy::kv_binding, emelk_kv_binding, dispatch_branch_sequence);
SAME_FIELD(hy::kv_binding, emelk_kv_binding, dispatch_free_sequence);
SAME_FIELD(hy::kv_binding, emelk_kv_binding, dispatch_rollback_slots);
SAME_FIELD(hy::kv_binding, emelk_kv_binding, dispatch_capture_view);

static int failures = 0;
#define CHECK(c)                                                   \
  do {                                                             \
    if (!(c)) {                                                    \
      std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #c);    \
      ++failures;                                                  \
    }                                                              \
  } while (0)

static int copies = 0;
static bool count_copy(int32_t, int32_t, int32_t, void *, int32_t *err) {
  ++copies;
  if (err != nullptr) *err = 0;
  return true;
}

int main() {
  emelk_kv_actor *actor = emelk_kv_actor_create();
  emelk_kv_binding mine{};
  emelk_kv_bind(actor, &mine);
  hy::kv_binding ref{};
  std::memcpy(static_cast<void *>(&ref), &mine, sizeof ref);
  CHECK(ref.actor == actor);

  // From here on only the reference's types are used.
  int32_t err = -1;
  CHECK(ref.dispatch_reserve(ref.actor, ev::reserve{4, 8, 16, &err}) && err == 0);
  CHECK(ref.dispatch_allocate_sequence(ref.actor, ev::allocate_sequence{0, &err}) && err == 0);
  int32_t blocks = -1;
  CHECK(ref.dispatch_allocate_slots(ref.actor,
                                    ev::allocate_slots{0, 20, &blocks, &err, nullptr, nullptr}) &&
        err == 0 && blocks == 2);
  CHECK(ref.dispatch_branch_sequence(ref.actor,
                                     ev::branch_sequence{0, 1, nullptr, nullptr, &err}) &&
        err == 0);
  // the child appends into the shared, partly filled tail page: it must be
  // split through the caller's copy_block callback
  CHECK(ref.dispatch_allocate_slots(
            ref.actor, ev::allocate_slots{1, 1, &blocks, &err, count_copy, nullptr}) &&
        err == 0 && copies == 1);
  static vw::snapshot snap;
  CHECK(ref.dispatch_capture_view(ref.actor, ev::capture_view{&snap, &err}) && err == 0);
  CHECK(snap.is_sequence_active(0) && snap.is_sequence_active(1));
  CHECK(snap.sequence_length(0) == 20 && snap.sequence_length(1) == 21);
  CHECK(snap.lookup_kv_block(0, 0) == snap.lookup_kv_block(1, 0));   // shared head page
  CHECK(snap.lookup_kv_block(0, 16) != snap.lookup_kv_block(1, 16));  // split tail page
  CHECK(snap.lookup_kv_block(0, 0) == emelk_kv_lookup_kv_block(actor, 0, 0));
  CHECK(ref.dispatch_rollback_slots(ref.actor, ev::rollback_slots{1, 5, &blocks, &err}) &&
        err == 0 && blocks == 1);
  CHECK(ref.dispatch_free_sequence(ref.actor, ev::free_sequence{0, &err}) && err == 0);
  // rejected events keep the reference's bool + error convention
  CHECK(!ref.dispatch_allocate_sequence(ref.actor, ev::allocate_sequence{-1, &err}) &&
        err == EMELK_ERR_INVALID_REQUEST);
  CHECK(ref.dispatch_capture_view(ref.actor, ev::capture_view{&snap, &err}) && err == 0);
  CHECK(!snap.is_sequence_active(0) && snap.sequence_length(1) == 16);
  emelk_kv_actor_destroy(actor);
  if (failures == 0) std::printf("ref layout ok\n");
  return failures == 0 ? 0 : 1;
}
