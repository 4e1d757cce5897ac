// White-box check of the allocate_slots effect with a shared-tail split whose
// refcounts cannot be updated, ported from the reference test
// tests/memory/kv/lifecycle_tests.cpp:358-399
// (memory_kv_allocate_slots_failed_tail_split_keeps_map_and_free_stack).
// Built and run by tests/test_kv_actor.py with the host compiler.
#include <cstdio>

#include "kv_actor.hpp"

#define CHECK(c)                                               \
  do {                                                         \
    if (!(c)) {                                                \
      std::printf("CHECK failed line %d: %s\n", __LINE__, #c); \
      return 1;                                                \
    }                                                          \
  } while (0)

int main() {
  emelk::kv::actor a;
  emelk_event_reserve r{2, 2, 4, nullptr};
  CHECK(a.process_event(r));
  auto &s = a.raw();
  s.active[0] = true;
  s.length[0] = 2;
  s.block_count[0] = 1;
  s.blocks[0][0] = 0;
  s.free_count = 1;
  s.free_stack[0] = 1;
  s.refs[0] = 0;
  s.refs[1] = 0;
  int32_t count = -1;
  const bool accepted = a.effect_allocate_slots(0, 1, true, count);
  CHECK(!accepted);
  CHECK(count == 0);
  CHECK(s.blocks[0][0] == 0);
  CHECK(s.free_count == 1);
  CHECK(s.length[0] == 2);
  CHECK(s.block_count[0] == 1);
  CHECK(s.refs[1] == 0);
  CHECK(s.refs[0] == 0);
  std::printf("ok\n");
  return 0;
}
