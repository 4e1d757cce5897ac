/* A plain C11 client of include/emelk.h linked against libemelk.so: the
 * header compiles as C, and the host entry points work from C the way the
 * reference's hybrid memory facade drives a kv_binding (every event through
 * the dispatch table, src/emel/memory/hybrid/actions.hpp:199-213) and the
 * way its generator plans a prompt (text/generator/actions.hpp:209-242).
 * No device calls: it runs on a machine without a GPU.  Built and run by
 * tests/test_abi.py. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "emelk.h"

#define CHECK(c)                                                    \
  do {                                                              \
    if (!(c)) {                                                     \
      printf("CHECK failed at line %d: %s\n", __LINE__, #c);        \
      return 1;                                                     \
    }                                                               \
  } while (0)

int main(void) {
  emelk_kv_actor *actor = emelk_kv_actor_create();
  CHECK(actor != NULL);
  emelk_kv_binding b;
  memset(&b, 0, sizeof(b));
  emelk_kv_bind(actor, &b);
  CHECK(b.actor == actor && b.dispatch_reserve && b.dispatch_capture_view);

  /* reserve 4 sequences over 8 pages of 16 tokens, through the table */
  int32_t err = -1;
  emelk_event_reserve rs = {4, 8, 16, &err};
  CHECK(b.dispatch_reserve(b.actor, &rs) && err == 0);
  emelk_event_allocate_sequence as = {1, &err};
  CHECK(b.dispatch_allocate_sequence(b.actor, &as) && err == 0);
  int32_t blocks = -1;
  emelk_event_allocate_slots sl = {1, 20, &blocks, &err, NULL, NULL};
  CHECK(b.dispatch_allocate_slots(b.actor, &sl) && err == 0 && blocks == 2);
  /* fresh pops are ascending: pages 0 and 1 */
  CHECK(emelk_kv_lookup_kv_block(actor, 1, 0) == 0);
  CHECK(emelk_kv_lookup_kv_block(actor, 1, 19) == 1);
  /* a refused event leaves the state as it was and sets the error bits */
  emelk_event_allocate_slots big = {1, 1000, &blocks, &err, NULL, NULL};
  CHECK(!b.dispatch_allocate_slots(b.actor, &big) && err != 0 && blocks == 0);
  CHECK(emelk_kv_sequence_length(actor, 1) == 20);

  static emelk_view_snapshot snap;
  emelk_event_capture_view cv = {&snap, &err};
  CHECK(b.dispatch_capture_view(b.actor, &cv) && err == 0);
  CHECK(snap.sequence_active[1] == 1 && snap.sequence_length_values[1] == 20);
  CHECK(snap.sequence_kv_block_count[1] == 2 && snap.sequence_kv_blocks[1][1] == 1);

  int32_t ids[1] = {1};
  uint16_t table[4];
  CHECK(emelk_kv_export_block_tables(actor, ids, 1, table, 4) == EMELK_ERR_NONE);
  CHECK(table[0] == 0 && table[1] == 1 && table[2] == EMELK_INVALID_KV_BLOCK);

  emelk_event_free_sequence fs = {1, &err};
  CHECK(b.dispatch_free_sequence(b.actor, &fs) && err == 0);
  CHECK(emelk_kv_free_count(actor) == 8);
  emelk_kv_actor_destroy(actor);

  /* the generator's prompt plan: simple mode, step 4 over 10 tokens */
  int32_t tokens[10] = {5, 6, 7, 8, 9, 10, 11, 12, 13, 14};
  emelk_plan_request rq;
  memset(&rq, 0, sizeof(rq));
  rq.token_ids = tokens;
  rq.n_tokens = 10;
  rq.n_steps = 4;
  rq.mode = EMELK_PLAN_SIMPLE;
  rq.equal_sequential = 1;
  rq.seq_mask_words = 1;
  emelk_plan_result *plan = (emelk_plan_result *)malloc(sizeof(emelk_plan_result));
  CHECK(plan != NULL);
  uint32_t perr = 99;
  CHECK(emelk_batch_plan(&rq, plan, &perr) && perr == 0);
  CHECK(plan->step_count == 3 && plan->step_sizes[0] == 4 && plan->step_sizes[2] == 2);
  CHECK(plan->step_token_offsets[3] == 10 && plan->total_outputs == 1);

  /* equal mode over two interleaved sequences: decoder-shaped steps */
  int32_t seq[10] = {0, 1, 0, 1, 0, 1, 0, 1, 1, 1};
  rq.mode = EMELK_PLAN_EQUAL;
  rq.seq_primary_ids = seq;
  rq.seq_primary_ids_count = 10;
  rq.equal_sequential = 0;
  CHECK(emelk_batch_plan(&rq, plan, &perr) && perr == 0);
  CHECK(plan->step_count == 3);
  int32_t sids[EMELK_MAX_SEQUENCES], n_seq = 0, per = 0;
  CHECK(emelk_plan_step_sequences(&rq, plan, 0, sids, &n_seq, &per) == EMELK_ERR_NONE);
  CHECK(n_seq == 2 && per == 2 && sids[0] == 0 && sids[1] == 1);
  CHECK(plan->step_token_indices[0] == 0 && plan->step_token_indices[1] == 2);
  CHECK(plan->step_token_indices[2] == 1 && plan->step_token_indices[3] == 3);
  CHECK(emelk_plan_step_sequences(&rq, plan, 2, sids, &n_seq, &per) == EMELK_ERR_NONE);
  CHECK(n_seq == 1 && sids[0] == 1 && per == 2);

  /* a bad request: the reference's bits */
  rq.mode = 99;
  CHECK(!emelk_batch_plan(&rq, plan, &perr));
  CHECK(perr == (EMELK_PLAN_ERR_INVALID_MODE | EMELK_PLAN_ERR_INVALID_REQUEST));
  free(plan);
  printf("ok\n");
  return 0;
}
