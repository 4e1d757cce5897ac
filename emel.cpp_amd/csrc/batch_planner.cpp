// Host batch planner over the C ABI (include/emelk.h, "Batch planner").
//
// Restates emel::batch::planner (src/emel/batch/planner/): the outer
// machine validates the request and normalises the step size
// (sm.hpp:20-60, detail.hpp:129-233, actions.hpp:64-75), then one of three
// mode machines builds the plan (modes/simple/actions.hpp:32-54,
// modes/sequential/actions.hpp:30-93, modes/equal/actions.hpp:34-269), and
// a plan counts as complete only when every token was placed
// (guards.hpp:9-23).  Error bits accumulate as the reference's transitions
// add them: a failure inside a mode's planning pass is reported together
// with planning_progress_stalled, which the mode's result decision adds
// (modes/*/sm.hpp result transitions); a refused request carries
// invalid_request besides its causes.  The reference writes every branch as
// a select; this restatement branches, and bounds every read by the counts
// the request gives.
#include <algorithm>
#include <array>
#include <cstring>
#include <vector>

#include "emelk.h"

namespace {

constexpr int32_t k_max_steps = EMELK_PLAN_MAX_STEPS;
constexpr int32_t k_words = EMELK_PLAN_SEQ_WORDS;
constexpr int32_t k_max_seq = k_words * 64;

using seq_mask = std::array<uint64_t, k_words>;

struct plan_state {
  const emelk_plan_request &rq;
  emelk_plan_result &out;
  uint32_t err = 0;
  int32_t step = 0;  // effective step size

  // Sequence set of token i (detail.hpp:190-233): its mask row when masks
  // are given, else the bit of its primary id, else sequence 0.
  seq_mask mask_of(int32_t i) const {
    seq_mask m{};
    const bool words_ok = rq.seq_mask_words > 0 && rq.seq_mask_words <= k_words;
    const int32_t words = words_ok ? rq.seq_mask_words : 0;
    if (rq.seq_masks != nullptr && words_ok && i >= 0) {
      for (int32_t w = 0; w < words; ++w) m[w] = rq.seq_masks[static_cast<size_t>(i) * words + w];
      return m;
    }
    if (rq.seq_primary_ids != nullptr && i >= 0) {
      const int32_t id = rq.seq_primary_ids[i];
      if (id >= 0 && id < words * 64) m[id / 64] = uint64_t{1} << (id % 64);
      return m;
    }
    m[0] = 1;
    return m;
  }

  // Plan storage (detail.hpp:297-346).
  void clear() {
    out.step_count = 0;
    out.total_outputs = 0;
    out.token_indices_count = 0;
  }
  void fail(uint32_t code) {
    err |= code;
    clear();
  }
  bool open_step() {
    if (out.step_count >= k_max_steps) return false;
    out.step_token_offsets[out.step_count] = out.token_indices_count;
    return true;
  }
  bool add_token(int32_t idx) {
    if (out.token_indices_count >= k_max_steps) return false;
    out.step_token_indices[out.token_indices_count++] = idx;
    return true;
  }
  bool close_step(int32_t size) {
    if (size <= 0 || out.step_count >= k_max_steps) return false;
    out.step_sizes[out.step_count++] = size;
    return true;
  }
  void finish_offsets() {
    if (out.step_count >= 0 && out.step_count <= k_max_steps) {
      out.step_token_offsets[out.step_count] = out.token_indices_count;
    }
  }

  // Outputs of the plan (detail.hpp:279-295): every token, the masked
  // tokens, or the last token only.
  int32_t count_outputs() const {
    if (rq.output_all) return rq.n_tokens;
    if (rq.output_mask != nullptr) {
      int32_t n = 0;
      for (int32_t i = 0; i < rq.n_tokens; ++i) n += rq.output_mask[i] != 0 ? 1 : 0;
      return n;
    }
    return rq.n_tokens > 0 ? 1 : 0;
  }

  bool complete() const {  // guards.hpp:9-23
    return err == 0 && out.step_count > 0 && out.total_outputs >= 0 &&
           out.token_indices_count == rq.n_tokens && out.step_count <= k_max_steps &&
           out.step_token_offsets[out.step_count] == out.token_indices_count;
  }
};

bool any_bit(const seq_mask &m) {
  for (uint64_t w : m) {
    if (w != 0) return true;
  }
  return false;
}
bool overlaps(const seq_mask &a, const seq_mask &b) {
  for (int32_t w = 0; w < k_words; ++w) {
    if ((a[w] & b[w]) != 0) return true;
  }
  return false;
}
bool contains(const seq_mask &outer, const seq_mask &inner) {
  for (int32_t w = 0; w < k_words; ++w) {
    if ((outer[w] & inner[w]) != inner[w]) return false;
  }
  return true;
}
bool more_than_one_bit(const seq_mask &m) {
  int32_t bits = 0;
  for (uint64_t w : m) bits += __builtin_popcountll(w);
  return bits > 1;
}

int32_t ceil_steps(int32_t n, int32_t step) { return n / step + (n % step != 0 ? 1 : 0); }

// Request checks of collect_input_errors (detail.hpp:129-185).  The
// per-token scan stops at the counts the request gives (the reference
// reads n_tokens entries whatever the count).
uint32_t input_errors(const emelk_plan_request &rq) {
  uint32_t e = 0;
  if (rq.token_ids == nullptr) e |= EMELK_PLAN_ERR_INVALID_TOKEN_DATA;
  if (rq.n_tokens <= 0) e |= EMELK_PLAN_ERR_INVALID_REQUEST;
  if (rq.n_tokens > k_max_steps) e |= EMELK_PLAN_ERR_OUTPUT_PLAN_FULL;
  const bool words_ok = rq.seq_mask_words > 0 && rq.seq_mask_words <= k_words;
  if (!words_ok) e |= EMELK_PLAN_ERR_INVALID_SEQUENCE_METADATA;
  if (rq.output_mask != nullptr && rq.output_mask_count < rq.n_tokens) {
    e |= EMELK_PLAN_ERR_INVALID_SEQUENCE_METADATA;
  }
  if (rq.seq_masks != nullptr && rq.seq_masks_count < rq.n_tokens) {
    e |= EMELK_PLAN_ERR_INVALID_SEQUENCE_METADATA;
  }
  if (rq.seq_primary_ids != nullptr && rq.seq_primary_ids_count < rq.n_tokens) {
    e |= EMELK_PLAN_ERR_INVALID_SEQUENCE_ID;
  }
  const bool equal_seq = rq.mode == EMELK_PLAN_EQUAL && rq.equal_sequential != 0;
  if (equal_seq && rq.seq_masks != nullptr && rq.seq_primary_ids == nullptr) {
    e |= EMELK_PLAN_ERR_INVALID_SEQUENCE_METADATA;
  }
  const int32_t max_seq = rq.seq_mask_words * 64;
  const int32_t n = std::max(rq.n_tokens, 0);
  if (rq.seq_primary_ids != nullptr) {
    const int32_t scan = std::min(n, rq.seq_primary_ids_count);
    for (int32_t i = 0; i < scan; ++i) {
      const int32_t id = rq.seq_primary_ids[i];
      if (id < 0 || id >= max_seq) e |= EMELK_PLAN_ERR_INVALID_SEQUENCE_ID;
    }
  }
  if (rq.seq_masks != nullptr && words_ok) {
    emelk_plan_result scratch_unused;  // mask_of reads only the request
    plan_state probe{rq, scratch_unused};
    const int32_t scan = std::min(n, rq.seq_masks_count);
    for (int32_t i = 0; i < scan; ++i) {
      const seq_mask m = probe.mask_of(i);
      if (!any_bit(m)) e |= EMELK_PLAN_ERR_INVALID_SEQUENCE_MASK;
      if (equal_seq && more_than_one_bit(m)) e |= EMELK_PLAN_ERR_MULTIPLE_BITS_IN_MASK;
    }
  }
  return e;
}

// ---- modes ------------------------------------------------------------

// simple (modes/simple/actions.hpp:32-54): consecutive chunks of `step`.
void plan_simple(plan_state &S) {
  const int32_t n = S.rq.n_tokens;
  for (int32_t start = 0; start < n; start += S.step) {
    const int32_t size = std::min(S.step, n - start);
    (void)S.open_step();
    for (int32_t i = 0; i < size; ++i) (void)S.add_token(start + i);
    (void)S.close_step(size);
  }
  S.finish_offsets();
}

// sequential (modes/sequential/actions.hpp:30-93): a step starts at the
// first unused token and takes, in order, unused tokens whose sequence set
// lies inside the set of the token taken before them, up to `step` tokens.
// Unused tokens are kept in a linked list in token order, so a step's
// search skips the tokens earlier steps took.
void plan_sequential(plan_state &S) {
  const int32_t n = S.rq.n_tokens;
  std::vector<seq_mask> masks(static_cast<size_t>(n));
  for (int32_t i = 0; i < n; ++i) masks[i] = S.mask_of(i);
  // doubly linked list of the unused tokens in token order; node n is the
  // sentinel (next[n] is the first unused token, n when none is left)
  std::vector<int32_t> next(static_cast<size_t>(n) + 1), prev(static_cast<size_t>(n) + 1);
  for (int32_t i = 0; i <= n; ++i) {
    next[i] = i == n ? (n > 0 ? 0 : n) : (i + 1 < n ? i + 1 : n);
    prev[i] = i == n ? (n > 0 ? n - 1 : n) : (i > 0 ? i - 1 : n);
  }
  auto unlink = [&](int32_t i) {
    next[prev[i]] = next[i];
    prev[next[i]] = prev[i];
  };
  while (next[n] != n) {
    int32_t cur = next[n];  // first unused token
    seq_mask cur_mask = masks[cur];
    if (!S.open_step()) return S.fail(EMELK_PLAN_ERR_OUTPUT_STEPS_FULL);
    int32_t taken = 0;
    for (;;) {
      int32_t after = next[cur];
      unlink(cur);
      ++taken;
      if (!S.add_token(cur)) return S.fail(EMELK_PLAN_ERR_OUTPUT_INDICES_FULL);
      if (taken >= S.step) break;
      while (after != n && !contains(cur_mask, masks[after])) after = next[after];
      if (after == n) break;
      cur = after;
      cur_mask = masks[cur];
    }
    if (!S.close_step(taken)) return S.fail(EMELK_PLAN_ERR_OUTPUT_STEPS_FULL);
  }
  S.finish_offsets();
}

// equal, general path (modes/equal/actions.hpp:34-145): each step picks a
// group of pairwise disjoint sequence sets in token order (with
// equal_sequential and primary ids, each next primary id one above the
// last; the scan stops once the group has one more member than the step
// size, which then leaves no room and stalls), then takes the same number
// of tokens, min(step / group size, fewest available), from every member,
// each member's earliest unused tokens first.  Tokens are bucketed by
// their exact set: a member's tokens are then the next ones of its bucket,
// and a token clashes with the group iff it meets the union of its sets.
void plan_equal_general(plan_state &S) {
  const int32_t n = S.rq.n_tokens;
  std::vector<seq_mask> masks(static_cast<size_t>(n));
  for (int32_t i = 0; i < n; ++i) masks[i] = S.mask_of(i);
  // buckets of equal sets, each a list of token indices in order
  std::vector<int32_t> bucket_of(static_cast<size_t>(n));
  std::vector<std::vector<int32_t>> buckets;
  std::vector<seq_mask> bucket_mask;
  {
    std::vector<int32_t> order(static_cast<size_t>(n));
    for (int32_t i = 0; i < n; ++i) order[i] = i;
    std::stable_sort(order.begin(), order.end(),
                     [&](int32_t x, int32_t y) { return masks[x] < masks[y]; });
    for (int32_t k = 0; k < n; ++k) {
      const int32_t i = order[k];
      if (k == 0 || masks[i] != masks[order[k - 1]]) {
        buckets.emplace_back();
        bucket_mask.push_back(masks[i]);
      }
      bucket_of[i] = static_cast<int32_t>(buckets.size()) - 1;
      buckets.back().push_back(i);  // ascending: stable over token order
    }
  }
  std::vector<int32_t> cursor(buckets.size(), 0);
  std::vector<uint8_t> used(static_cast<size_t>(n), 0);
  std::vector<int32_t> group;
  int32_t n_used = 0;
  while (n_used < n) {
    group.clear();
    seq_mask taken_bits{};
    int32_t last_primary = -1;
    for (int32_t i = 0; i < n; ++i) {
      if (used[i] != 0 || overlaps(taken_bits, masks[i])) continue;
      if (S.rq.equal_sequential != 0 && S.rq.seq_primary_ids != nullptr) {
        const int32_t primary = S.rq.seq_primary_ids[i];
        if (!group.empty() && primary != last_primary + 1) continue;
        last_primary = primary;
      }
      group.push_back(bucket_of[i]);
      for (int32_t w = 0; w < k_words; ++w) taken_bits[w] |= masks[i][w];
      if (static_cast<int32_t>(group.size()) > S.step) break;
    }
    const int32_t n_groups = static_cast<int32_t>(group.size());
    if (n_groups == 0) return S.fail(EMELK_PLAN_ERR_PLANNING_PROGRESS_STALLED);
    int32_t fewest = n + 1;
    for (int32_t b : group) {
      fewest = std::min(fewest, static_cast<int32_t>(buckets[b].size()) - cursor[b]);
    }
    const int32_t per_seq = std::min(S.step / n_groups, fewest);
    if (per_seq <= 0) return S.fail(EMELK_PLAN_ERR_PLANNING_PROGRESS_STALLED);
    if (!S.open_step()) return S.fail(EMELK_PLAN_ERR_OUTPUT_STEPS_FULL);
    for (int32_t b : group) {
      // members with the same set (possible only for an empty set, which
      // the request checks refuse) share a bucket and may run it dry
      if (cursor[b] + per_seq > static_cast<int32_t>(buckets[b].size())) {
        return S.fail(EMELK_PLAN_ERR_ALGORITHM_FAILED);
      }
      for (int32_t k = 0; k < per_seq; ++k) {
        const int32_t i = buckets[b][cursor[b] + k];
        used[i] = 1;
        ++n_used;
        if (!S.add_token(i)) return S.fail(EMELK_PLAN_ERR_OUTPUT_INDICES_FULL);
      }
      cursor[b] += per_seq;
    }
    if (!S.close_step(per_seq * n_groups)) return S.fail(EMELK_PLAN_ERR_OUTPUT_STEPS_FULL);
  }
  S.finish_offsets();
}

// equal, primary-id path (modes/equal/actions.hpp:147-269): the same
// grouping over primary ids only, with each sequence's tokens listed once
// in token order.
void plan_equal_primary(plan_state &S) {
  const int32_t n = S.rq.n_tokens;
  const int32_t *ids = S.rq.seq_primary_ids;
  if (ids == nullptr) return S.fail(EMELK_PLAN_ERR_INVALID_SEQUENCE_ID);
  const int32_t max_seq = S.rq.seq_mask_words * 64;
  std::array<int32_t, k_max_seq> count{}, first{}, taken{};
  std::vector<int32_t> by_seq(static_cast<size_t>(n));
  for (int32_t i = 0; i < n; ++i) {
    if (ids[i] < 0 || ids[i] >= max_seq) return S.fail(EMELK_PLAN_ERR_INVALID_SEQUENCE_ID);
    ++count[ids[i]];
  }
  {
    std::array<int32_t, k_max_seq> cursor{};
    int32_t run = 0;
    for (int32_t s = 0; s < max_seq; ++s) {
      first[s] = run;
      cursor[s] = run;
      run += count[s];
    }
    for (int32_t i = 0; i < n; ++i) by_seq[cursor[ids[i]]++] = i;
  }
  int32_t left_total = n;
  while (left_total > 0) {
    std::array<uint8_t, k_max_seq> in_group{};
    std::array<int32_t, k_max_seq> group{};
    int32_t n_groups = 0;
    int32_t last_primary = -1;
    for (int32_t i = 0; i < n; ++i) {
      const int32_t s = ids[i];
      if (taken[s] >= count[s] || in_group[s] != 0) continue;
      if (S.rq.equal_sequential != 0 && n_groups > 0 && s != last_primary + 1) continue;
      in_group[s] = 1;
      group[n_groups++] = s;
      last_primary = s;
      if (n_groups > S.step) break;
    }
    if (n_groups == 0) return S.fail(EMELK_PLAN_ERR_PLANNING_PROGRESS_STALLED);
    int32_t fewest = n + 1;
    for (int32_t g = 0; g < n_groups; ++g) fewest = std::min(fewest, count[group[g]] - taken[group[g]]);
    const int32_t per_seq = std::min(S.step / n_groups, fewest);
    if (per_seq <= 0) return S.fail(EMELK_PLAN_ERR_PLANNING_PROGRESS_STALLED);
    if (!S.open_step()) return S.fail(EMELK_PLAN_ERR_OUTPUT_STEPS_FULL);
    for (int32_t g = 0; g < n_groups; ++g) {
      const int32_t s = group[g];
      for (int32_t k = 0; k < per_seq; ++k) {
        if (!S.add_token(by_seq[first[s] + taken[s] + k])) {
          return S.fail(EMELK_PLAN_ERR_OUTPUT_INDICES_FULL);
        }
      }
      taken[s] += per_seq;
      left_total -= per_seq;
    }
    if (!S.close_step(per_seq * n_groups)) return S.fail(EMELK_PLAN_ERR_OUTPUT_STEPS_FULL);
  }
  S.finish_offsets();
}

// One mode machine (modes/*/sm.hpp): its entry checks, the planning pass,
// and the result decision, which adds planning_progress_stalled to any
// incomplete plan.
void run_mode(plan_state &S) {
  S.clear();
  S.out.total_outputs = S.count_outputs();
  const int32_t n = S.rq.n_tokens;
  if (S.step <= 0) return S.fail(EMELK_PLAN_ERR_INVALID_STEP_SIZE);
  switch (S.rq.mode) {
    case EMELK_PLAN_SIMPLE:
    case EMELK_PLAN_SEQUENTIAL:
      if (ceil_steps(n, S.step) > k_max_steps) return S.fail(EMELK_PLAN_ERR_OUTPUT_STEPS_FULL);
      if (n > k_max_steps) return S.fail(EMELK_PLAN_ERR_OUTPUT_INDICES_FULL);
      if (S.rq.mode == EMELK_PLAN_SIMPLE) {
        plan_simple(S);
      } else {
        plan_sequential(S);
      }
      break;
    case EMELK_PLAN_EQUAL: {
      const bool primary_path = S.rq.seq_masks == nullptr && S.rq.seq_primary_ids != nullptr;
      if (primary_path) {
        const int32_t max_seq = S.rq.seq_mask_words * 64;
        bool ids_ok = max_seq > 0 && max_seq <= k_max_seq;
        for (int32_t i = 0; ids_ok && i < n; ++i) {
          ids_ok = S.rq.seq_primary_ids[i] >= 0 && S.rq.seq_primary_ids[i] < max_seq;
        }
        if (!ids_ok) return S.fail(EMELK_PLAN_ERR_INVALID_SEQUENCE_ID);
      }
      // step and index storage start empty, so only an oversized request
      // lacks room
      if (n > k_max_steps) return S.fail(EMELK_PLAN_ERR_OUTPUT_INDICES_FULL);
      if (primary_path) {
        plan_equal_primary(S);
      } else {
        plan_equal_general(S);
      }
      break;
    }
    default:
      return S.fail(EMELK_PLAN_ERR_INVALID_MODE);
  }
  if (!S.complete()) S.fail(EMELK_PLAN_ERR_PLANNING_PROGRESS_STALLED);
}

}  // namespace

extern "C" bool emelk_batch_plan_mode(const emelk_plan_request *request,
                                      int32_t effective_step_size, emelk_plan_result *result,
                                      uint32_t *error_out) {
  uint32_t sink = 0;
  uint32_t &err = error_out != nullptr ? *error_out : sink;
  if (request == nullptr || result == nullptr) {
    err = EMELK_PLAN_ERR_INVALID_REQUEST;
    return false;
  }
  plan_state S{*request, *result};
  S.step = effective_step_size;
  // the mode machines trust the outer checks; here only what keeps every
  // read inside the arrays the request gives
  const int32_t n = request->n_tokens;
  const bool words_ok = request->seq_mask_words > 0 && request->seq_mask_words <= k_words;
  if (n < 0 || (request->seq_masks != nullptr && (request->seq_masks_count < n || !words_ok)) ||
      (request->seq_primary_ids != nullptr && request->seq_primary_ids_count < n) ||
      (request->output_mask != nullptr && request->output_mask_count < n)) {
    S.clear();
    err = EMELK_PLAN_ERR_INVALID_REQUEST;
    return false;
  }
  run_mode(S);
  err = S.err != 0 ? S.err : (S.complete() ? 0u : EMELK_PLAN_ERR_INTERNAL_ERROR);
  return err == 0;
}

extern "C" bool emelk_batch_plan(const emelk_plan_request *request, emelk_plan_result *result,
                                 uint32_t *error_out) {
  uint32_t sink = 0;
  uint32_t &err = error_out != nullptr ? *error_out : sink;
  if (request == nullptr || result == nullptr) {
    err = EMELK_PLAN_ERR_INVALID_REQUEST;
    return false;
  }
  plan_state S{*request, *result};
  S.clear();
  // input validation (sm.hpp:28-35): every cause, plus invalid_request
  const uint32_t bad = input_errors(*request);
  if (bad != 0) {
    err = bad | EMELK_PLAN_ERR_INVALID_REQUEST;
    return false;
  }
  // step size (actions.hpp:64-75): n_steps when positive, within [1, n_tokens]
  const int32_t requested = request->n_steps > 0 ? request->n_steps : request->n_tokens;
  S.step = std::max<int32_t>(1, std::min<int32_t>(requested, request->n_tokens));
  if (request->mode != EMELK_PLAN_SIMPLE && request->mode != EMELK_PLAN_EQUAL &&
      request->mode != EMELK_PLAN_SEQUENTIAL) {
    err = EMELK_PLAN_ERR_INVALID_MODE | EMELK_PLAN_ERR_INVALID_REQUEST;  // actions.hpp:101-106
    return false;
  }
  run_mode(S);
  // a failed mode reports its own bits; an incomplete plan without any
  // is an internal error (actions.hpp:113-116)
  err = S.err != 0 ? S.err : (S.complete() ? 0u : EMELK_PLAN_ERR_INTERNAL_ERROR);
  return err == 0;
}

extern "C" emel_error_type emelk_plan_step_sequences(const emelk_plan_request *request,
                                                     const emelk_plan_result *result, int32_t step,
                                                     int32_t *seq_ids_out, int32_t *n_seq_out,
                                                     int32_t *n_tokens_out) {
  if (request == nullptr || result == nullptr || seq_ids_out == nullptr || n_seq_out == nullptr ||
      n_tokens_out == nullptr || step < 0 || step >= result->step_count ||
      result->step_count > k_max_steps) {
    return EMELK_ERR_INVALID_REQUEST;
  }
  const int32_t lo = result->step_token_offsets[step];
  const int32_t hi = result->step_token_offsets[step + 1];
  if (lo < 0 || hi <= lo || hi > result->token_indices_count ||
      hi > request->n_tokens) {
    return EMELK_ERR_INVALID_REQUEST;
  }
  emelk_plan_result unused;
  plan_state probe{*request, unused};
  auto seq_of = [&](int32_t token) -> int32_t {
    if (token < 0 || token >= request->n_tokens) return -1;
    if (request->seq_primary_ids != nullptr) return request->seq_primary_ids[token];
    const seq_mask m = probe.mask_of(token);
    int32_t found = -1;
    for (int32_t w = 0; w < k_words; ++w) {
      if (m[w] == 0) continue;
      if (found >= 0 || (m[w] & (m[w] - 1)) != 0) return -1;  // more than one sequence
      found = w * 64 + __builtin_ctzll(m[w]);
    }
    return found;
  };
  int32_t n_seq = 0;
  int32_t run_len = 0;
  int32_t prev = -2;
  int32_t cur_run = 0;
  for (int32_t k = lo; k < hi; ++k) {
    const int32_t s = seq_of(result->step_token_indices[k]);
    if (s < 0 || s >= EMELK_MAX_SEQUENCES) return EMELK_ERR_INVALID_REQUEST;
    if (s != prev) {
      if (prev != -2) {
        if (run_len == 0) run_len = cur_run;
        if (cur_run != run_len) return EMELK_ERR_INVALID_REQUEST;
      }
      for (int32_t j = 0; j < n_seq; ++j) {
        if (seq_ids_out[j] == s) return EMELK_ERR_INVALID_REQUEST;  // a sequence in two runs
      }
      if (n_seq >= EMELK_MAX_SEQUENCES) return EMELK_ERR_INVALID_REQUEST;
      seq_ids_out[n_seq++] = s;
      prev = s;
      cur_run = 0;
    }
    ++cur_run;
  }
  if (run_len == 0) run_len = cur_run;
  if (cur_run != run_len) return EMELK_ERR_INVALID_REQUEST;
  *n_seq_out = n_seq;
  *n_tokens_out = run_len;
  return EMELK_ERR_NONE;
}
