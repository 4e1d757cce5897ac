"""Host batch planner (emelk_batch_plan, emelk_batch_plan_mode,
emelk_plan_step_sequences) against the known answers of the reference's
planner tests (tests/batch/planner/*.cpp, cited per case), plus plan
invariants on seeded random batches: every token is placed exactly once,
steps respect the step size, equal steps take the same number of tokens from
each of their sequences in token order, and sequential steps nest their
sequence sets."""
import numpy as np
import pytest

import emelk
from emelk import PLAN_EQUAL, PLAN_SEQUENTIAL, PLAN_SIMPLE, PLAN_ERR as E, BatchPlan


def plan(tokens, **kw):
    return BatchPlan(np.asarray(tokens, np.int32), **kw)


# ---- planner_tests.cpp -------------------------------------------------

def test_splits_tokens_into_steps():  # planner_tests.cpp:62-84
    p = plan([1, 2, 3, 4, 5], n_steps=2, mode=PLAN_SIMPLE, output_all=True)
    assert p.accepted and p.error == 0
    assert p.step_sizes == [2, 2, 1] and p.total_outputs == 5
    assert p.steps == [[0, 1], [2, 3], [4]]


def test_equal_mode_fills_single_sequence_steps():  # planner_tests.cpp:86-107
    p = plan(range(1, 11), n_steps=4, mode=PLAN_EQUAL, equal_sequential=False, output_all=True)
    assert p.accepted and p.step_sizes == [4, 4, 2]


@pytest.mark.parametrize("mode", [PLAN_SEQUENTIAL])
def test_seq_mode_uses_sequential_chunking(mode):  # planner_tests.cpp:109-151
    p = plan(range(1, 8), n_steps=3, mode=mode, output_all=True)
    assert p.accepted and p.step_sizes == [3, 3, 1]


def test_equal_mode_supports_sequence_masks():  # planner_tests.cpp:153-180
    p = plan(range(1, 7), n_steps=4, mode=PLAN_EQUAL, seq_masks=[1, 2, 1, 2, 1, 2],
             seq_primary_ids=[0, 1, 0, 1, 0, 1], equal_sequential=True, output_all=True)
    assert p.accepted and p.step_sizes == [4, 2] and p.total_outputs == 6
    assert p.steps == [[0, 2, 1, 3], [4, 5]]


def test_seq_mode_supports_sequence_masks():  # planner_tests.cpp:182-205
    p = plan([1, 2, 3, 4], n_steps=3, mode=PLAN_SEQUENTIAL, seq_masks=[3, 1, 2, 1],
             output_all=True)
    assert p.accepted and p.step_sizes == [3, 1] and p.total_outputs == 4
    assert p.steps == [[0, 1, 3], [2]]


def test_counts_outputs_with_output_mask():  # planner_tests.cpp:207-226
    p = plan([1, 2, 3, 4], n_steps=2, mode=PLAN_SIMPLE, output_mask=[1, 0, 1, 0])
    assert p.accepted and p.total_outputs == 2
    # without a mask and without output_all only the last token is an output
    assert plan([1, 2, 3], n_steps=2).total_outputs == 1


def test_reports_invalid_arguments():  # planner_tests.cpp:228-260
    p = BatchPlan(None, n_steps=2, mode=PLAN_SIMPLE, n_tokens=4)
    assert not p.accepted
    assert p.error == E["invalid_request"] | E["invalid_token_data"]
    p = plan([1, 2, 3], n_steps=1, mode=99, equal_sequential=False)
    assert not p.accepted and p.error == E["invalid_request"] | E["invalid_mode"]
    assert p.step_count == 0 and p.total_outputs == 0


# ---- planner_additional_tests.cpp --------------------------------------

def test_rejects_invalid_token_counts():  # planner_additional_tests.cpp:58-74
    p = BatchPlan(None, n_steps=2, n_tokens=0)
    assert not p.accepted
    # the reference's test names the pair its own flags give: no tokens is
    # itself an invalid request, and null token data adds its own bit
    assert p.error == E["invalid_request"] | E["invalid_token_data"]


def test_equal_and_seq_modes_with_seq_masks():  # planner_additional_tests.cpp:76-126
    for mode in (PLAN_EQUAL, PLAN_SEQUENTIAL):
        p = plan([1, 2, 3, 4], n_steps=2, mode=mode, seq_masks=[1, 1, 2, 2],
                 seq_primary_ids=[0, 0, 1, 1], equal_sequential=True, output_all=True)
        assert p.accepted and p.total_outputs == 4


def test_equal_mode_rejects_coupled_sequences_when_sequential():  # additional:128-152
    p = plan([1, 2], n_steps=2, mode=PLAN_EQUAL, seq_masks=[3, 1], seq_primary_ids=[0, 1],
             equal_sequential=True)
    assert not p.accepted
    assert p.error == E["invalid_request"] | E["multiple_bits_in_mask"]


def test_supports_multiword_sequence_masks():  # planner_additional_tests.cpp:154-175
    p = BatchPlan(np.array([1, 2], np.int32), n_steps=2, mode=PLAN_EQUAL,
                  seq_masks=np.array([0, 1, 0, 2], np.uint64), equal_sequential=False,
                  seq_mask_words=2, n_tokens=2)
    # seq_masks_count counts rows of seq_mask_words words (2 here)
    assert p.accepted and p.step_count == 1 and p.step_sizes == [2]


def test_rejects_unknown_mode():  # planner_additional_tests.cpp:177-193
    p = plan([1, 2], n_steps=2, mode=99)
    assert not p.accepted and p.error == E["invalid_request"] | E["invalid_mode"]


# ---- planner_action_branch_tests.cpp: input guards -----------------------

def test_input_guard_rejects_invalid_metadata():  # planner_action_branch_tests.cpp:71-124
    tok = [1, 2]
    for words in (0, emelk.PLAN_SEQ_WORDS + 1):
        p = plan(tok, seq_mask_words=words)
        assert not p.accepted and p.error & E["invalid_sequence_metadata"]
    p = BatchPlan(np.array(tok, np.int32), output_mask=np.array([1], np.int8))
    assert not p.accepted and p.error & E["invalid_sequence_metadata"]
    p = BatchPlan(np.array(tok, np.int32), seq_masks=np.array([0], np.uint64))
    assert not p.accepted and p.error & E["invalid_sequence_metadata"]
    p = BatchPlan(np.array(tok, np.int32), seq_masks=[1, 1], seq_primary_ids=[0])
    assert not p.accepted and p.error & E["invalid_sequence_id"]
    p = plan(tok, seq_masks=[1, 1], seq_primary_ids=[0, 64])  # 64 needs a second word
    assert not p.accepted and p.error & E["invalid_sequence_id"]
    p = plan(tok, seq_masks=[0, 1], seq_primary_ids=[0, 0])  # a token on no sequence
    assert not p.accepted and p.error & E["invalid_sequence_mask"]
    assert plan(tok, seq_masks=[1, 1], seq_primary_ids=[0, 0]).accepted


def test_equal_sequential_requires_primary_ids():  # planner_action_branch_tests.cpp:126-159
    p = plan([1, 2], mode=PLAN_EQUAL, seq_masks=[1, 2], equal_sequential=True)
    assert not p.accepted and p.error & E["invalid_sequence_metadata"]
    p = plan([1, 2], mode=PLAN_EQUAL, seq_masks=[1, 3], seq_primary_ids=[0, 1])
    assert not p.accepted and p.error & E["multiple_bits_in_mask"]
    assert plan([1, 2], mode=PLAN_EQUAL, seq_masks=[1, 2], seq_primary_ids=[0, 1]).accepted


def test_normalize_step_size_clamps():  # planner_actions_tests.cpp:84-108
    assert plan(range(5), n_steps=0).step_sizes == [5]       # n_steps <= 0: one step
    assert plan(range(5), n_steps=-3).step_sizes == [5]
    assert plan(range(5), n_steps=99).step_sizes == [5]      # clamped to n_tokens


# ---- modes/*_actions_tests.cpp: the mode machines with a given step -------

def mode_plan(tokens, step, **kw):
    return BatchPlan(np.asarray(tokens, np.int32), effective_step_size=step, **kw)


def test_mode_equal_without_masks():  # modes/equal_actions_tests.cpp:139-163
    p = mode_plan(range(1, 6), 2, mode=PLAN_EQUAL)
    assert p.accepted and p.step_sizes == [2, 2, 1]


def test_mode_equal_skips_nonconsecutive_primary():  # equal_actions_tests.cpp:165-193
    p = mode_plan([1, 2, 3], 2, mode=PLAN_EQUAL, seq_masks=[1, 2, 4],
                  seq_primary_ids=[0, 2, 1], equal_sequential=True)
    assert p.accepted and p.step_sizes == [2, 1]
    assert p.steps == [[0, 2], [1]]


def test_mode_equal_rejects_zero_step():  # equal_actions_tests.cpp:195-216
    p = mode_plan([1, 2], 0, mode=PLAN_EQUAL)
    assert not p.accepted and p.error == E["invalid_step_size"]
    assert p.step_count == 0 and p.total_outputs == 0


def test_mode_equal_stalls_when_groups_exceed_step():  # equal_actions_tests.cpp:218-244
    p = mode_plan([1, 2], 1, mode=PLAN_EQUAL, seq_masks=[1, 2], seq_mask_words=1,
                  equal_sequential=False)
    assert not p.accepted and p.error == E["planning_progress_stalled"]
    assert p.step_count == 0 and p.total_outputs == 0


def test_mode_equal_fast_path():  # equal_actions_tests.cpp:246-278
    p = mode_plan(range(1, 7), 4, mode=PLAN_EQUAL, seq_primary_ids=[0, 0, 1, 1, 2, 2],
                  equal_sequential=True)
    assert p.accepted and p.step_sizes == [3, 3] and p.token_indices_count == 6
    assert p.offsets == [0, 3, 6]
    assert p.steps == [[0, 2, 4], [1, 3, 5]]


def test_mode_equal_fast_path_rejections():  # equal_actions_tests.cpp:307-364
    p = mode_plan([1, 2], 2, mode=PLAN_EQUAL, seq_primary_ids=[0, -1])
    assert not p.accepted and p.error == E["invalid_sequence_id"]
    p = mode_plan([1, 2], 1, mode=PLAN_EQUAL, seq_primary_ids=[0, 1], equal_sequential=False)
    assert not p.accepted and p.error == E["planning_progress_stalled"]
    assert p.step_count == 0 and p.total_outputs == 0


def test_mode_sequential_with_masks():  # modes/sequential_actions_tests.cpp:89-116
    p = mode_plan([1, 2, 3, 4], 3, mode=PLAN_SEQUENTIAL, seq_masks=[3, 1, 2, 1])
    assert p.accepted and p.step_sizes == [3, 1]


def test_mode_step_size_zero_fails():  # sequential:118-144, simple:171-195
    for mode in (PLAN_SEQUENTIAL, PLAN_SIMPLE):
        p = mode_plan([1, 2], 0, mode=mode)
        assert not p.accepted and p.error == E["invalid_step_size"]
        assert p.step_count == 0 and p.total_outputs == 0


def test_mode_simple():  # modes/simple_actions_tests.cpp:90-169
    p = mode_plan([1, 2, 3, 4], 2, mode=PLAN_SIMPLE)
    assert p.accepted and p.step_sizes == [2, 2]
    big = np.ones(emelk.PLAN_MAX_STEPS + 1, np.int32)
    p = mode_plan(big, len(big), mode=PLAN_SIMPLE)
    assert not p.accepted and p.error == E["output_indices_full"] and p.step_count == 0
    p = mode_plan(big, 1, mode=PLAN_SIMPLE)
    assert not p.accepted and p.error == E["output_steps_full"] and p.step_count == 0
    # through the outer machine the same request is an oversized plan
    p = BatchPlan(big, n_steps=1)
    assert not p.accepted and p.error == E["invalid_request"] | E["output_plan_full"]


# ---- invariants on seeded random batches -------------------------------

def _check_partition(p, n, step):
    assert sorted(i for s in p.steps for i in s) == list(range(n))
    assert all(0 < len(s) <= step for s in p.steps)
    assert p.step_sizes == [len(s) for s in p.steps]
    assert p.offsets[0] == 0 and p.offsets[-1] == n


@pytest.mark.parametrize("seed", range(12))
def test_plans_partition_the_batch(seed):
    rng = np.random.default_rng(seed)
    n_seq = int(rng.integers(1, 9))
    lens = rng.integers(1, 40, size=n_seq)
    ids = np.concatenate([np.full(l, s, np.int32) for s, l in enumerate(lens)])
    rng.shuffle(ids)
    n = len(ids)
    step = int(rng.integers(1, 3 * n_seq + 8))
    tokens = rng.integers(0, 32000, size=n).astype(np.int32)
    for mode in (PLAN_SIMPLE, PLAN_SEQUENTIAL):
        p = plan(tokens, n_steps=step, mode=mode, seq_primary_ids=ids)
        assert p.accepted, (mode, p.error)
        _check_partition(p, n, min(step, n))
    p = plan(tokens, n_steps=step, mode=PLAN_EQUAL, seq_primary_ids=ids, equal_sequential=False)
    if min(step, n) < n_seq:
        # a step smaller than the number of sequences stalls, as the
        # reference's grouping does (it admits one member past the step size)
        assert not p.accepted and p.error == E["planning_progress_stalled"]
        return
    assert p.accepted, p.error
    _check_partition(p, n, min(step, n))
    seen = {s: [] for s in range(n_seq)}
    for k, s in enumerate(p.steps):
        seqs, per = p.step_sequences(k)
        assert per * len(seqs) == len(s)
        for g, sq in enumerate(seqs):
            chunk = s[g * per:(g + 1) * per]
            assert all(ids[i] == sq for i in chunk)
            seen[sq].extend(chunk)
    for sq, got in seen.items():  # each sequence's tokens in token order
        assert got == [i for i in range(n) if ids[i] == sq]


def test_sequential_steps_nest_their_sequence_sets():
    rng = np.random.default_rng(3)
    n = 200
    masks = rng.integers(1, 16, size=n).astype(np.uint64)
    p = plan(np.arange(n, dtype=np.int32), n_steps=7, mode=PLAN_SEQUENTIAL, seq_masks=masks)
    assert p.accepted
    _check_partition(p, n, 7)
    for s in p.steps:
        for a, b in zip(s, s[1:]):
            assert a < b and (int(masks[a]) & int(masks[b])) == int(masks[b])


def test_step_sequences_rejects_mixed_steps():
    # a simple-mode step over interleaved sequences is not one decoder step
    p = plan(range(4), n_steps=4, mode=PLAN_SIMPLE, seq_primary_ids=[0, 1, 0, 1])
    assert p.accepted
    with pytest.raises(RuntimeError):
        p.step_sequences(0)
    q = plan(range(4), n_steps=4, mode=PLAN_SIMPLE, seq_primary_ids=[0, 0, 1, 1])
    assert q.step_sequences(0) == ([0, 1], 2)
    r = plan(range(3), n_steps=3, mode=PLAN_SIMPLE, seq_primary_ids=[0, 0, 1])
    with pytest.raises(RuntimeError):
        r.step_sequences(0)
    with pytest.raises(RuntimeError):
        q.step_sequences(1)


# ---- the bucketed / linked-list passes against the step rules written out
# token by token (modes/sequential/actions.hpp:30-93, modes/equal/
# actions.hpp:34-139), on seeded batches with multi-sequence masks ----------

def _sequential_rules(masks, step):
    n = len(masks)
    used = [False] * n
    steps = []
    while not all(used):
        cur = used.index(False)
        cur_mask = masks[cur]
        cur_step = []
        while True:
            used[cur] = True
            cur_step.append(cur)
            if len(cur_step) >= step:
                break
            nxt = next((j for j in range(cur + 1, n)
                        if not used[j] and (cur_mask & masks[j]) == masks[j]), None)
            if nxt is None:
                break
            cur, cur_mask = nxt, masks[nxt]
        steps.append(cur_step)
    return steps


def _equal_rules(masks, step):
    n = len(masks)
    used = [False] * n
    steps = []
    while not all(used):
        group = []
        for i in range(n):
            if used[i] or any(g & masks[i] for g in group):
                continue
            group.append(masks[i])
            if len(group) > step:
                break
        fewest = min(sum(1 for i in range(n) if not used[i] and masks[i] == g) for g in group)
        per = min(step // len(group), fewest)
        if per <= 0:
            return None
        cur_step = []
        for g in group:
            take = [i for i in range(n) if not used[i] and masks[i] == g][:per]
            for i in take:
                used[i] = True
            cur_step.extend(take)
        steps.append(cur_step)
    return steps


@pytest.mark.parametrize("seed", range(10))
def test_fast_passes_follow_the_step_rules(seed):
    rng = np.random.default_rng(100 + seed)
    n = int(rng.integers(1, 300))
    n_seq = int(rng.integers(1, 12))
    step = int(rng.integers(1, 40))
    # sequential: arbitrary non-empty sets over n_seq sequences
    masks = rng.integers(1, 1 << n_seq, size=n).astype(np.uint64)
    p = plan(np.arange(n, dtype=np.int32), n_steps=step, mode=PLAN_SEQUENTIAL, seq_masks=masks)
    assert p.accepted and p.steps == _sequential_rules([int(m) for m in masks], min(step, n))
    # equal (general path): disjoint sets, a few sequences sharing tokens
    groups = [1 << s for s in range(n_seq)] + [3 << (2 * k) for k in range(n_seq // 2)]
    masks = np.array([groups[j] for j in rng.integers(0, len(groups), size=n)], np.uint64)
    p = plan(np.arange(n, dtype=np.int32), n_steps=step, mode=PLAN_EQUAL, seq_masks=masks,
             equal_sequential=False)
    want = _equal_rules([int(m) for m in masks], min(step, n))
    if want is None:
        assert not p.accepted and p.error == E["planning_progress_stalled"]
    else:
        assert p.accepted and p.steps == want
