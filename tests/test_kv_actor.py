"""Known-answer tests of the host KV actor through the C ABI, ported from the
reference's tests/memory/kv/lifecycle_tests.cpp (line ranges cited per test)
and tests/memory/hybrid/lifecycle_tests.cpp, plus the new evict/compact
events.  CPU only: the actor never touches the GPU."""
import ctypes

import numpy as np
import pytest

import emelk
from emelk import (ERR_BACKEND, ERR_INVALID_REQUEST, ERR_NONE, ERR_OUT_OF_MEMORY, KvActor,
                   Snapshot)


def fresh(max_sequences, max_blocks, block_tokens):
    a = KvActor()
    ok, err = a.reserve(max_sequences, max_blocks, block_tokens)
    assert ok and err == ERR_NONE
    return a


class CopyProbe:
    """block_copy_probe + copy_block_cb (lifecycle_tests.cpp:16-47)."""

    def __init__(self, accepted=True, error=ERR_NONE):
        self.calls = 0
        self.src = self.dst = -1
        self.bt = 0
        self.accepted = accepted
        self.error = error
        self.fn = emelk.COPY_BLOCK_FN(self._cb)

    def _cb(self, src, dst, bt, user, err_out):
        self.calls += 1
        self.src, self.dst, self.bt = src, dst, bt
        if err_out:
            err_out[0] = self.error
        return self.accepted


def test_geometry_helpers():  # 51-62 (restated in the C++ header; exercised via allocate)
    a = fresh(4, 16, 4)
    for tokens, blocks in [(1, 1), (4, 1), (5, 2)]:
        b = fresh(4, 16, 4)
        b.allocate_sequence(0)
        ok, err, cnt = b.allocate_slots(0, tokens)
        assert ok and cnt == blocks
    a.close()


def test_reserve_success_and_failure():  # 64-84
    a = KvActor()
    assert a.reserve(8, 16, 4) == (True, ERR_NONE)
    assert a.reserve(999999, 16, 4) == (False, ERR_INVALID_REQUEST)
    assert a.reserve(8, 40000, 4) == (False, ERR_INVALID_REQUEST)
    # non-positive fields resolve to the defaults
    assert a.reserve(0, 0, 0) == (True, ERR_NONE)
    assert a.view().block_tokens == 16 and a.view().max_sequences == 256
    assert a.free_count() == 32768


def test_allocate_sequence_idempotent():  # 86-107
    a = fresh(8, 8, 2)
    assert a.allocate_sequence(3)[0]
    assert a.allocate_slots(3, 3)[0]
    assert a.allocate_sequence(3)[0]
    v = a.view()
    assert v.is_sequence_active(3) and v.sequence_length(3) == 3


def test_block_oom():  # 109-130
    a = fresh(4, 2, 1)
    a.allocate_sequence(0)
    ok, err, cnt = a.allocate_slots(0, 3)
    assert not ok and err == ERR_OUT_OF_MEMORY and cnt == 0


def test_branch_refcounts_and_free_pool():  # 132-209
    a = fresh(8, 8, 2)
    a.allocate_sequence(1)
    ok, err, cnt = a.allocate_slots(1, 4)
    assert ok and cnt == 2
    p0, p1 = a.lookup_kv_block(1, 0), a.lookup_kv_block(1, 2)
    assert p0 >= 0 and p1 >= 0 and p0 != p1
    assert a.branch_sequence(1, 2)[0]
    assert a.lookup_kv_block(2, 0) == p0 and a.lookup_kv_block(2, 2) == p1
    assert a.block_refs(p0) == 2
    assert a.free_sequence(2)[0]
    assert a.view().is_sequence_active(1)
    a.allocate_sequence(3)
    assert a.allocate_slots(3, 2)[0]
    fresh_block = a.lookup_kv_block(3, 0)
    assert fresh_block not in (p0, p1)
    assert a.free_sequence(1)[0]
    a.allocate_sequence(4)
    assert a.allocate_slots(4, 4)[0]
    r0, r1 = a.lookup_kv_block(4, 0), a.lookup_kv_block(4, 2)
    assert {r0, r1} == {p0, p1}


def test_mapping_order_is_deterministic():  # 211-254
    a = fresh(8, 6, 1)
    a.allocate_sequence(0)
    a.allocate_sequence(1)
    assert a.allocate_slots(0, 1)[0] and a.allocate_slots(1, 1)[0]
    assert a.lookup_kv_block(0, 0) == 0 and a.lookup_kv_block(1, 0) == 1
    assert a.allocate_slots(0, 3)[0]
    assert [a.lookup_kv_block(0, p) for p in (1, 2, 3)] == [2, 3, 4]


def test_recycles_multiblock_sequence_in_logical_order():  # 256-294
    a = fresh(2, 4, 2)
    a.allocate_sequence(0)
    assert a.allocate_slots(0, 4)[0]
    assert a.lookup_kv_block(0, 0) == 0 and a.lookup_kv_block(0, 2) == 1
    assert a.free_sequence(0)[0]
    a.allocate_sequence(1)
    assert a.allocate_slots(1, 4)[0]
    assert a.lookup_kv_block(1, 0) == 0 and a.lookup_kv_block(1, 2) == 1


def test_splits_shared_partial_tail_before_append():  # 296-356
    a = fresh(3, 4, 4)
    a.allocate_sequence(0)
    assert a.allocate_slots(0, 2)[0]
    tail = a.lookup_kv_block(0, 0)
    assert a.branch_sequence(0, 1)[0]
    assert a.lookup_kv_block(1, 0) == tail
    ok, err, cnt = a.allocate_slots(1, 1)
    assert not ok and err == ERR_INVALID_REQUEST and cnt == 0
    assert a.lookup_kv_block(1, 0) == tail
    probe = CopyProbe()
    ok, err, cnt = a.allocate_slots(1, 1, copy_block=probe.fn)
    assert ok and err == ERR_NONE and cnt == 1
    assert probe.calls == 1 and probe.src == tail and probe.bt == 4
    assert probe.dst == a.lookup_kv_block(1, 0)
    v = a.view()
    assert v.sequence_length(0) == 2 and v.sequence_length(1) == 3
    assert a.lookup_kv_block(0, 0) == tail and a.lookup_kv_block(1, 0) != tail
    assert a.lookup_kv_block(1, 2) == a.lookup_kv_block(1, 0)
    assert a.block_refs(tail) == 1


def test_tail_copy_failure_maps_error_and_keeps_state():
    # effect_copy_shared_tail_block result routing (kv/sm.hpp:146-153)
    a = fresh(3, 4, 4)
    a.allocate_sequence(0)
    a.allocate_slots(0, 2)
    a.branch_sequence(0, 1)
    free_before = a.free_count()
    ok, err, _ = a.allocate_slots(1, 1, copy_block=CopyProbe(False, ERR_NONE).fn)
    assert not ok and err == ERR_BACKEND
    ok, err, _ = a.allocate_slots(1, 1, copy_block=CopyProbe(True, ERR_OUT_OF_MEMORY).fn)
    assert not ok and err == ERR_OUT_OF_MEMORY
    assert a.free_count() == free_before and a.view().sequence_length(1) == 2


def test_failed_tail_split_keeps_map_and_free_stack(tmp_path):  # 358-399
    # White-box: the effect is driven directly on hand-built state (old tail
    # refcount 0), as the reference test does with action::context.
    import os
    import subprocess
    root = os.path.normpath(os.path.join(os.path.dirname(__file__), ".."))
    csrc = os.path.join(root, "emel.cpp_amd", "csrc")
    exe = str(tmp_path / "actor_whitebox")
    subprocess.run(["g++", "-std=c++20", "-O1", "-I", csrc, "-I", os.path.join(root, "include"),
                    os.path.join(root, "tests", "cpp", "actor_whitebox.cpp"),
                    os.path.join(csrc, "kv_actor.cpp"), "-o", exe], check=True)
    res = subprocess.run([exe], capture_output=True, text=True)
    assert res.returncode == 0, res.stdout + res.stderr


def test_append_and_rollback_use_partial_tail_capacity():  # 401-449
    a = fresh(2, 4, 16)
    a.allocate_sequence(0)
    ok, err, cnt = a.allocate_slots(0, 1)
    assert ok and cnt == 1
    first = a.lookup_kv_block(0, 0)
    ok, err, cnt = a.allocate_slots(0, 1)
    assert ok and cnt == 0 and a.lookup_kv_block(0, 1) == first
    assert a.view().sequence_length(0) == 2
    ok, err, cnt = a.rollback_slots(0, 1)
    assert ok and cnt == 0 and a.lookup_kv_block(0, 0) == first
    assert a.view().sequence_length(0) == 1
    ok, err, cnt = a.rollback_slots(0, 5)
    assert ok and cnt == 1 and a.view().sequence_length(0) == 0 and a.free_count() == 4


def test_validation_paths():  # 451-521
    a = fresh(4, 4, 2)
    assert a.allocate_sequence(-1) == (False, ERR_INVALID_REQUEST)
    assert a.allocate_slots(1, 1)[:2] == (False, ERR_INVALID_REQUEST)
    assert a.branch_sequence(0, 0) == (False, ERR_INVALID_REQUEST)
    assert a.free_sequence(-1) == (False, ERR_INVALID_REQUEST)
    assert a.rollback_slots(0, 1)[:2] == (False, ERR_INVALID_REQUEST)
    assert a.reserve(4, 4, 2) == (True, ERR_NONE)
    # free of an inactive but valid sequence is accepted as a no-op
    assert a.free_sequence(2) == (True, ERR_NONE)
    # null out-params go to a sink
    assert a.allocate_sequence(0, error_out=False)[0]
    ok, _, _ = a.allocate_slots(0, 1, block_count_out=False, error_out=False)
    assert ok


def test_capture_view_tracks_state_and_rejects_null():  # 523-551
    a = fresh(8, 8, 2)
    a.allocate_sequence(0)
    assert a.allocate_slots(0, 4)[0]
    snap = Snapshot()
    assert a.capture_view(snap) == (True, ERR_NONE)
    assert snap.is_sequence_active(0) and snap.sequence_length(0) == 4
    assert snap.lookup_kv_block(0, 0) >= 0 and snap.lookup_recurrent_slot(0) == -1
    assert snap.max_sequences == 8 and snap.block_tokens == 2
    assert a.capture_view(None) == (False, ERR_INVALID_REQUEST)


def test_interleaved_sequences_get_disjoint_pages():
    # tests/text/generator/detail_tests.cpp:2562-2641 (interleaved sequences,
    # free -> realloc returns the identity map)
    a = fresh(4, 64, 4)
    a.allocate_sequence(0)
    a.allocate_sequence(1)
    for _ in range(5):
        assert a.allocate_slots(0, 3)[0]
        assert a.allocate_slots(1, 2)[0]
    v = a.view()
    b0 = set(v.sequence_kv_blocks[0][:v.sequence_kv_block_count[0]])
    b1 = set(v.sequence_kv_blocks[1][:v.sequence_kv_block_count[1]])
    assert not (b0 & b1)
    a.free_sequence(0)
    a.free_sequence(1)
    a2 = fresh(4, 64, 4)
    a2.allocate_sequence(0)
    a2.allocate_slots(0, 20)
    assert [a2.lookup_kv_block(0, 4 * i) for i in range(5)] == list(range(5))


def test_hybrid_binding_dispatches_through_table():
    # hybrid/context.hpp:77-89 + tests/memory/hybrid/lifecycle_tests.cpp:49-155:
    # a filled binding routes every event to the same actor.
    a = KvActor()
    b = a.binding()
    assert b.actor == a.handle
    assert all(getattr(b, f) for f, _ in emelk.KvBinding._fields_)
    reserve = ctypes.CFUNCTYPE(ctypes.c_bool, ctypes.c_void_p,
                               ctypes.POINTER(emelk.EvReserve))(b.dispatch_reserve)
    err = ctypes.c_int32(0)
    ev = emelk.EvReserve(4, 8, 2, ctypes.pointer(err))
    assert reserve(b.actor, ctypes.byref(ev)) and err.value == 0
    alloc_seq = ctypes.CFUNCTYPE(ctypes.c_bool, ctypes.c_void_p,
                                 ctypes.POINTER(emelk.EvAllocateSequence))(
        b.dispatch_allocate_sequence)
    assert alloc_seq(b.actor, ctypes.byref(emelk.EvAllocateSequence(1, None)))
    assert a.view().is_sequence_active(1)


def test_set_free_order_installs_permutation():
    a = fresh(2, 16, 4)
    order = np.random.default_rng(7).permutation(16).astype(np.uint16)
    a.set_free_order(order)
    a.allocate_sequence(0)
    assert a.allocate_slots(0, 64)[0]
    assert [a.lookup_kv_block(0, 4 * i) for i in range(16)] == list(order)
    with pytest.raises(ValueError):
        a.set_free_order(order)  # free stack is now empty: count mismatch


def test_export_block_tables():
    a = fresh(4, 32, 4)
    for s in range(3):
        a.allocate_sequence(s)
        a.allocate_slots(s, 4 * (s + 1) + 1)
    t = a.export_block_tables([2, 0], 8)
    v = a.view()
    assert list(t[0][:4]) == list(v.sequence_kv_blocks[2][:4]) and t[0][4] == emelk.INVALID_KV_BLOCK
    assert list(t[1][:2]) == list(v.sequence_kv_blocks[0][:2]) and t[1][2] == emelk.INVALID_KV_BLOCK
    with pytest.raises(ValueError):
        a.export_block_tables([3], 8)  # inactive


def test_evict_blocks_and_compact_renumber_live_pages():
    a = fresh(4, 32, 4)
    a.set_free_order(np.random.default_rng(1).permutation(32).astype(np.uint16))
    for s in range(3):
        a.allocate_sequence(s)
        assert a.allocate_slots(s, 30)[0]  # 8 blocks each, last one holds 2 tokens
    before = {s: [a.lookup_kv_block(s, 4 * i) for i in range(8)] for s in range(3)}
    ok, err, removed = a.evict_blocks(1, [0, 5, 7])
    assert ok and removed == 4 + 4 + 2
    assert a.view().sequence_length(1) == 20
    assert [a.lookup_kv_block(1, 4 * i) for i in range(5)] == \
        [before[1][i] for i in (1, 2, 3, 4, 6)]
    for b in (before[1][0], before[1][5], before[1][7]):
        assert a.block_refs(b) == 0
    ok, err, removed = a.evict_blocks(1, [9])
    assert not ok and err == ERR_INVALID_REQUEST
    ok, err, removed = a.evict_blocks(1, [1, 1])
    assert not ok and err == ERR_INVALID_REQUEST
    logical = {s: [a.lookup_kv_block(s, 4 * i) for i in range(a.view().sequence_kv_block_count[s])]
               for s in range(3)}
    ok, err, moves = a.compact()
    assert ok and err == ERR_NONE
    n_live = 8 + 8 + 5
    srcs = [m[0] for m in moves]
    dsts = [m[1] for m in moves]
    assert all(s >= n_live for s in srcs) and all(d < n_live for d in dsts)
    assert not set(srcs) & set(dsts)
    remap = dict(moves)
    for s in range(3):
        now = [a.lookup_kv_block(s, 4 * i) for i in range(len(logical[s]))]
        assert now == [remap.get(b, b) for b in logical[s]]
        assert all(b < n_live for b in now)
    assert a.free_count() == 32 - n_live
    # later pops continue ascending above the live set
    a.allocate_sequence(3)
    assert a.allocate_slots(3, 8)[0]
    assert [a.lookup_kv_block(3, 0), a.lookup_kv_block(3, 4)] == [n_live, n_live + 1]
    ok, err, moves = a.compact(max_moves=0)
    assert ok and moves == []


def test_compact_rejects_short_move_buffer():
    a = fresh(2, 8, 1)
    a.allocate_sequence(0)
    a.allocate_slots(0, 6)
    a.evict_blocks(0, [0, 1])
    ok, err, moves = a.compact(max_moves=1)
    assert not ok and err == ERR_INVALID_REQUEST
    assert a.lookup_kv_block(0, 0) == 2  # unchanged
