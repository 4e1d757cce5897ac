"""Python host binding of libemelk.so (the MI355X KV-cache hot path).

ctypes over the C ABI declared in include/emelk.h.  The library is the only
implementation: if it is missing, importing this module raises.  Device
buffers are passed as raw HIP device addresses; helpers accept torch tensors
and take their ``data_ptr()`` and the current torch stream.

Mirrors the reference's memory/kv actor API (src/emel/memory/kv/sm.hpp:364-507,
src/emel/memory/events.hpp:9-62): ``KvActor.process_event``-style methods take
the same fields and return ``(accepted, error, out)``.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.normpath(os.path.join(_HERE, "..", "lib", "libemelk.so"))

ERR_NONE = 0
ERR_INVALID_REQUEST = 1 << 0
ERR_BACKEND = 1 << 1
ERR_INTERNAL = 1 << 2
ERR_OUT_OF_MEMORY = 1 << 3
ERR_UNTRACKED = 1 << 4

MAX_SEQUENCES = 256
MAX_BLOCKS_PER_SEQUENCE = 4096
MAX_BLOCKS = 32768
INVALID_KV_BLOCK = 0xFFFF

KV_F16 = 1
KV_Q8_0 = 8

c_i32p = ctypes.POINTER(ctypes.c_int32)
COPY_BLOCK_FN = ctypes.CFUNCTYPE(ctypes.c_bool, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                 ctypes.c_void_p, c_i32p)
COPY_STATE_FN = ctypes.CFUNCTYPE(ctypes.c_bool, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p,
                                 c_i32p)


class EvReserve(ctypes.Structure):
    _fields_ = [("max_sequences", ctypes.c_int32), ("max_blocks", ctypes.c_int32),
                ("block_tokens", ctypes.c_int32), ("error_out", c_i32p)]


class EvAllocateSequence(ctypes.Structure):
    _fields_ = [("seq_id", ctypes.c_int32), ("error_out", c_i32p)]


class EvAllocateSlots(ctypes.Structure):
    _fields_ = [("seq_id", ctypes.c_int32), ("token_count", ctypes.c_int32),
                ("block_count_out", c_i32p), ("error_out", c_i32p),
                ("copy_block", ctypes.c_void_p), ("copy_block_user_data", ctypes.c_void_p)]


class EvBranchSequence(ctypes.Structure):
    _fields_ = [("parent_seq_id", ctypes.c_int32), ("child_seq_id", ctypes.c_int32),
                ("copy_state", ctypes.c_void_p), ("copy_state_user_data", ctypes.c_void_p),
                ("error_out", c_i32p)]


class EvFreeSequence(ctypes.Structure):
    _fields_ = [("seq_id", ctypes.c_int32), ("error_out", c_i32p)]


class EvRollbackSlots(ctypes.Structure):
    _fields_ = [("seq_id", ctypes.c_int32), ("token_count", ctypes.c_int32),
                ("block_count_out", c_i32p), ("error_out", c_i32p)]


class Snapshot(ctypes.Structure):
    _fields_ = [("max_sequences", ctypes.c_int32), ("block_tokens", ctypes.c_int32),
                ("sequence_active", ctypes.c_uint8 * MAX_SEQUENCES),
                ("sequence_length_values", ctypes.c_int32 * MAX_SEQUENCES),
                ("sequence_kv_block_count", ctypes.c_int32 * MAX_SEQUENCES),
                ("sequence_kv_blocks", (ctypes.c_uint16 * MAX_BLOCKS_PER_SEQUENCE) * MAX_SEQUENCES),
                ("sequence_recurrent_slot", ctypes.c_int32 * MAX_SEQUENCES)]

    # view::snapshot helpers (src/emel/memory/view.hpp:69-116)
    def is_sequence_active(self, seq: int) -> bool:
        return 0 <= seq < self.max_sequences and seq < MAX_SEQUENCES and \
            self.sequence_active[seq] != 0

    def sequence_length(self, seq: int) -> int:
        return self.sequence_length_values[seq] if self.is_sequence_active(seq) else 0

    def lookup_kv_block(self, seq: int, pos: int) -> int:
        if not self.is_sequence_active(seq) or pos < 0 or self.block_tokens <= 0:
            return -1
        if pos >= self.sequence_length_values[seq]:
            return -1
        n = self.sequence_kv_block_count[seq]
        if n <= 0 or n > MAX_BLOCKS_PER_SEQUENCE:
            return -1
        lb = pos // self.block_tokens
        if lb >= n:
            return -1
        b = self.sequence_kv_blocks[seq][lb]
        return -1 if b == INVALID_KV_BLOCK else int(b)

    def lookup_recurrent_slot(self, seq: int) -> int:
        return self.sequence_recurrent_slot[seq] if self.is_sequence_active(seq) else -1


class EvCaptureView(ctypes.Structure):
    _fields_ = [("snapshot_out", ctypes.POINTER(Snapshot)), ("error_out", c_i32p)]


class EvEvictBlocks(ctypes.Structure):
    _fields_ = [("seq_id", ctypes.c_int32), ("logical_blocks", c_i32p),
                ("block_count", ctypes.c_int32), ("tokens_removed_out", c_i32p),
                ("error_out", c_i32p)]


class EvCompact(ctypes.Structure):
    _fields_ = [("moves_out", c_i32p), ("max_moves", ctypes.c_int32),
                ("move_count_out", c_i32p), ("error_out", c_i32p)]


class KvBinding(ctypes.Structure):
    _fields_ = [("actor", ctypes.c_void_p)] + [
        (n, ctypes.c_void_p) for n in (
            "dispatch_reserve", "dispatch_allocate_sequence", "dispatch_allocate_slots",
            "dispatch_branch_sequence", "dispatch_free_sequence", "dispatch_rollback_slots",
            "dispatch_capture_view")]


class Geometry(ctypes.Structure):
    _fields_ = [("n_layer", ctypes.c_int32), ("n_head", ctypes.c_int32),
                ("n_head_kv", ctypes.c_int32), ("head_dim", ctypes.c_int32),
                ("block_tokens", ctypes.c_int32), ("max_blocks", ctypes.c_int32),
                ("kv_type", ctypes.c_int32)]


class RopeParams(ctypes.Structure):
    _fields_ = [("n_rot", ctypes.c_int32), ("x0_stride", ctypes.c_int32),
                ("x1_stride", ctypes.c_int32), ("x1_offset", ctypes.c_int32),
                ("x1_half_rot_offset", ctypes.c_int32), ("freq_base", ctypes.c_float)]


# rope_pairing presets (text/generator/detail.hpp:39-50)
NORMAL_PAIRING = (2, 2, 1, 0)
NEOX_PAIRING = (1, 1, 0, 1)


# Batch planner (src/emel/batch/planner/): modes, limits and error bits.
PLAN_SIMPLE, PLAN_EQUAL, PLAN_SEQUENTIAL = 0, 1, 2
PLAN_MAX_STEPS = 4096
PLAN_SEQ_WORDS = 4
PLAN_ERR = {
    "invalid_request": 1 << 0, "invalid_token_data": 1 << 1, "invalid_step_size": 1 << 2,
    "invalid_sequence_metadata": 1 << 3, "invalid_sequence_id": 1 << 4,
    "invalid_sequence_mask": 1 << 5, "multiple_bits_in_mask": 1 << 6, "invalid_mode": 1 << 8,
    "output_plan_full": 1 << 9, "output_indices_full": 1 << 10, "output_steps_full": 1 << 11,
    "planning_progress_stalled": 1 << 12, "algorithm_failed": 1 << 13,
    "internal_error": 1 << 15,
}


class PlanRequest(ctypes.Structure):
    _fields_ = [("token_ids", c_i32p), ("n_tokens", ctypes.c_int32),
                ("n_steps", ctypes.c_int32), ("mode", ctypes.c_int32),
                ("seq_masks", ctypes.POINTER(ctypes.c_uint64)), ("seq_masks_count", ctypes.c_int32),
                ("seq_primary_ids", c_i32p), ("seq_primary_ids_count", ctypes.c_int32),
                ("equal_sequential", ctypes.c_int32), ("seq_mask_words", ctypes.c_int32),
                ("output_mask", ctypes.POINTER(ctypes.c_int8)), ("output_mask_count", ctypes.c_int32),
                ("output_all", ctypes.c_int32)]


class PlanResult(ctypes.Structure):
    _fields_ = [("step_count", ctypes.c_int32), ("total_outputs", ctypes.c_int32),
                ("token_indices_count", ctypes.c_int32),
                ("step_sizes", ctypes.c_int32 * PLAN_MAX_STEPS),
                ("step_token_indices", ctypes.c_int32 * PLAN_MAX_STEPS),
                ("step_token_offsets", ctypes.c_int32 * (PLAN_MAX_STEPS + 1))]


# (name, restype, argtypes) for every symbol include/emelk.h declares.
_P = ctypes.c_void_p
_SIGNATURES = [
    ("emelk_kv_actor_create", _P, []),
    ("emelk_kv_actor_destroy", None, [_P]),
    ("emelk_kv_reserve", ctypes.c_bool, [_P, ctypes.POINTER(EvReserve)]),
    ("emelk_kv_allocate_sequence", ctypes.c_bool, [_P, ctypes.POINTER(EvAllocateSequence)]),
    ("emelk_kv_allocate_slots", ctypes.c_bool, [_P, ctypes.POINTER(EvAllocateSlots)]),
    ("emelk_kv_branch_sequence", ctypes.c_bool, [_P, ctypes.POINTER(EvBranchSequence)]),
    ("emelk_kv_free_sequence", ctypes.c_bool, [_P, ctypes.POINTER(EvFreeSequence)]),
    ("emelk_kv_rollback_slots", ctypes.c_bool, [_P, ctypes.POINTER(EvRollbackSlots)]),
    ("emelk_kv_capture_view", ctypes.c_bool, [_P, ctypes.POINTER(EvCaptureView)]),
    ("emelk_kv_view", ctypes.POINTER(Snapshot), [_P]),
    ("emelk_kv_lookup_kv_block", ctypes.c_int32, [_P, ctypes.c_int32, ctypes.c_int32]),
    ("emelk_kv_evict_blocks", ctypes.c_bool, [_P, ctypes.POINTER(EvEvictBlocks)]),
    ("emelk_kv_compact", ctypes.c_bool, [_P, ctypes.POINTER(EvCompact)]),
    ("emelk_kv_bind", None, [_P, ctypes.POINTER(KvBinding)]),
    ("emelk_kv_export_block_tables", ctypes.c_uint32,
     [_P, c_i32p, ctypes.c_int32, ctypes.POINTER(ctypes.c_uint16), ctypes.c_int32]),
    ("emelk_kv_set_free_order", ctypes.c_uint32,
     [_P, ctypes.POINTER(ctypes.c_uint16), ctypes.c_int32]),
    ("emelk_kv_block_refs", ctypes.c_int32, [_P, ctypes.c_int32]),
    ("emelk_kv_free_count", ctypes.c_int32, [_P]),
    ("emelk_kv_pool_bytes", ctypes.c_uint32,
     [ctypes.POINTER(Geometry), ctypes.POINTER(ctypes.c_uint64)]),
    ("emelk_kv_append", ctypes.c_uint32,
     [ctypes.POINTER(Geometry), _P, _P, ctypes.c_int32, _P, _P, ctypes.c_int32, ctypes.c_int32,
      _P, _P, ctypes.c_int32, _P]),
    ("emelk_kv_gather", ctypes.c_uint32,
     [ctypes.POINTER(Geometry), _P, _P, ctypes.c_int32, ctypes.c_int32, _P, _P, ctypes.c_int32,
      _P, _P, ctypes.c_int32, _P]),
    ("emelk_kv_copy_blocks", ctypes.c_uint32,
     [ctypes.POINTER(Geometry), _P, _P, _P, ctypes.c_int32, _P]),
    ("emelk_attn_decode_workspace_size", ctypes.c_uint32,
     [ctypes.POINTER(Geometry), ctypes.c_int32, ctypes.c_int32, ctypes.POINTER(ctypes.c_uint64)]),
    ("emelk_attn_decode_plan", ctypes.c_uint32,
     [ctypes.POINTER(Geometry), ctypes.c_int32, ctypes.c_int32, c_i32p, c_i32p,
      ctypes.POINTER(ctypes.c_uint64)]),
    ("emelk_attn_decode", ctypes.c_uint32,
     [ctypes.POINTER(Geometry), _P, _P, ctypes.c_int32, _P, _P, ctypes.c_int32, _P,
      ctypes.c_int32, _P, ctypes.c_int32, ctypes.c_float, _P, ctypes.c_uint64, _P]),
    ("emelk_attn_decode_append", ctypes.c_uint32,
     [ctypes.POINTER(Geometry), _P, _P, ctypes.c_int32, _P, _P, _P, _P, ctypes.c_int32, _P,
      ctypes.c_int32, _P, ctypes.c_int32, ctypes.c_float, _P, ctypes.c_uint64, _P]),
    ("emelk_attn_decode_contiguous", ctypes.c_uint32,
     [ctypes.POINTER(Geometry), _P, _P, ctypes.c_int32, _P, _P, _P, _P, ctypes.c_int32, _P,
      ctypes.c_int32, ctypes.c_int32, ctypes.c_float, _P, ctypes.c_uint64, _P]),
    ("emelk_attn_decode_noalloc", ctypes.c_uint32,
     [ctypes.POINTER(Geometry), _P, _P, ctypes.c_int32, _P, _P, _P, _P, ctypes.c_int32, _P,
      ctypes.c_int32, _P, ctypes.c_int32, ctypes.c_float, _P]),
    ("emelk_attn_prefill_chunk", ctypes.c_uint32,
     [ctypes.POINTER(Geometry), _P, _P, ctypes.c_int32, _P, _P, ctypes.c_int32, ctypes.c_int32,
      _P, _P, ctypes.c_int32, ctypes.c_float, _P]),
    ("emelk_rope_table_create", ctypes.c_uint32,
     [ctypes.POINTER(RopeParams), ctypes.c_int32, ctypes.c_int32, _P,
      ctypes.POINTER(ctypes.c_void_p)]),
    ("emelk_rope_table_destroy", None, [_P]),
    ("emelk_kv_qkv_rope_append", ctypes.c_uint32,
     [ctypes.POINTER(Geometry), _P, _P, ctypes.c_int32, _P, _P, _P, _P, ctypes.c_int32,
      ctypes.c_int32, _P, _P, ctypes.c_int32, _P, _P, _P, ctypes.c_int32, ctypes.c_float, _P]),
    ("emelk_rope_table_positions", ctypes.c_int32, [_P]),
    ("emelk_kv_sequence_length", ctypes.c_int32, [_P, ctypes.c_int32]),
    ("emelk_batch_decoder_create", ctypes.c_uint32,
     [ctypes.POINTER(Geometry), _P, _P, _P, ctypes.c_int32, ctypes.c_int32, _P,
      ctypes.POINTER(ctypes.c_void_p)]),
    ("emelk_batch_decoder_destroy", None, [_P]),
    ("emelk_batch_decoder_begin_step", ctypes.c_uint32,
     [_P, c_i32p, ctypes.c_int32, ctypes.c_int32, c_i32p]),
    ("emelk_batch_decoder_set_fixed_plan", ctypes.c_uint32, [_P, ctypes.c_int32]),
    ("emelk_batch_decoder_layer", ctypes.c_uint32,
     [_P, ctypes.c_int32, _P, _P, _P, _P, _P, _P, ctypes.c_int32, ctypes.c_float, ctypes.c_float,
      _P]),
    ("emelk_kv_cache_create", ctypes.c_uint32,
     [ctypes.POINTER(Geometry), _P, ctypes.POINTER(ctypes.c_void_p)]),
    ("emelk_kv_cache_destroy", None, [_P]),
    ("emelk_kv_cache_k_pool", _P, [_P]),
    ("emelk_kv_cache_v_pool", _P, [_P]),
    ("emelk_kv_cache_stream", _P, [_P]),
    ("emelk_kv_cache_copy_block", ctypes.c_bool,
     [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, _P, c_i32p]),
    ("emelk_kv_cache_upload_view", ctypes.c_uint32, [_P, _P, _P]),
    ("emelk_batch_plan", ctypes.c_bool,
     [ctypes.POINTER(PlanRequest), ctypes.POINTER(PlanResult), ctypes.POINTER(ctypes.c_uint32)]),
    ("emelk_batch_plan_mode", ctypes.c_bool,
     [ctypes.POINTER(PlanRequest), ctypes.c_int32, ctypes.POINTER(PlanResult),
      ctypes.POINTER(ctypes.c_uint32)]),
    ("emelk_plan_step_sequences", ctypes.c_uint32,
     [ctypes.POINTER(PlanRequest), ctypes.POINTER(PlanResult), ctypes.c_int32, c_i32p, c_i32p,
      c_i32p]),
    ("emelk_build_info", ctypes.c_char_p, []),
]
SYMBOLS = [s[0] for s in _SIGNATURES]

if not os.path.exists(LIB_PATH):
    raise ImportError(f"libemelk.so not built at {LIB_PATH}: run __graft_entry__.build()")
# PyTorch-ROCm wheels ship their own HIP/HSA runtimes.  Loading torch first
# makes libemelk.so's libamdhip64.so.7 / libhsa-runtime64.so.1 dependencies
# resolve (by SONAME) to the runtime torch already holds, so streams and
# device pointers from torch are valid here; loading libemelk.so first would
# put a second HIP runtime in the process.
try:
    import torch  # noqa: F401
except ImportError:  # plain C/C++ or numpy callers: the system ROCm runtime is used
    pass
lib = ctypes.CDLL(LIB_PATH)
for _name, _res, _args in _SIGNATURES:
    _fn = getattr(lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args


def _i32():
    return ctypes.c_int32(0)


class KvActor:
    """Host KV block-map actor (memory::kv::sm), one per cache."""

    def __init__(self):
        self.handle = lib.emelk_kv_actor_create()
        if not self.handle:
            raise MemoryError("emelk_kv_actor_create failed")
        self._keep = []

    def close(self):
        if self.handle and lib is not None:  # lib is None during interpreter teardown
            lib.emelk_kv_actor_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reserve(self, max_sequences=0, max_blocks=0, block_tokens=16, error_out=True):
        err = _i32()
        ev = EvReserve(max_sequences, max_blocks, block_tokens,
                       ctypes.pointer(err) if error_out else None)
        return bool(lib.emelk_kv_reserve(self.handle, ctypes.byref(ev))), err.value

    def allocate_sequence(self, seq_id, error_out=True):
        err = _i32()
        ev = EvAllocateSequence(seq_id, ctypes.pointer(err) if error_out else None)
        return bool(lib.emelk_kv_allocate_sequence(self.handle, ctypes.byref(ev))), err.value

    def allocate_slots(self, seq_id, token_count, copy_block=None, copy_block_user_data=None,
                       block_count_out=True, error_out=True):
        """Returns (accepted, error, block_count).  copy_block: a COPY_BLOCK_FN
        instance or a raw function address (int)."""
        err, cnt = _i32(), _i32()
        cb = None
        if copy_block is not None:
            cb = copy_block if isinstance(copy_block, int) else ctypes.cast(copy_block,
                                                                            ctypes.c_void_p).value
        ev = EvAllocateSlots(seq_id, token_count, ctypes.pointer(cnt) if block_count_out else None,
                             ctypes.pointer(err) if error_out else None, cb, copy_block_user_data)
        ok = bool(lib.emelk_kv_allocate_slots(self.handle, ctypes.byref(ev)))
        return ok, err.value, cnt.value

    def branch_sequence(self, parent_seq_id, child_seq_id):
        err = _i32()
        ev = EvBranchSequence(parent_seq_id, child_seq_id, None, None, ctypes.pointer(err))
        return bool(lib.emelk_kv_branch_sequence(self.handle, ctypes.byref(ev))), err.value

    def free_sequence(self, seq_id):
        err = _i32()
        ev = EvFreeSequence(seq_id, ctypes.pointer(err))
        return bool(lib.emelk_kv_free_sequence(self.handle, ctypes.byref(ev))), err.value

    def rollback_slots(self, seq_id, token_count):
        err, cnt = _i32(), _i32()
        ev = EvRollbackSlots(seq_id, token_count, ctypes.pointer(cnt), ctypes.pointer(err))
        ok = bool(lib.emelk_kv_rollback_slots(self.handle, ctypes.byref(ev)))
        return ok, err.value, cnt.value

    def capture_view(self, snapshot: Optional[Snapshot]):
        err = _i32()
        ev = EvCaptureView(ctypes.pointer(snapshot) if snapshot is not None else None,
                           ctypes.pointer(err))
        return bool(lib.emelk_kv_capture_view(self.handle, ctypes.byref(ev))), err.value

    def view(self) -> Snapshot:
        return lib.emelk_kv_view(self.handle).contents

    def lookup_kv_block(self, seq_id, pos):
        return int(lib.emelk_kv_lookup_kv_block(self.handle, seq_id, pos))

    def evict_blocks(self, seq_id, logical_blocks: Sequence[int]):
        err, removed = _i32(), _i32()
        arr = (ctypes.c_int32 * max(1, len(logical_blocks)))(*logical_blocks)
        ev = EvEvictBlocks(seq_id, arr, len(logical_blocks), ctypes.pointer(removed),
                           ctypes.pointer(err))
        ok = bool(lib.emelk_kv_evict_blocks(self.handle, ctypes.byref(ev)))
        return ok, err.value, removed.value

    def compact(self, max_moves=MAX_BLOCKS):
        """Returns (accepted, error, moves) with moves a list of (src, dst)."""
        err, cnt = _i32(), _i32()
        buf = (ctypes.c_int32 * (2 * max(1, max_moves)))()
        ev = EvCompact(buf, max_moves, ctypes.pointer(cnt), ctypes.pointer(err))
        ok = bool(lib.emelk_kv_compact(self.handle, ctypes.byref(ev)))
        moves = [(buf[2 * i], buf[2 * i + 1]) for i in range(cnt.value)]
        return ok, err.value, moves

    def export_block_tables(self, seq_ids: Sequence[int], stride: int):
        import numpy as np
        out = np.empty((len(seq_ids), stride), dtype=np.uint16)
        ids = (ctypes.c_int32 * max(1, len(seq_ids)))(*seq_ids)
        e = lib.emelk_kv_export_block_tables(
            self.handle, ids, len(seq_ids),
            out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), stride)
        if e != ERR_NONE:
            raise ValueError(f"emelk_kv_export_block_tables error {e}")
        return out

    def set_free_order(self, order):
        import numpy as np
        arr = np.ascontiguousarray(order, dtype=np.uint16)
        e = lib.emelk_kv_set_free_order(self.handle,
                                        arr.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)),
                                        len(arr))
        if e != ERR_NONE:
            raise ValueError(f"emelk_kv_set_free_order error {e}")

    def block_refs(self, block):
        return int(lib.emelk_kv_block_refs(self.handle, block))

    def free_count(self):
        return int(lib.emelk_kv_free_count(self.handle))

    def binding(self) -> KvBinding:
        b = KvBinding()
        lib.emelk_kv_bind(self.handle, ctypes.byref(b))
        return b


# ---- device side (torch tensors as device buffers) -------------------------

def geometry(n_layer, n_head, n_head_kv, head_dim, block_tokens, max_blocks, kv_type=KV_F16):
    return Geometry(n_layer, n_head, n_head_kv, head_dim, block_tokens, max_blocks, kv_type)


def pool_bytes(g: Geometry) -> int:
    out = ctypes.c_uint64(0)
    e = lib.emelk_kv_pool_bytes(ctypes.byref(g), ctypes.byref(out))
    if e != ERR_NONE:
        raise ValueError(f"invalid geometry (error {e})")
    return int(out.value)


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


# Tensor checks run before every device call: a tensor of the wrong dtype,
# device, layout or size would otherwise become an out-of-bounds device read
# or write instead of a Python error.  Objects that only carry data_ptr()
# (DevPtr, library-owned pools) are raw addresses the caller vouches for.
_I16 = ("int16", "uint16")


_DTYPE_NAMES = {}


def _is_tensor(t):
    return hasattr(t, "is_cuda") and hasattr(t, "dtype")


def _need(t, name, dtypes=None, shape=None, min_bytes=None, optional=False):
    if t is None:
        if optional:
            return
        raise ValueError(f"{name}: a device tensor is required")
    if not _is_tensor(t):
        if hasattr(t, "data_ptr"):
            return
        raise TypeError(f"{name}: expected a device tensor, got {type(t).__name__}")
    if not t.is_cuda:
        raise ValueError(f"{name}: tensor must be on the GPU (got device {t.device})")
    if not t.is_contiguous():
        raise ValueError(f"{name}: tensor must be contiguous")
    if dtypes is not None:
        dt = _DTYPE_NAMES.get(t.dtype)
        if dt is None:
            dt = _DTYPE_NAMES[t.dtype] = str(t.dtype).replace("torch.", "")
        if dt not in dtypes:
            raise TypeError(f"{name}: dtype {dt}, expected {' or '.join(dtypes)}")
    if shape is not None:
        got = tuple(int(x) for x in t.shape)
        want = tuple(shape)
        if len(got) != len(want) or any(w is not None and w != x for w, x in zip(want, got)):
            raise ValueError(f"{name}: shape {got}, expected {want} (None = any)")
    if min_bytes is not None and t.numel() * t.element_size() < min_bytes:
        raise ValueError(f"{name}: {t.numel() * t.element_size()} bytes, need {min_bytes}")


_POOL_BYTES = {}


def _pool_bytes_cached(g):
    key = (g.n_layer, g.n_head, g.n_head_kv, g.head_dim, g.block_tokens, g.max_blocks, g.kv_type)
    pb = _POOL_BYTES.get(key)
    if pb is None:
        pb = _POOL_BYTES[key] = pool_bytes(g)
    return pb


def _pools(g, k_pool, v_pool):
    pb = _pool_bytes_cached(g)
    _need(k_pool, "k_pool", min_bytes=pb)
    _need(v_pool, "v_pool", min_bytes=pb)


def _numel(t):
    n = 1
    for x in t.shape:
        n *= int(x)
    return n


def _rows(t, name, n_seq, n_tokens, width):
    """fp32 rows [n_seq][n_tokens][width], given as 3-D or flattened."""
    _need(t, name, ("float32",))
    if _is_tensor(t) and _numel(t) != n_seq * n_tokens * width:
        raise ValueError(f"{name}: {_numel(t)} floats, expected {n_seq}*{n_tokens}*{width}")


def _tables(t, n_seq):
    _need(t, "block_tables", _I16)
    if _is_tensor(t) and (t.dim() != 2 or int(t.shape[0]) < n_seq):
        raise ValueError(f"block_tables: shape {tuple(t.shape)}, expected [>= {n_seq}, stride]")


def _stream(stream):
    if stream is not None:
        return ctypes.c_void_p(stream)
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _check(e, what):
    if e != ERR_NONE:
        raise RuntimeError(f"{what} failed with emel error {e}")


def append(g, k_pool, v_pool, layer, k_rows, v_rows, positions, block_tables, stream=None):
    """k_rows/v_rows: float32 [n_seq, n_tokens, n_head_kv*head_dim] on the device."""
    n_seq, n_tokens = int(k_rows.shape[0]), int(k_rows.shape[1])
    kvd = g.n_head_kv * g.head_dim
    _pools(g, k_pool, v_pool)
    _rows(k_rows, "k_rows", n_seq, n_tokens, kvd)
    _rows(v_rows, "v_rows", n_seq, n_tokens, kvd)
    _need(positions, "positions", ("int32",), (n_seq,))
    _tables(block_tables, n_seq)
    _check(lib.emelk_kv_append(ctypes.byref(g), _ptr(k_pool), _ptr(v_pool), layer, _ptr(k_rows),
                               _ptr(v_rows), n_seq, n_tokens, _ptr(positions), _ptr(block_tables),
                               int(block_tables.shape[1]), _stream(stream)), "emelk_kv_append")


def gather(g, k_pool, v_pool, layer, lengths, block_tables, k_out, v_out, out_tokens,
           stream=None):
    n_seq = int(lengths.shape[0])
    _pools(g, k_pool, v_pool)
    _need(lengths, "lengths", ("int32",), (n_seq,))
    _tables(block_tables, n_seq)
    row = g.n_head_kv * g.head_dim * 2 if g.kv_type == KV_F16 else g.n_head_kv * g.head_dim // 32 * 34
    _need(k_out, "k_out", min_bytes=n_seq * out_tokens * row)
    _need(v_out, "v_out", min_bytes=n_seq * out_tokens * row)
    _check(lib.emelk_kv_gather(ctypes.byref(g), _ptr(k_pool), _ptr(v_pool), layer,
                               int(lengths.shape[0]), _ptr(lengths), _ptr(block_tables),
                               int(block_tables.shape[1]), _ptr(k_out), _ptr(v_out), out_tokens,
                               _stream(stream)), "emelk_kv_gather")


def copy_blocks(g, k_pool, v_pool, moves, stream=None):
    """moves: int32 [n, 2] device tensor of (src, dst) page ids."""
    _pools(g, k_pool, v_pool)
    _need(moves, "moves", ("int32",), (None, 2))
    _check(lib.emelk_kv_copy_blocks(ctypes.byref(g), _ptr(k_pool), _ptr(v_pool), _ptr(moves),
                                    int(moves.shape[0]), _stream(stream)),
           "emelk_kv_copy_blocks")


def decode_workspace_bytes(g, n_seq, max_kv_len) -> int:
    out = ctypes.c_uint64(0)
    _check(lib.emelk_attn_decode_workspace_size(ctypes.byref(g), n_seq, max_kv_len,
                                                ctypes.byref(out)), "workspace_size")
    return int(out.value)


def decode_plan(g, n_seq, max_kv_len):
    """(tokens_per_split, n_splits, workspace_bytes) of one decode call."""
    tps, ns, b = ctypes.c_int32(0), ctypes.c_int32(0), ctypes.c_uint64(0)
    _check(lib.emelk_attn_decode_plan(ctypes.byref(g), n_seq, max_kv_len, ctypes.byref(tps),
                                      ctypes.byref(ns), ctypes.byref(b)), "decode_plan")
    return tps.value, ns.value, int(b.value)


def _decode_args(g, k_pool, v_pool, q, out, kv_lens, block_tables, workspace):
    _pools(g, k_pool, v_pool)
    if not _is_tensor(q):
        raise TypeError("q: expected a device tensor (its first dimension is n_seq)")
    n_seq = int(q.shape[0])
    _rows(q, "q", n_seq, g.n_head, g.head_dim)
    _rows(out, "out", n_seq, g.n_head, g.head_dim)
    _need(kv_lens, "kv_lens", ("int32",), (n_seq,))
    _tables(block_tables, n_seq)
    _need(workspace, "workspace")


def decode(g, k_pool, v_pool, layer, q, out, kv_lens, max_kv_len, block_tables, scale,
           workspace, stream=None):
    _decode_args(g, k_pool, v_pool, q, out, kv_lens, block_tables, workspace)
    _check(lib.emelk_attn_decode(ctypes.byref(g), _ptr(k_pool), _ptr(v_pool), layer, _ptr(q),
                                 _ptr(out), int(q.shape[0]), _ptr(kv_lens), max_kv_len,
                                 _ptr(block_tables), int(block_tables.shape[1]), scale,
                                 _ptr(workspace), workspace.numel() * workspace.element_size(),
                                 _stream(stream)), "emelk_attn_decode")


def decode_append(g, k_pool, v_pool, layer, k_rows, v_rows, q, out, kv_lens, max_kv_len,
                  block_tables, scale, workspace, stream=None):
    """Store the token at position kv_lens - 1 (k_rows/v_rows float32
    [n_seq, n_head_kv*head_dim]) and attend over kv_lens tokens, one launch."""
    _decode_args(g, k_pool, v_pool, q, out, kv_lens, block_tables, workspace)
    n_seq = int(q.shape[0])
    _rows(k_rows, "k_rows", n_seq, 1, g.n_head_kv * g.head_dim)
    _rows(v_rows, "v_rows", n_seq, 1, g.n_head_kv * g.head_dim)
    _check(lib.emelk_attn_decode_append(ctypes.byref(g), _ptr(k_pool), _ptr(v_pool), layer,
                                        _ptr(k_rows), _ptr(v_rows), _ptr(q), _ptr(out),
                                        int(q.shape[0]), _ptr(kv_lens), max_kv_len,
                                        _ptr(block_tables), int(block_tables.shape[1]), scale,
                                        _ptr(workspace),
                                        workspace.numel() * workspace.element_size(),
                                        _stream(stream)), "emelk_attn_decode_append")


def decode_contiguous(g, k_pool, v_pool, layer, q, out, kv_lens, max_kv_len, seq_stride_tokens,
                      scale, workspace, k_rows=None, v_rows=None, stream=None):
    """Decode on contiguous caches (no block table): sequence s holds token t
    at page s * seq_stride_tokens / block_tokens + t / block_tokens.  With
    k_rows/v_rows the token at kv_lens - 1 is stored first."""
    _pools(g, k_pool, v_pool)
    if not _is_tensor(q):
        raise TypeError("q: expected a device tensor (its first dimension is n_seq)")
    n_seq = int(q.shape[0])
    _rows(q, "q", n_seq, g.n_head, g.head_dim)
    _rows(out, "out", n_seq, g.n_head, g.head_dim)
    _need(kv_lens, "kv_lens", ("int32",), (n_seq,))
    _need(workspace, "workspace")
    if (k_rows is None) != (v_rows is None):
        raise ValueError("k_rows and v_rows: both or neither")
    if k_rows is not None:
        _rows(k_rows, "k_rows", n_seq, 1, g.n_head_kv * g.head_dim)
        _rows(v_rows, "v_rows", n_seq, 1, g.n_head_kv * g.head_dim)
    _check(lib.emelk_attn_decode_contiguous(
        ctypes.byref(g), _ptr(k_pool), _ptr(v_pool), layer,
        _ptr(k_rows), _ptr(v_rows), _ptr(q), _ptr(out), n_seq, _ptr(kv_lens),
        max_kv_len, seq_stride_tokens, scale, _ptr(workspace),
        workspace.numel() * workspace.element_size(), _stream(stream)),
        "emelk_attn_decode_contiguous")


def prefill_chunk(g, k_pool, v_pool, layer, q, out, q_start, block_tables, scale, stream=None):
    """q/out: float32 [n_seq, n_q, n_head, head_dim]."""
    _pools(g, k_pool, v_pool)
    if not _is_tensor(q) or q.dim() < 2:
        raise TypeError("q: expected a device tensor [n_seq, n_q, ...]")
    n_seq, n_q = int(q.shape[0]), int(q.shape[1])
    _rows(q, "q", n_seq, n_q, g.n_head * g.head_dim)
    _rows(out, "out", n_seq, n_q, g.n_head * g.head_dim)
    _need(q_start, "q_start", ("int32",), (n_seq,))
    _tables(block_tables, n_seq)
    _check(lib.emelk_attn_prefill_chunk(ctypes.byref(g), _ptr(k_pool), _ptr(v_pool), layer,
                                        _ptr(q), _ptr(out), int(q.shape[0]), int(q.shape[1]),
                                        _ptr(q_start), _ptr(block_tables),
                                        int(block_tables.shape[1]), scale, _stream(stream)),
           "emelk_attn_prefill_chunk")


class RopeTable:
    """Device (cos, sin) table of emelk_rope_table_create."""

    def __init__(self, n_rot, head_dim, max_positions, freq_base, pairing=NORMAL_PAIRING,
                 stream=None):
        self.handle = None
        self.params = RopeParams(n_rot, *pairing, freq_base)
        h = ctypes.c_void_p(None)
        _check(lib.emelk_rope_table_create(ctypes.byref(self.params), head_dim, max_positions,
                                           _stream(stream), ctypes.byref(h)),
               "emelk_rope_table_create")
        self.handle = h

    def close(self):
        if self.handle and lib is not None:  # lib is None during interpreter teardown
            lib.emelk_rope_table_destroy(self.handle)
            self.handle = None

    def __del__(self):
        self.close()


def qkv_rope_append(g, k_pool, v_pool, layer, q_in, q_out, k_rows, v_rows, positions,
                    block_tables, rope: RopeTable, q_norm=None, k_norm=None, v_rms=False,
                    eps=1e-6, stream=None):
    """q_in/q_out: float32 [n_seq, n_tokens, n_head*head_dim]; k_rows/v_rows:
    float32 [n_seq, n_tokens, n_head_kv*head_dim]; all on the device."""
    n_seq, n_tokens = int(k_rows.shape[0]), int(k_rows.shape[1])
    _pools(g, k_pool, v_pool)
    _rows(q_in, "q_in", n_seq, n_tokens, g.n_head * g.head_dim)
    _rows(q_out, "q_out", n_seq, n_tokens, g.n_head * g.head_dim)
    _rows(k_rows, "k_rows", n_seq, n_tokens, g.n_head_kv * g.head_dim)
    _rows(v_rows, "v_rows", n_seq, n_tokens, g.n_head_kv * g.head_dim)
    _need(positions, "positions", ("int32",), (n_seq,))
    _tables(block_tables, n_seq)
    _need(q_norm, "q_norm", ("float32",), (g.head_dim,), optional=True)
    _need(k_norm, "k_norm", ("float32",), (g.head_dim,), optional=True)
    _check(lib.emelk_kv_qkv_rope_append(
        ctypes.byref(g), _ptr(k_pool), _ptr(v_pool), layer, _ptr(q_in), _ptr(q_out),
        _ptr(k_rows), _ptr(v_rows), n_seq, n_tokens, _ptr(positions), _ptr(block_tables),
        int(block_tables.shape[1]), rope.handle, _ptr(q_norm), _ptr(k_norm), int(bool(v_rms)),
        eps, _stream(stream)), "emelk_kv_qkv_rope_append")


class KvCache:
    """Device pools owned by the library (emelk_kv_cache_create)."""

    def __init__(self, g, stream=None):
        self.handle = None
        self.g = g
        h = ctypes.c_void_p(None)
        _check(lib.emelk_kv_cache_create(ctypes.byref(g), _stream(stream), ctypes.byref(h)),
               "emelk_kv_cache_create")
        self.handle = h

    def k_pool_ptr(self):
        return lib.emelk_kv_cache_k_pool(self.handle)

    def v_pool_ptr(self):
        return lib.emelk_kv_cache_v_pool(self.handle)

    def upload_view(self, actor, view_dev):
        """capture_view into the device buffer view_dev (uint8 tensor of at
        least ctypes.sizeof(Snapshot) bytes) on the cache's stream."""
        assert view_dev.numel() * view_dev.element_size() >= ctypes.sizeof(Snapshot)
        _check(lib.emelk_kv_cache_upload_view(self.handle, actor.handle, _ptr(view_dev)),
               "emelk_kv_cache_upload_view")

    @staticmethod
    def view_fields(view_dev, n_seq):
        """(kv_lens, block_tables) of sequences 0..n_seq-1, as tensors over
        the device snapshot (no copy)."""
        lo = Snapshot.sequence_length_values.offset
        bo = Snapshot.sequence_kv_blocks.offset
        lens = view_dev[lo:lo + 4 * n_seq].view(dtype=__import__("torch").int32)
        tables = view_dev[bo:bo + 2 * MAX_BLOCKS_PER_SEQUENCE * n_seq].view(
            dtype=__import__("torch").int16).view(n_seq, MAX_BLOCKS_PER_SEQUENCE)
        return lens, tables

    def close(self):
        if self.handle and lib is not None:  # lib is None during interpreter teardown
            lib.emelk_kv_cache_destroy(self.handle)
            self.handle = None

    def __del__(self):
        self.close()


class BatchDecoder:
    """emelk_batch_decoder: multi-sequence steps over an actor, a cache and a
    rope table (which must outlive it)."""

    def __init__(self, g, actor: "KvActor", cache: KvCache, rope: RopeTable, max_batch,
                 max_kv_len, stream=None):
        self.handle = None  # set only once creation succeeds (close() checks it)
        self._keep = (actor, cache, rope)
        h = ctypes.c_void_p(None)
        _check(lib.emelk_batch_decoder_create(ctypes.byref(g), actor.handle, cache.handle,
                                              rope.handle, max_batch, max_kv_len, _stream(stream),
                                              ctypes.byref(h)), "emelk_batch_decoder_create")
        self.handle = h

    def begin_step(self, seq_ids, n_tokens):
        ids = (ctypes.c_int32 * len(seq_ids))(*seq_ids)
        pos = (ctypes.c_int32 * len(seq_ids))()
        _check(lib.emelk_batch_decoder_begin_step(self.handle, ids, len(seq_ids), n_tokens, pos),
               "emelk_batch_decoder_begin_step")
        return list(pos)

    def set_fixed_plan(self, on=True):
        """Graph-stable launches (emelk_batch_decoder_set_fixed_plan)."""
        _check(lib.emelk_batch_decoder_set_fixed_plan(self.handle, int(bool(on))),
               "emelk_batch_decoder_set_fixed_plan")

    def layer(self, layer, q_in, q_roped, k_rows, v_rows, out, scale, q_norm=None, k_norm=None,
              v_rms=False, eps=1e-6):
        _check(lib.emelk_batch_decoder_layer(self.handle, layer, _ptr(q_in), _ptr(q_roped),
                                             _ptr(k_rows), _ptr(v_rows), _ptr(q_norm),
                                             _ptr(k_norm), int(bool(v_rms)), eps, scale,
                                             _ptr(out)), "emelk_batch_decoder_layer")

    def close(self):
        if self.handle and lib is not None:  # lib is None during interpreter teardown
            lib.emelk_batch_decoder_destroy(self.handle)
            self.handle = None

    def __del__(self):
        self.close()


class DevPtr:
    """A raw device address where the helpers above expect a tensor."""

    def __init__(self, address):
        self.address = int(address)

    def data_ptr(self):
        return self.address


class BatchPlan:
    """The batch planner's process_event (src/emel/batch/planner/sm.hpp:130-136)
    on host arrays: ``BatchPlan(token_ids, n_steps, mode, ...)`` runs it and
    keeps ``accepted``, ``error`` (planner error bits), ``step_sizes``,
    ``steps`` (the token indices of each step), ``total_outputs`` and
    ``offsets``.  ``effective_step_size`` runs one mode's planner directly
    (the mode machines' entry, with the step size given)."""

    def __init__(self, token_ids, n_steps=0, mode=PLAN_SIMPLE, seq_masks=None,
                 seq_primary_ids=None, equal_sequential=True, seq_mask_words=1,
                 output_mask=None, output_all=False, n_tokens=None, effective_step_size=None):
        import numpy as np
        keep = []

        def arr(x, dtype):
            if x is None:
                return None, 0
            a = np.ascontiguousarray(np.asarray(x, dtype=dtype))
            keep.append(a)
            return a.ctypes.data_as(ctypes.POINTER(np.ctypeslib.as_ctypes_type(dtype))), \
                (a.shape[0] if a.ndim else 1)

        tok, ntok = arr(token_ids, np.int32)
        masks, nmask = arr(seq_masks, np.uint64)
        prim, nprim = arr(seq_primary_ids, np.int32)
        outm, nout = arr(output_mask, np.int8)
        if masks is not None and seq_mask_words > 0:
            nmask //= seq_mask_words  # rows of seq_mask_words words
        self.request = PlanRequest(tok, ntok if n_tokens is None else n_tokens, n_steps, mode,
                                   masks, nmask, prim, nprim, int(bool(equal_sequential)),
                                   seq_mask_words, outm, nout, int(bool(output_all)))
        self._keep = keep
        self.result = PlanResult()
        err = ctypes.c_uint32(0)
        if effective_step_size is None:
            self.accepted = lib.emelk_batch_plan(ctypes.byref(self.request),
                                                 ctypes.byref(self.result), ctypes.byref(err))
        else:
            self.accepted = lib.emelk_batch_plan_mode(ctypes.byref(self.request),
                                                      effective_step_size,
                                                      ctypes.byref(self.result), ctypes.byref(err))
        self.error = err.value
        r = self.result
        self.step_count = r.step_count
        self.total_outputs = r.total_outputs
        self.token_indices_count = r.token_indices_count
        self.step_sizes = list(r.step_sizes[:r.step_count])
        self.offsets = list(r.step_token_offsets[:r.step_count + 1]) if r.step_count else []
        idx = list(r.step_token_indices[:r.token_indices_count])
        self.steps = [idx[self.offsets[i]:self.offsets[i + 1]] for i in range(r.step_count)]

    def step_sequences(self, step):
        """(seq_ids, n_tokens) of an equal-shaped step, the arguments of
        emelk_batch_decoder_begin_step; raises if the step is not one."""
        seq = (ctypes.c_int32 * MAX_SEQUENCES)()
        n_seq = ctypes.c_int32(0)
        n_tok = ctypes.c_int32(0)
        _check(lib.emelk_plan_step_sequences(ctypes.byref(self.request), ctypes.byref(self.result),
                                             step, seq, ctypes.byref(n_seq), ctypes.byref(n_tok)),
               "emelk_plan_step_sequences")
        return list(seq[:n_seq.value]), n_tok.value
