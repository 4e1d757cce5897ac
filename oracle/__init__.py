"""TEST INFRASTRUCTURE — numpy/ctypes front end of the CPU oracle.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, as the checker (or the timed CPU baseline).  The product path
(emel.cpp_amd/) never does.  See oracle.c for what each function restates and
how it is pinned.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")
REF_LIB_PATH = os.path.join(_HERE, "_ref", "libemelref.so")

BLOCK_Q8_0 = np.dtype([("d", "<u2"), ("qs", "i1", (32,))], align=False)
assert BLOCK_Q8_0.itemsize == 34

_f32p = ctypes.POINTER(ctypes.c_float)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_i32p = ctypes.POINTER(ctypes.c_int32)
_vp = ctypes.c_void_p

_SIGNATURES = [
    ("orc_fp32_to_fp16", ctypes.c_uint16, [ctypes.c_float]),
    ("orc_fp16_to_fp32", ctypes.c_float, [ctypes.c_uint16]),
    ("orc_fp32_to_fp16_sweep", ctypes.c_uint64, [ctypes.c_uint64, ctypes.c_uint64]),
    ("orc_fp32_to_fp16_row", None, [_f32p, _u16p, ctypes.c_int64]),
    ("orc_fp16_to_fp32_row", None, [_u16p, _f32p, ctypes.c_int64]),
    ("orc_quantize_row_q8_0", None, [_f32p, ctypes.c_uint64, _vp, ctypes.c_int64]),
    ("orc_dequantize_row_q8_0", None, [_vp, _f32p, ctypes.c_int64]),
    ("orc_dot_f32_f16", ctypes.c_float, [_f32p, _u16p, ctypes.c_int64]),
    ("orc_dot_f32_f32_f16r", ctypes.c_float, [_f32p, _f32p, ctypes.c_int64]),
    ("orc_exp_and_sum", ctypes.c_double, [_f32p, _f32p, ctypes.c_int64, ctypes.c_float]),
    ("orc_round_fp16_weight", ctypes.c_float, [ctypes.c_float]),
    ("orc_physical_kv_position", ctypes.c_int64, [_u16p, ctypes.c_int32, ctypes.c_int32]),
    ("orc_compute_attention_f16", ctypes.c_int,
     [_f32p, _u16p, _u16p, _u16p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
      ctypes.c_int32, ctypes.c_int32, ctypes.c_float, _f32p, _f32p]),
    ("orc_compute_attention_q8_0", ctypes.c_int,
     [_f32p, _vp, _vp, _u16p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
      ctypes.c_int32, ctypes.c_int32, ctypes.c_float, _f32p, _f32p]),
    ("orc_flash_attn_f16acc", ctypes.c_int,
     [_f32p, _u16p, _u16p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
      ctypes.c_int64, ctypes.c_float, _f32p]),
    ("orc_attention_f64", None,
     [_f32p, _f32p, _f32p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
      ctypes.c_double, _f32p]),
    ("orc_rope_pairing", None,
     [_f32p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
      ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_float]),
    ("orc_headwise_rms_norm", ctypes.c_int,
     [_f32p, _f32p, ctypes.c_int32, ctypes.c_int32, ctypes.c_float]),
    ("orc_rms_norm_in_place", ctypes.c_int, [_f32p, ctypes.c_int64, ctypes.c_float]),
    ("orc_decode_batch_f16", ctypes.c_double,
     [_f32p, _u16p, _u16p, _u16p, ctypes.c_int32, _i32p, ctypes.c_int32, ctypes.c_int32,
      ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_float, _f32p,
      ctypes.c_int32]),
    ("orc_attention_rows", ctypes.c_double,
     [ctypes.c_int32, _f32p, _vp, _vp, _u16p, ctypes.c_int32, _i32p, _i32p, ctypes.c_int32,
      ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
      ctypes.c_float, _f32p, ctypes.c_int32]),
]


def _load(path):
    lib_ = ctypes.CDLL(path)
    for name, res, args in _SIGNATURES:
        fn = getattr(lib_, name)
        fn.restype = res
        fn.argtypes = args
    return lib_


lib = _load(LIB_PATH)
_native = None


def native_lib():
    """The oracle built -O3 -march=native on this host (the CPU baseline's
    build), compiled on first use by `make native`; (lib, build note).
    Falls back to the portable build, saying so, when the compiler fails."""
    global _native
    if _native is None:
        import subprocess
        try:
            subprocess.run(["make", "-s", "-C", _HERE, "native"], check=True,
                           capture_output=True, timeout=120)
            _native = (_load(os.path.join(_HERE, "_native", "liboracle.so")),
                       "gcc -O3 -march=native -ffp-contract=off, built on this host")
        except Exception as e:  # noqa: BLE001 - reported on the baseline line
            _native = (lib, f"portable -O3 build (native build failed: {e!r})")
    return _native




def _p(a, t):
    return a.ctypes.data_as(t)


def fp32_to_fp16(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib.orc_fp32_to_fp16_row(_p(x, _f32p), _p(out, _u16p), x.size)
    return out


def fp16_to_fp32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib.orc_fp16_to_fp32_row(_p(h, _u16p), _p(out, _f32p), h.size)
    return out


def quantize_q8_0(x) -> np.ndarray:
    """x: float32 [..., k] with k % 32 == 0 -> structured BLOCK_Q8_0 [..., k/32]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    k = x.shape[-1]
    out = np.zeros(x.shape[:-1] + (k // 32,), dtype=BLOCK_Q8_0)
    lib.orc_quantize_row_q8_0(_p(x, _f32p), 1, out.ctypes.data, x.size)
    return out


def dequantize_q8_0(blocks) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=BLOCK_Q8_0)
    out = np.empty(blocks.shape[:-1] + (blocks.shape[-1] * 32,), dtype=np.float32)
    lib.orc_dequantize_row_q8_0(blocks.ctypes.data, _p(out, _f32p), out.size)
    return out


def compute_attention_f16(q, key_cache, value_cache, blocks, block_tokens, n_head, n_head_kv,
                          head_dim, position_limit, n_ctx, inv_scale):
    """Reference nonflash route for one (sequence, layer).  key/value_cache:
    uint16 token-major [positions, n_head_kv*head_dim]; q float32 [n_head*head_dim]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    blocks = np.ascontiguousarray(blocks, dtype=np.uint16)
    out = np.zeros(n_head * head_dim, dtype=np.float32)
    scratch = np.zeros(4 * n_ctx, dtype=np.float32)
    ok = lib.orc_compute_attention_f16(_p(q, _f32p), _p(key_cache, _u16p), _p(value_cache, _u16p),
                                       _p(blocks, _u16p), block_tokens, n_head, n_head_kv,
                                       head_dim, position_limit, n_ctx, inv_scale,
                                       _p(out, _f32p), _p(scratch, _f32p))
    if not ok:
        raise ValueError("orc_compute_attention_f16 rejected its inputs")
    return out


def compute_attention_q8_0(q, key_cache, value_cache, blocks, block_tokens, n_head, n_head_kv,
                           head_dim, position_limit, n_ctx, inv_scale):
    """As compute_attention_f16 over BLOCK_Q8_0 caches [positions, kv_dim/32]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    blocks = np.ascontiguousarray(blocks, dtype=np.uint16)
    out = np.zeros(n_head * head_dim, dtype=np.float32)
    scratch = np.zeros(4 * n_ctx, dtype=np.float32)
    ok = lib.orc_compute_attention_q8_0(_p(q, _f32p), key_cache.ctypes.data,
                                        value_cache.ctypes.data, _p(blocks, _u16p), block_tokens,
                                        n_head, n_head_kv, head_dim, position_limit, n_ctx,
                                        inv_scale, _p(out, _f32p), _p(scratch, _f32p))
    if not ok:
        raise ValueError("orc_compute_attention_q8_0 rejected its inputs")
    return out


def flash_attn_f16acc(q, k_headmajor, v_headmajor, head_dim, n_head, n_head_kv, kv_tokens,
                      kv_stride_tokens, scale, lib_=None):
    lib_ = lib if lib_ is None else lib_
    q = np.ascontiguousarray(q, dtype=np.float32)
    out = np.zeros(n_head * head_dim, dtype=np.float32)
    ok = lib_.orc_flash_attn_f16acc(_p(q, _f32p), _p(k_headmajor, _u16p), _p(v_headmajor, _u16p),
                                   head_dim, n_head, n_head_kv, kv_tokens, kv_stride_tokens,
                                   scale, _p(out, _f32p))
    if not ok:
        raise ValueError("orc_flash_attn_f16acc rejected its inputs")
    return out


def attention_f64(q, k, v, n_head, n_head_kv, head_dim, kv_tokens, inv_scale):
    """k/v float32 token-major logical [kv_tokens, n_head_kv*head_dim]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.zeros(n_head * head_dim, dtype=np.float32)
    lib.orc_attention_f64(_p(q, _f32p), _p(k, _f32p), _p(v, _f32p), n_head, n_head_kv, head_dim,
                          kv_tokens, inv_scale, _p(out, _f32p))
    return out


def decode_batch_f16(q, key_cache, value_cache, block_tables, position_limits, block_tokens,
                     n_head, n_head_kv, head_dim, n_ctx, inv_scale, n_threads, lib_=None):
    """Threaded reference route over a batch; returns (out, seconds)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    block_tables = np.ascontiguousarray(block_tables, dtype=np.uint16)
    limits = np.ascontiguousarray(position_limits, dtype=np.int32)
    n_seq = q.shape[0]
    out = np.zeros((n_seq, n_head * head_dim), dtype=np.float32)
    lib_ = lib if lib_ is None else lib_
    secs = lib_.orc_decode_batch_f16(_p(q, _f32p), _p(key_cache, _u16p), _p(value_cache, _u16p),
                                    _p(block_tables, _u16p), block_tables.shape[1],
                                    _p(limits, _i32p), n_seq, block_tokens, n_head, n_head_kv,
                                    head_dim, n_ctx, inv_scale, _p(out, _f32p), n_threads)
    return out, float(secs)


def attention_rows(kind, q, key_cache, value_cache, block_tables, limits, block_tokens, n_head,
                   n_head_kv, head_dim, inv_scale, n_threads, row_table=None, n_ctx=0,
                   lib_=None):
    """Threaded reference route over rows (orc_attention_rows): kind "f16" or
    "q8_0"; row i uses table row row_table[i] (i when None) and attends to
    [0, limits[i]).  Returns (out [n_rows, n_head*head_dim], seconds)."""
    lib_ = lib if lib_ is None else lib_
    q = np.ascontiguousarray(q, dtype=np.float32).reshape(len(limits), -1)
    block_tables = np.ascontiguousarray(block_tables, dtype=np.uint16)
    limits = np.ascontiguousarray(limits, dtype=np.int32)
    rt = None if row_table is None else np.ascontiguousarray(row_table, dtype=np.int32)
    out = np.zeros((len(limits), n_head * head_dim), dtype=np.float32)
    secs = lib_.orc_attention_rows(0 if kind == "f16" else 1, _p(q, _f32p),
                                   key_cache.ctypes.data_as(_vp), value_cache.ctypes.data_as(_vp),
                                   _p(block_tables, _u16p), block_tables.shape[1],
                                   None if rt is None else _p(rt, _i32p), _p(limits, _i32p),
                                   len(limits), block_tokens, n_head, n_head_kv, head_dim, n_ctx,
                                   inv_scale, _p(out, _f32p), n_threads)
    return out, float(secs)


NORMAL_PAIRING = (2, 2, 1, 0)  # rope_pairing defaults, text/generator/detail.hpp:39-46
NEOX_PAIRING = (1, 1, 0, 1)    # neox_rope_pairing, detail.hpp:48-50


def rope_pairing(vec, pairing, head_count, head_dim, n_rot, position, freq_base):
    """apply_rope_pairing on a copy of vec (head_count*head_dim floats)."""
    out = np.array(vec, dtype=np.float32, copy=True).ravel()
    lib.orc_rope_pairing(_p(out, _f32p), *pairing, head_count, head_dim, n_rot, position,
                         freq_base)
    return out


def headwise_rms_norm(vec, weights, head_count, head_dim, eps):
    out = np.array(vec, dtype=np.float32, copy=True).ravel()
    w = np.ascontiguousarray(weights, dtype=np.float32)
    assert lib.orc_headwise_rms_norm(_p(out, _f32p), _p(w, _f32p), head_count, head_dim, eps)
    return out


def rms_norm_in_place(vec, eps):
    out = np.array(vec, dtype=np.float32, copy=True).ravel()
    assert lib.orc_rms_norm_in_place(_p(out, _f32p), out.size, eps)
    return out


def qkv_rope_rows(q, k, v, n_head, n_head_kv, head_dim, pairing, n_rot, freq_base, position,
                  q_norm=None, k_norm=None, v_rms=False, eps=1e-6):
    """The reference's per-token steps between the projections and the KV
    store (compute_layer_attention_residual, detail.hpp:3806-3825): returns
    (q, k, v) fp32 rows after the optional norms and RoPE."""
    q = np.array(q, dtype=np.float32, copy=True).ravel()
    k = np.array(k, dtype=np.float32, copy=True).ravel()
    v = np.array(v, dtype=np.float32, copy=True).ravel()
    if q_norm is not None:
        q = headwise_rms_norm(q, q_norm, n_head, head_dim, eps)
    if k_norm is not None:
        k = headwise_rms_norm(k, k_norm, n_head_kv, head_dim, eps)
    if v_rms:
        v = rms_norm_in_place(v, eps)
    q = rope_pairing(q, pairing, n_head, head_dim, n_rot, position, freq_base)
    k = rope_pairing(k, pairing, n_head_kv, head_dim, n_rot, position, freq_base)
    return q, k, v


def load_ref():
    """The reference's own kernel header compiled here (None when absent)."""
    if not os.path.exists(REF_LIB_PATH):
        return None
    r = ctypes.CDLL(REF_LIB_PATH)
    for name, res, args in [
        ("ref_fp32_to_fp16", ctypes.c_uint16, [ctypes.c_float]),
        ("ref_fp16_to_fp32", ctypes.c_float, [ctypes.c_uint16]),
        ("ref_fp32_to_fp16_sweep", ctypes.c_uint64, [ctypes.c_uint64, ctypes.c_uint64]),
        ("ref_quantize_row_q8_0", None, [_f32p, ctypes.c_uint64, _vp, ctypes.c_int64]),
        ("ref_dequantize_row_q8_0", None, [_vp, _f32p, ctypes.c_int64]),
        ("ref_sizeof_block_q8_0", ctypes.c_uint64, []),
        ("ref_dot_f32_f16", ctypes.c_float, [_f32p, _u16p, ctypes.c_uint64]),
        ("ref_dot_f32_f32_f16r", ctypes.c_float, [_f32p, _f32p, ctypes.c_uint64]),
        ("ref_exp_and_sum", ctypes.c_double, [_f32p, _f32p, ctypes.c_uint64, ctypes.c_float]),
        ("ref_round_fp16_weight", ctypes.c_float, [ctypes.c_float]),
        ("ref_flash_attn_f16acc", ctypes.c_int,
         [_f32p, _u16p, _u16p, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64,
          ctypes.c_uint64, ctypes.c_float, ctypes.c_uint32, _f32p]),
    ]:
        fn = getattr(r, name)
        fn.restype = res
        fn.argtypes = args
    return r
