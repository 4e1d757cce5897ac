"""Pins the oracle's restatement of the step before append (RoPE and the
RMS norms, text/generator/detail.hpp:1060-1111, 2905-2936) against
mathematics that does not retype the oracle's formula: identities, norm
preservation, a float64 rotation, which dims each pairing touches, and the
input vector of the reference test detail_tests.cpp:1120-1133."""
import ctypes
import ctypes.util
import math

import numpy as np
import pytest

import oracle

F32_ULP = np.finfo(np.float32).eps

# the C library's powf, which apply_rope_pairing calls for theta_scale
_libm = ctypes.CDLL(ctypes.util.find_library("m"))
_libm.powf.restype = ctypes.c_float
_libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]


def rotation_f64(vec, pairs, position, rot_dim, freq_base):
    """float64 rotation with the float32 theta recurrence of the reference."""
    out = np.array(vec, dtype=np.float64)
    scale = np.float32(_libm.powf(freq_base, float(np.float32(-2.0) / np.float32(rot_dim))))
    theta = np.float32(position)
    for d0, d1 in pairs:
        c, s = math.cos(float(theta)), math.sin(float(theta))
        x0, x1 = out[d0], out[d1]
        out[d0] = x0 * c - x1 * s
        out[d1] = x0 * s + x1 * c
        theta = np.float32(theta * scale)
    return out


def pairs_of(pairing, rot_dim):
    x0s, x1s, x1o, x1h = pairing
    pc = rot_dim // 2
    base = x1o + x1h * pc
    return [(p * x0s, p * x1s + base) for p in range(pc)]


@pytest.mark.parametrize("pairing", [oracle.NORMAL_PAIRING, oracle.NEOX_PAIRING])
def test_rope_position_zero_is_identity(pairing):
    x = np.random.default_rng(1).standard_normal(4 * 128).astype(np.float32)
    y = oracle.rope_pairing(x, pairing, 4, 128, 128, 0, 10000.0)
    assert np.array_equal(x, y)


@pytest.mark.parametrize("pairing", [oracle.NORMAL_PAIRING, oracle.NEOX_PAIRING])
@pytest.mark.parametrize("position", [1, 103, 4097, 131071])
def test_rope_matches_float64_rotation(pairing, position):
    x = np.random.default_rng(position).standard_normal(128).astype(np.float32) * 3
    y = oracle.rope_pairing(x, pairing, 1, 128, 128, position, 500000.0)
    want = rotation_f64(x, pairs_of(pairing, 128), position, 128, 500000.0)
    # two float32 products and a sum, each rounded once, of |x| ~ 3
    np.testing.assert_allclose(y, want, rtol=0, atol=8 * F32_ULP * 8)
    # every pair keeps its length
    for d0, d1 in pairs_of(pairing, 128):
        r0 = math.hypot(x[d0], x[d1])
        r1 = math.hypot(y[d0], y[d1])
        assert abs(r0 - r1) <= 8 * F32_ULP * (r0 + 1)


def test_rope_reference_test_vector():
    # detail_tests.cpp:1120-1133: sin(idx/32)*3, apply_rope(., 1, 64, 64, 103, 10000)
    x = (np.sin(np.arange(64, dtype=np.float32) * np.float32(0.03125)) * 3).astype(np.float32)
    y = oracle.rope_pairing(x, oracle.NORMAL_PAIRING, 1, 64, 64, 103, 10000.0)
    want = rotation_f64(x, [(2 * p, 2 * p + 1) for p in range(32)], 103, 64, 10000.0)
    np.testing.assert_allclose(y, want, rtol=0, atol=1e-5)
    assert not np.array_equal(x, y)


@pytest.mark.parametrize("pairing,touched", [
    (oracle.NORMAL_PAIRING, set(range(64))),               # (2p, 2p+1), p < 32
    (oracle.NEOX_PAIRING, set(range(32)) | set(range(32, 64))),  # (p, p+32)
])
def test_rope_partial_rotation_touches_only_rot_dims(pairing, touched):
    x = np.random.default_rng(5).standard_normal(128).astype(np.float32)
    y = oracle.rope_pairing(x, pairing, 1, 128, 64, 77, 10000.0)
    changed = set(np.nonzero(x != y)[0].tolist())
    assert changed <= touched
    assert np.array_equal(x[64:], y[64:])
    # the neox pairs are (p, p + rot_dim/2), not (p, p + head_dim/2)
    want = rotation_f64(x, pairs_of(pairing, 64), 77, 64, 10000.0)
    np.testing.assert_allclose(y, want, rtol=0, atol=1e-5)


def test_rope_degenerate_shapes_are_noops():
    x = np.random.default_rng(2).standard_normal(64).astype(np.float32)
    assert np.array_equal(oracle.rope_pairing(x, oracle.NORMAL_PAIRING, 1, 64, 1, 9, 1e4), x)
    assert np.array_equal(oracle.rope_pairing(x, oracle.NORMAL_PAIRING, 0, 64, 64, 9, 1e4), x)


def test_headwise_rms_norm_closed_forms():
    rng = np.random.default_rng(3)
    x = rng.standard_normal(4 * 128).astype(np.float32)
    w = rng.standard_normal(128).astype(np.float32)
    eps = 1e-6
    y = oracle.headwise_rms_norm(x, w, 4, 128, eps)
    xh = x.reshape(4, 128).astype(np.float64)
    want = xh / np.sqrt((xh * xh).mean(axis=1, keepdims=True) + eps) * w.astype(np.float64)
    np.testing.assert_allclose(y.reshape(4, 128), want, rtol=2e-6, atol=1e-6)
    # constant head, unit weights: every value becomes c / sqrt(c^2 + eps)
    c = np.full(128, 2.5, dtype=np.float32)
    y = oracle.headwise_rms_norm(c, np.ones(128, np.float32), 1, 128, 0.0)
    assert np.all(np.abs(y - 1.0) <= 2 * F32_ULP)


def test_rms_norm_in_place_closed_form():
    x = np.random.default_rng(4).standard_normal(1024).astype(np.float32) * 7
    y = oracle.rms_norm_in_place(x, 1e-5)
    xd = x.astype(np.float64)
    want = xd / np.sqrt((xd * xd).mean() + 1e-5)
    np.testing.assert_allclose(y, want, rtol=2e-6, atol=1e-6)
    assert abs(float(np.sqrt(np.mean(y.astype(np.float64) ** 2))) - 1.0) < 1e-5


def test_qkv_rope_rows_order():
    """Norm first, then RoPE (compute_layer_attention_residual order)."""
    rng = np.random.default_rng(6)
    q = rng.standard_normal(2 * 64).astype(np.float32)
    k = rng.standard_normal(64).astype(np.float32)
    v = rng.standard_normal(64).astype(np.float32)
    w = rng.standard_normal(64).astype(np.float32)
    qo, ko, vo = oracle.qkv_rope_rows(q, k, v, 2, 1, 64, oracle.NEOX_PAIRING, 64, 1e6, 11,
                                      q_norm=w, k_norm=w, v_rms=True, eps=1e-6)
    qn = oracle.headwise_rms_norm(q, w, 2, 64, 1e-6)
    assert np.array_equal(qo, oracle.rope_pairing(qn, oracle.NEOX_PAIRING, 2, 64, 64, 11, 1e6))
    kn = oracle.headwise_rms_norm(k, w, 1, 64, 1e-6)
    assert np.array_equal(ko, oracle.rope_pairing(kn, oracle.NEOX_PAIRING, 1, 64, 64, 11, 1e6))
    assert np.array_equal(vo, oracle.rms_norm_in_place(v, 1e-6))
