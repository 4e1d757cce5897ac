"""Pins the CPU oracle (oracle/oracle.c) against the reference's own outputs
(golden fixtures written from the compiled reference header, see
tests/golden/gen_golden.py), the reference's known-answer tests, and closed
forms.  CPU only."""
import os

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


# ---- fp16 conversion (kernel/detail.hpp:350-392) ----

def test_fp16_exhaustive_sweep_matches_reference_checksum():
    g = load("fp16.npz")
    assert oracle.lib.orc_fp32_to_fp16_sweep(0, 1 << 32) == int(g["sweep"])


def test_fp16_sampled_vectors_match_reference():
    g = load("fp16.npz")
    got = oracle.fp32_to_fp16(g["in_bits"].view(np.float32))
    np.testing.assert_array_equal(got, g["out_f16"])


def test_fp16_to_fp32_all_65536_match_reference():
    g = load("fp16.npz")
    got = oracle.fp16_to_fp32(np.arange(65536, dtype=np.uint32).astype(np.uint16))
    got_bits = got.view(np.uint32)
    ref_bits = g["f16_to_f32_bits"]
    nan = np.isnan(got)
    np.testing.assert_array_equal(got_bits[~nan], ref_bits[~nan])
    assert np.all(np.isnan(ref_bits[nan].view(np.float32)))


def test_fp16_reference_known_answers():
    # tests/text/generator/detail_tests.cpp:1085-1118
    assert oracle.lib.orc_fp16_to_fp32(0x3C00) == 1.0
    assert oracle.lib.orc_fp16_to_fp32(0x3800) == 0.5
    assert np.isinf(oracle.lib.orc_fp16_to_fp32(0x7C00))
    assert oracle.lib.orc_fp16_to_fp32(0x0001) > 0.0
    for x in [0.0, 0.5, -0.934325, 0.0345459, -36.4516, 65504.0, 6.1035156e-05, -6.1035156e-05]:
        # IEEE binary16 RNE == numpy's conversion
        assert oracle.lib.orc_fp32_to_fp16(x) == np.float32(x).astype(np.float16).view(np.uint16)


def test_fp16_matches_ieee_rne_on_random_values():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(200000) * np.exp(rng.uniform(-20, 12, 200000))).astype(np.float32)
    np.testing.assert_array_equal(oracle.fp32_to_fp16(x), x.astype(np.float16).view(np.uint16))


# ---- q8_0 (kernel/detail.hpp:679-690, 804-824) ----

def test_q8_0_quantizer_matches_reference_blocks():
    g = load("q8_0.npz")
    got = oracle.quantize_q8_0(g["x"]).view(np.uint8).reshape(g["blocks"].shape)
    np.testing.assert_array_equal(got, g["blocks"])


def test_q8_0_dequantizer_matches_reference():
    g = load("q8_0.npz")
    blocks = g["blocks"].reshape(-1).view(oracle.BLOCK_Q8_0).reshape(g["x"].shape[0], -1)
    np.testing.assert_array_equal(oracle.dequantize_q8_0(blocks), g["dequant"])


def test_q8_0_reference_known_answer():
    # tests/text/generator/detail_tests.cpp:1309-1324
    blk = np.zeros(1, dtype=oracle.BLOCK_Q8_0)
    blk["d"] = oracle.lib.orc_fp32_to_fp16(0.5)
    blk["qs"][0] = (np.arange(32) % 7) - 3
    out = oracle.dequantize_q8_0(blk)
    assert out[0] == -1.5 and out[1] == -1.0 and out[2] == -0.5 and out[-1] == 0.0


def test_q8_0_closed_forms():
    # all-zero block: d = 0, inv_d = 0, all q = 0
    z = oracle.quantize_q8_0(np.zeros(32, np.float32))
    assert z["d"][0] == 0 and not z["qs"].any()
    # amax maps to +-127; round half away from zero on exact .5 (d = 1)
    x = np.full(32, 3.5, np.float32)
    x[0] = 127.0
    x[1] = -2.5
    b = oracle.quantize_q8_0(x)
    assert b["qs"][0][0] == 127 and b["qs"][0][2] == 4 and b["qs"][0][1] == -3
    assert oracle.lib.orc_fp16_to_fp32(int(b["d"][0])) == 1.0


# ---- attention helpers (kernel/detail.hpp:2055-2250, 4258) ----

def test_dot_and_softmax_helpers_match_reference():
    g = load("helpers.npz")
    import ctypes
    f32p = ctypes.POINTER(ctypes.c_float)
    u16p = ctypes.POINTER(ctypes.c_uint16)
    for i in range(16):
        a = np.ascontiguousarray(g["a"][i])
        b16 = np.ascontiguousarray(g["b16"][i])
        bf = np.ascontiguousarray(g["bf"][i])
        assert np.float32(oracle.lib.orc_dot_f32_f16(a.ctypes.data_as(f32p),
                                                     b16.ctypes.data_as(u16p), a.size)) \
            == g["dot_f16"][i]
        assert np.float32(oracle.lib.orc_dot_f32_f32_f16r(a.ctypes.data_as(f32p),
                                                          bf.ctypes.data_as(f32p), a.size)) \
            == g["dot_ff"][i]
        s = np.ascontiguousarray(g["scores"][i])
        e = np.zeros_like(s)
        tot = oracle.lib.orc_exp_and_sum(s.ctypes.data_as(f32p), e.ctypes.data_as(f32p), s.size,
                                         float(s.max()))
        assert tot == g["sums"][i]
        np.testing.assert_array_equal(e, g["exps"][i])
    rw = np.array([oracle.lib.orc_round_fp16_weight(float(w)) for w in g["w"]], np.float32)
    np.testing.assert_array_equal(rw, g["rw"])


# ---- flash route with f16 accumulator (kernel/detail.hpp:5238-5291) ----

@pytest.mark.parametrize("case", ["bench", "t32x19", "qwen3"])
def test_flash_f16acc_matches_reference_bit_exact(case):
    g = load("flash.npz")
    D, H, HK, T = (int(v) for v in g[case + "_shape"])
    out = oracle.flash_attn_f16acc(g[case + "_q"], g[case + "_k"], g[case + "_v"], D, H, HK, T,
                                   T, float(g[case + "_scale"]))
    np.testing.assert_array_equal(out, g[case + "_out"])


# ---- paged nonflash route (text/generator/detail.hpp:3153-3230) ----

def _paged_cache(rng, n_tokens, n_kv, D, bt, n_blocks):
    """Logical K/V (fp16 bits) scattered into a token-major paged cache through
    a random block table."""
    kv_dim = n_kv * D
    n_lb = -(-n_tokens // bt)
    blocks = rng.permutation(n_blocks)[:n_lb].astype(np.uint16)
    k_log = oracle.fp32_to_fp16(rng.standard_normal((n_tokens, kv_dim)).astype(np.float32))
    v_log = oracle.fp32_to_fp16(rng.standard_normal((n_tokens, kv_dim)).astype(np.float32))
    kc = np.zeros((n_blocks * bt, kv_dim), np.uint16)
    vc = np.zeros_like(kc)
    pos = np.arange(n_tokens)
    phys = blocks[pos // bt].astype(np.int64) * bt + pos % bt
    kc[phys] = k_log
    vc[phys] = v_log
    return blocks, k_log, v_log, kc, vc


def _numpy_attention(q, k, v, n_head, n_kv, D, scale):
    """Brute-force float64 softmax attention (independent of the oracle)."""
    q = q.reshape(n_head, D).astype(np.float64)
    k = k.reshape(-1, n_kv, D).astype(np.float64)
    v = v.reshape(-1, n_kv, D).astype(np.float64)
    rep = n_head // n_kv
    out = np.zeros((n_head, D))
    for h in range(n_head):
        s = k[:, h // rep, :] @ q[h] * scale
        w = np.exp(s - s.max())
        w /= w.sum()
        out[h] = w @ v[:, h // rep, :]
    return out.ravel()


@pytest.mark.parametrize("n_tokens,bt,n_head,n_kv,D", [(37, 4, 4, 2, 64), (300, 16, 8, 2, 64),
                                                        (129, 32, 4, 1, 128)])
def test_compute_attention_close_to_f64_ideal(n_tokens, bt, n_head, n_kv, D):
    rng = np.random.default_rng(n_tokens)
    blocks, k16, v16, kc, vc = _paged_cache(rng, n_tokens, n_kv, D, bt, 64)
    q = rng.standard_normal(n_head * D).astype(np.float32)
    scale = 1.0 / np.sqrt(D)
    got = oracle.compute_attention_f16(q, kc, vc, blocks, bt, n_head, n_kv, D, n_tokens,
                                       n_tokens + 5, scale)
    kf, vf = oracle.fp16_to_fp32(k16), oracle.fp16_to_fp32(v16)
    ideal = _numpy_attention(q, kf, vf, n_head, n_kv, D, scale)
    np.testing.assert_allclose(oracle.attention_f64(q, kf, vf, n_head, n_kv, D, n_tokens, scale),
                               ideal, atol=1e-6, rtol=1e-6)
    # fp16-rounded q and probabilities: within 2e-3 of the ideal
    np.testing.assert_allclose(got, ideal, atol=2e-3, rtol=1e-2)


def test_compute_attention_single_token_returns_v_exactly():
    rng = np.random.default_rng(1)
    blocks, k16, v16, kc, vc = _paged_cache(rng, 1, 2, 64, 4, 8)
    q = rng.standard_normal(4 * 64).astype(np.float32)
    got = oracle.compute_attention_f16(q, kc, vc, blocks, 4, 4, 2, 64, 1, 9, 0.125)
    v = oracle.fp16_to_fp32(v16).reshape(2, 64)
    np.testing.assert_array_equal(got.reshape(4, 64), v[[0, 0, 1, 1]])


def test_compute_attention_uniform_scores_average_v():
    # K = 0 -> every score 0 -> p = 1/n (rounded to fp16) -> mean of V
    rng = np.random.default_rng(2)
    n = 8
    blocks, k16, v16, kc, vc = _paged_cache(rng, n, 1, 64, 4, 8)
    kc[:] = 0
    q = rng.standard_normal(64).astype(np.float32)
    got = oracle.compute_attention_f16(q, kc, vc, blocks, 4, 1, 1, 64, n, n, 0.125)
    v = oracle.fp16_to_fp32(v16).astype(np.float64)
    np.testing.assert_allclose(got, v.mean(axis=0), atol=1e-6)  # 1/8 is exact in fp16


def test_compute_attention_reversed_two_block_map():
    # tests/text/generator/detail_tests.cpp:2460-2560: blocks [1, 0], 4-token
    # blocks: logical p lands at physical p+4 and p+4 at p.
    blocks = np.array([1, 0], np.uint16)
    for p in range(4):
        assert oracle.lib.orc_physical_kv_position(blocks.ctypes.data_as(
            oracle._u16p), 4, p) == p + 4
        assert oracle.lib.orc_physical_kv_position(blocks.ctypes.data_as(
            oracle._u16p), 4, p + 4) == p


def test_compute_attention_q8_0_close_to_ideal_and_single_token():
    rng = np.random.default_rng(5)
    n, bt, H, HK, D = 70, 32, 4, 1, 128
    kv_dim = HK * D
    k = rng.standard_normal((n, kv_dim)).astype(np.float32)
    v = rng.standard_normal((n, kv_dim)).astype(np.float32)
    kq, vq = oracle.quantize_q8_0(k), oracle.quantize_q8_0(v)
    blocks = np.array([3, 0, 5], np.uint16)
    kc = np.zeros((8 * bt, kv_dim // 32), oracle.BLOCK_Q8_0)
    vc = np.zeros_like(kc)
    pos = np.arange(n)
    phys = blocks[pos // bt].astype(np.int64) * bt + pos % bt
    kc[phys], vc[phys] = kq, vq
    q = rng.standard_normal(H * D).astype(np.float32)
    got = oracle.compute_attention_q8_0(q, kc, vc, blocks, bt, H, HK, D, n, n, 1 / np.sqrt(D))
    ideal = _numpy_attention(q, oracle.dequantize_q8_0(kq), oracle.dequantize_q8_0(vq), H, HK, D,
                             1 / np.sqrt(D))
    np.testing.assert_allclose(got, ideal, atol=2e-3, rtol=1e-2)
    one = oracle.compute_attention_q8_0(q, kc, vc, blocks, bt, H, HK, D, 1, n, 1 / np.sqrt(D))
    np.testing.assert_array_equal(
        one.reshape(H, D),
        np.tile(oracle.dequantize_q8_0(vq[0]), (H, 1)))  # p = 1 exactly: out = d*q


def test_flash_f16acc_vs_nonflash_routes_agree_loosely():
    # Both reference routes approximate the same attention; the f16
    # accumulator makes the flash route the lossier one.
    g = load("flash.npz")
    D, H, HK, T = (int(v) for v in g["qwen3_shape"])
    q = g["qwen3_q"]
    flash = oracle.flash_attn_f16acc(q, g["qwen3_k"], g["qwen3_v"], D, H, HK, T, T,
                                     float(g["qwen3_scale"]))
    k = oracle.fp16_to_fp32(g["qwen3_k"]).transpose(1, 0, 2).reshape(T, HK * D)
    v = oracle.fp16_to_fp32(g["qwen3_v"]).transpose(1, 0, 2).reshape(T, HK * D)
    ideal = oracle.attention_f64(q, k, v, H, HK, D, T, float(g["qwen3_scale"]))
    assert np.max(np.abs(flash - ideal)) < 2e-2


def test_decode_batch_threads_equal_per_sequence_route_bit_for_bit():
    """orc_decode_batch_f16 (the bench's full-size checker and CPU baseline)
    is the per-sequence route on worker threads: every thread count gives the
    per-sequence outputs bit for bit, on ragged lengths over one shared
    paged cache."""
    rng = np.random.default_rng(11)
    n_head, n_kv, D, bt, n_blocks, stride = 8, 2, 64, 16, 96, 8
    kv_dim = n_kv * D
    kc = oracle.fp32_to_fp16(rng.standard_normal((n_blocks * bt, kv_dim)).astype(np.float32))
    vc = oracle.fp32_to_fp16(rng.standard_normal((n_blocks * bt, kv_dim)).astype(np.float32))
    n_seq = 7
    tables = np.stack([rng.permutation(n_blocks)[:stride] for _ in range(n_seq)]).astype(np.uint16)
    limits = rng.integers(1, stride * bt + 1, size=n_seq).astype(np.int32)
    limits[0], limits[1] = 1, stride * bt
    q = rng.standard_normal((n_seq, n_head * D)).astype(np.float32)
    n_ctx = stride * bt
    scale = 1.0 / np.sqrt(D)
    want = np.stack([oracle.compute_attention_f16(q[s], kc, vc, tables[s], bt, n_head, n_kv, D,
                                                  int(limits[s]), n_ctx, scale)
                     for s in range(n_seq)])
    for threads in (1, 3, 7, 16):
        got, secs = oracle.decode_batch_f16(q, kc, vc, tables, limits, bt, n_head, n_kv, D, n_ctx,
                                            scale, threads)
        assert secs >= 0.0
        assert got.shape == want.shape
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("kind", ["f16", "q8_0"])
def test_attention_rows_equal_per_row_route_bit_for_bit(kind):
    """orc_attention_rows (the bench's threaded CPU baseline for decode
    batches and chunked-prefill rows) is the per-row route on worker
    threads: any thread count, rows sharing a table row (a prefill chunk's
    rows), and the -march=native build all give the per-row outputs bit for
    bit."""
    rng = np.random.default_rng(12)
    n_head, n_kv, D, bt, n_blocks, stride = 8, 2, 64, 16, 64, 8
    kv_dim = n_kv * D
    rows_k = rng.standard_normal((n_blocks * bt, kv_dim)).astype(np.float32)
    rows_v = rng.standard_normal((n_blocks * bt, kv_dim)).astype(np.float32)
    if kind == "f16":
        kc, vc = oracle.fp32_to_fp16(rows_k), oracle.fp32_to_fp16(rows_v)
        route = oracle.compute_attention_f16
    else:
        kc, vc = oracle.quantize_q8_0(rows_k), oracle.quantize_q8_0(rows_v)
        route = oracle.compute_attention_q8_0
    tables = np.stack([rng.permutation(n_blocks)[:stride] for _ in range(3)]).astype(np.uint16)
    n_rows = 9
    row_table = np.array([0, 0, 0, 1, 1, 2, 2, 2, 2], np.int32)
    limits = rng.integers(1, stride * bt + 1, size=n_rows).astype(np.int32)
    q = rng.standard_normal((n_rows, n_head * D)).astype(np.float32)
    scale = 1.0 / np.sqrt(D)
    want = np.stack([route(q[i], kc, vc, tables[row_table[i]], bt, n_head, n_kv, D,
                           int(limits[i]), int(limits[i]), scale) for i in range(n_rows)])
    native, _note = oracle.native_lib()
    for threads, lib_ in ((1, None), (4, None), (16, None), (5, native)):
        got, secs = oracle.attention_rows(kind, q, kc, vc, tables, limits, bt, n_head, n_kv, D,
                                          scale, threads, row_table=row_table, lib_=lib_)
        assert secs >= 0.0
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
