"""Writes the golden fixtures of tests/golden/ from the reference's own kernel
header, compiled from /root/reference into oracle/_ref/libemelref.so
(see oracle/Makefile).  Run in the build container only:

    make -C oracle && python tests/golden/gen_golden.py

The fixtures are data (inputs and the reference's outputs); no reference
source is kept.  Cases:
  fp16.npz    exhaustive fp32->fp16 sweep checksum, sampled inputs/outputs,
              all 65536 fp16->fp32 results (quant::fp32_to_fp16/fp16_to_fp32,
              src/emel/kernel/detail.hpp:350-392)
  q8_0.npz    quantize_row_q8_0_strided on the q8_0 workload distribution
              (N(0,1), 1% of values x20), exact .5 ties, an all-zero block
              (src/emel/kernel/detail.hpp:804-824)
  helpers.npz dot_product_f32_f16_scores, dot_product_ggml_f16_scores,
              exp_and_sum_ggml_f32, round_fp16_weight (detail.hpp:2055-2250, 4258)
  flash.npz   the scalar flash route with its f16 accumulator
              (detail.hpp:5238-5291) on the reference bench case
              (tools/bench/kernel/flash_attention_bench.cpp:25-28, 145-176),
              the 32x19 test case (tests/kernel/lifecycle_tests.cpp:941-967)
              and a Qwen3-0.6B-shaped N(0,1) case (4/2 heads, 128 dims,
              513 tokens).
"""
from __future__ import annotations

import ctypes
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.normpath(os.path.join(HERE, "..", "..")))
import oracle  # noqa: E402

_f32p = ctypes.POINTER(ctypes.c_float)
_u16p = ctypes.POINTER(ctypes.c_uint16)


def p(a, t):
    return a.ctypes.data_as(t)


def main():
    ref = oracle.load_ref()
    if ref is None:
        raise SystemExit("oracle/_ref/libemelref.so missing: build it with `make -C oracle`")
    rng = np.random.default_rng(20260101)

    # ---- fp16 ----
    sweep = ref.ref_fp32_to_fp16_sweep(0, 1 << 32)
    specials = np.array([0.0, -0.0, 1.0, 0.5, -0.934325, 0.0345459, -36.4516, 65504.0,
                         65519.99, 65520.0, 6.1035156e-05, -6.1035156e-05, 5.9604645e-08,
                         2.9802322e-08, 2.9802326e-08, 1e-9, np.inf, -np.inf],
                        dtype=np.float32).view(np.uint32)
    rand_bits = rng.integers(0, 1 << 32, size=20000, dtype=np.uint64).astype(np.uint32)
    small = (rng.standard_normal(8000) * 1e-5).astype(np.float32).view(np.uint32)
    bits = np.concatenate([specials, rand_bits, small])
    # keep NaNs out of the sampled set: their payload is the one place where
    # the reference (0x7E00) and the hardware conversion differ.
    f = bits.view(np.float32)
    bits = bits[~np.isnan(f)]
    f16_of = np.array([ref.ref_fp32_to_fp16(float(x)) for x in bits.view(np.float32)],
                      dtype=np.uint16)
    all_h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f32_of_h = np.array([ref.ref_fp16_to_fp32(int(h)) for h in all_h],
                        dtype=np.float32).view(np.uint32)
    np.savez_compressed(os.path.join(HERE, "fp16.npz"), sweep=np.uint64(sweep), in_bits=bits,
                        out_f16=f16_of, f16_to_f32_bits=f32_of_h)

    # ---- q8_0 ----
    assert ref.ref_sizeof_block_q8_0() == 34
    x = rng.standard_normal((64, 1024)).astype(np.float32)
    mask = rng.random(x.shape) < 0.01
    x[mask] *= 20.0
    ties = np.zeros((2, 1024), dtype=np.float32)
    # amax 127 -> d = 1, inv_d = 1: values k + 0.5 are exact halves
    for r in range(2):
        vals = (np.arange(1024) % 200 - 100).astype(np.float32) + (0.5 if r == 0 else -0.5)
        vals = np.clip(vals, -126.5, 126.5)
        vals[::32] = 127.0
        ties[r] = vals
    zero = np.zeros((1, 1024), dtype=np.float32)
    tiny = (rng.standard_normal((1, 1024)) * 1e-6).astype(np.float32)
    xin = np.ascontiguousarray(np.concatenate([x, ties, zero, tiny]))
    out = np.zeros((xin.shape[0], 1024 // 32), dtype=oracle.BLOCK_Q8_0)
    ref.ref_quantize_row_q8_0(p(xin, _f32p), 1, out.ctypes.data, xin.size)
    deq = np.zeros_like(xin)
    ref.ref_dequantize_row_q8_0(out.ctypes.data, p(deq, _f32p), xin.size)
    np.savez_compressed(os.path.join(HERE, "q8_0.npz"), x=xin,
                        blocks=out.view(np.uint8).reshape(xin.shape[0], -1), dequant=deq)

    # ---- helpers ----
    n = 257
    a = rng.standard_normal((16, n)).astype(np.float32)
    b16 = oracle.fp32_to_fp16(rng.standard_normal((16, n)).astype(np.float32))
    bf = rng.standard_normal((16, n)).astype(np.float32)
    dot_f16 = np.array([ref.ref_dot_f32_f16(p(np.ascontiguousarray(a[i]), _f32p),
                                            p(np.ascontiguousarray(b16[i]), _u16p), n)
                        for i in range(16)], dtype=np.float32)
    dot_ff = np.array([ref.ref_dot_f32_f32_f16r(p(np.ascontiguousarray(a[i]), _f32p),
                                                p(np.ascontiguousarray(bf[i]), _f32p), n)
                       for i in range(16)], dtype=np.float32)
    scores = (rng.standard_normal((16, n)) * 3).astype(np.float32)
    scores[:, -20:] = -np.inf
    exps = np.zeros_like(scores)
    sums = np.zeros(16, dtype=np.float64)
    for i in range(16):
        row = np.ascontiguousarray(scores[i])
        e = np.zeros(n, dtype=np.float32)
        sums[i] = ref.ref_exp_and_sum(p(row, _f32p), p(e, _f32p), n, float(row.max()))
        exps[i] = e
    w = rng.random(4096).astype(np.float32)
    rw = np.array([ref.ref_round_fp16_weight(float(v)) for v in w], dtype=np.float32)
    np.savez_compressed(os.path.join(HERE, "helpers.npz"), a=a, b16=b16, bf=bf, dot_f16=dot_f16,
                        dot_ff=dot_ff, scores=scores, exps=exps, sums=sums, w=w, rw=rw)

    # ---- flash (scalar route, f16 accumulator) ----
    cases = {}

    def run_flash(name, q, k16, v16, head_dim, n_head, n_kv, tokens, scale):
        out = np.zeros(n_head * head_dim, dtype=np.float32)
        ok = ref.ref_flash_attn_f16acc(p(q, _f32p), p(k16, _u16p), p(v16, _u16p), head_dim,
                                       n_head, n_kv, tokens, tokens, scale, tokens, p(out, _f32p))
        assert ok, name
        cases[name + "_q"] = q
        cases[name + "_k"] = k16
        cases[name + "_v"] = v16
        cases[name + "_shape"] = np.array([head_dim, n_head, n_kv, tokens], dtype=np.int64)
        cases[name + "_scale"] = np.float32(scale)
        cases[name + "_out"] = out

    # bench case: 64 dims, 12 heads, 12 kv heads, 104 tokens
    D, H, HK, T = 64, 12, 12, 104
    hh, dd = np.meshgrid(np.arange(H), np.arange(D), indexing="ij")
    q = oracle.fp16_to_fp32(oracle.fp32_to_fp16(
        np.sin(((hh + 1) * (dd + 3)).astype(np.float64) * 0.03125).astype(np.float32))).ravel()
    hk, tk, dk = np.meshgrid(np.arange(HK), np.arange(T), np.arange(D), indexing="ij")
    base = ((tk + 1) * (hk + 3) * (dk + 5)).astype(np.float64)
    k16 = oracle.fp32_to_fp16(np.cos(base * 0.0078125).astype(np.float32))
    v16 = oracle.fp32_to_fp16(np.sin(base * 0.01171875).astype(np.float32))
    run_flash("bench", np.ascontiguousarray(q), np.ascontiguousarray(k16),
              np.ascontiguousarray(v16), D, H, HK, T, 1.0 / np.sqrt(D))

    # test case: 32 dims x 19 tokens, scale 0.125, one head
    D, T = 32, 19
    dims = np.arange(D)
    q = ((dims * 7 % 23) - 11).astype(np.float32) * 0.09375
    tt, dd = np.meshgrid(np.arange(T), dims, indexing="ij")
    k = (((tt + 3) * (dd + 5) % 29) - 14).astype(np.float32) * 0.0625
    v = (((tt + 11) * (dd + 7) % 31) - 15).astype(np.float32) * 0.28125
    run_flash("t32x19", np.ascontiguousarray(q), oracle.fp32_to_fp16(k), oracle.fp32_to_fp16(v),
              D, 1, 1, T, 0.125)

    # Qwen3-0.6B-shaped head group (2 q heads per kv head, 128 dims, 513
    # tokens, N(0,1)); two kv heads keep the fixture small.
    D, H, HK, T = 128, 4, 2, 513
    q = rng.standard_normal(H * D).astype(np.float32)
    k16 = oracle.fp32_to_fp16(rng.standard_normal((HK, T, D)).astype(np.float32))
    v16 = oracle.fp32_to_fp16(rng.standard_normal((HK, T, D)).astype(np.float32))
    run_flash("qwen3", q, k16, v16, D, H, HK, T, 1.0 / np.sqrt(D))
    np.savez_compressed(os.path.join(HERE, "flash.npz"), **cases)
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
