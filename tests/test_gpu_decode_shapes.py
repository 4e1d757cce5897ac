"""Seeded sweep of decode shapes against the oracle's reference route (2e-3
abs + 1e-2 rel) and the fp64 ideal (the same bar; q8_0 pools, which carry
outliers, also allow the reference's fp16 rounding of the probabilities
there): head_dim 64/128/256, 1-8 query heads per
KV head, 1-8 KV heads, page sizes that do and do not hold a whole wave tile,
f16 and q8_0 pools, 1-70 ragged sequences, and pools whose never-written
bytes are NaN patterns.  It covers the decode kernel's routes together: the
MFMA route (scores and P.V on 4x4x4 blocks), the q8_0 MFMA-score route,
the scalar route, the fixed and the balanced split plans, and one split per
sequence."""
import numpy as np
import pytest

import emelk
import oracle
from kvsetup import Scenario, assert_close

pytestmark = pytest.mark.gpu


def _cases(n=24, seed=2024):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n:
        D = int(rng.choice([64, 128, 256]))
        n_kv = int(rng.choice([1, 2, 4, 8]))
        group = int(rng.choice([1, 2, 4, 8]))
        bt = int(rng.choice([8, 12, 16, 32]))
        kv_type = emelk.KV_F16 if rng.random() < 0.5 else emelk.KV_Q8_0
        if kv_type == emelk.KV_Q8_0 and (bt * D) % 256 != 0:
            continue
        n_seq = int(rng.choice([1, 2, 5, 16, 40, 70]))
        max_len = int(rng.choice([40, 300, 1500, 3000]))
        budget = 48000 // max(1, n_kv)  # keeps the oracle within seconds
        lens = [int(x) for x in rng.integers(1, max_len + 1, size=n_seq)]
        while sum(lens) > budget:
            lens = [max(1, x // 2) for x in lens]
        pool_byte = 0xFF if rng.random() < 0.3 else 0
        cases.append((D, n_kv, group, bt, kv_type, lens, pool_byte, int(rng.integers(1 << 30))))
    return cases


CASES = _cases()


@pytest.mark.parametrize("case", CASES, ids=[f"shape{i}" for i in range(len(CASES))])
def test_decode_shape_sweep(device, case):
    D, n_kv, group, bt, kv_type, lens, pool_byte, seed = case
    print(f"\n[gpu-case] decode sweep D={D} n_kv={n_kv} G={group} bt={bt} type={kv_type} "
          f"n_seq={len(lens)} max_len={max(lens)} pool_byte={pool_byte:#x}", flush=True)
    sc = Scenario(n_layer=1, n_head=n_kv * group, n_kv=n_kv, head_dim=D, block_tokens=bt, lens=lens,
                  seed=seed, kv_type=kv_type, pool_byte=pool_byte,
                  outlier_frac=0.01 if kv_type == emelk.KV_Q8_0 else 0.0)
    q = np.random.default_rng(seed + 1).standard_normal((sc.n_seq, sc.n_head * D)).astype(np.float32)
    got = sc.gpu_decode(0, q)
    if kv_type == emelk.KV_F16:
        assert_close(got, sc.oracle_decode(0, q), what="gpu vs reference route")
        assert_close(got, sc.ideal_decode(0, q), what="gpu vs fp64 ideal")
        return
    # Against the reference route: the plain bar.  Against the fp64 ideal,
    # q8_0 pools (x20 outliers) also allow 2^-10 of sum_p p |v| per output:
    # the reference route's own fp16 rounding of P (2^-11 relative per
    # weight) moves it that far from the ideal when outliers make sum_p p |v|
    # much larger than a cancelling output.
    assert_close(got, sc.oracle_decode(0, q), what="gpu vs reference route")
    scale = 1.0 / np.sqrt(D)
    qr = oracle.fp16_to_fp32(oracle.fp32_to_fp16(q))
    mag = np.zeros_like(got)
    for s_, n in enumerate(sc.lens):
        k = oracle.dequantize_q8_0(oracle.quantize_q8_0(sc.k_rows[0][s_]))
        v = oracle.dequantize_q8_0(oracle.quantize_q8_0(sc.v_rows[0][s_]))
        mag[s_] = oracle.attention_f64(qr[s_], k, np.abs(v), sc.n_head, n_kv, D, n, scale)
    assert_close(got, sc.ideal_decode(0, q), atol=2e-3 + 2.0 ** -10 * mag,
                 what="gpu vs fp64 ideal")


F16_OUTLIER_CASES = [c for c in _cases(n=40, seed=77) if c[4] == emelk.KV_F16][:6]


@pytest.mark.parametrize("case", F16_OUTLIER_CASES,
                         ids=[f"f16_outliers{i}" for i in range(len(F16_OUTLIER_CASES))])
def test_decode_f16_with_outliers_strict_bar(device, case):
    # f16 pools with 1% of K/V values scaled x20, the q8_0 cases' data: the
    # fp16 rounding of P that both routes do then weighs most, and the GPU
    # must still stay within the plain bar of the reference route.
    D, n_kv, group, bt, kv_type, lens, pool_byte, seed = case
    print(f"\n[gpu-case] f16 outlier decode D={D} n_kv={n_kv} G={group} bt={bt} "
          f"n_seq={len(lens)} max_len={max(lens)}", flush=True)
    sc = Scenario(n_layer=1, n_head=n_kv * group, n_kv=n_kv, head_dim=D, block_tokens=bt, lens=lens,
                  seed=seed, kv_type=kv_type, pool_byte=pool_byte, outlier_frac=0.01)
    q = np.random.default_rng(seed + 1).standard_normal((sc.n_seq, sc.n_head * D)).astype(np.float32)
    got = sc.gpu_decode(0, q)
    assert_close(got, sc.oracle_decode(0, q), what="gpu vs reference route")
