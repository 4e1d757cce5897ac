"""Seeded sweep of chunked-prefill shapes against the oracle's per-row
reference route (text/generator/detail.hpp:4297-4372: row r of a chunk that
starts at q_start attends causally to positions [0, q_start + r]) and the
fp64 ideal, at the 2e-3 abs + 1e-2 rel bar.  It covers head_dim 64/128/256/
512, 1-8 query heads per KV head, pages of 8-64 tokens (whole 32-key
sub-tiles per page and not), f16 and q8_0 pools, empty and ragged prefixes,
chunks of 1-100 rows, and NaN-filled pools with an invalid page in a
prefix.  Against the reference route every case is held to the plain bar;
against the fp64 ideal, q8_0 pools (x20 outliers) also allow 2^-10 of
sum_p p |v| per output, the reference route's own fp16 rounding of P."""
import numpy as np
import pytest

import emelk
import oracle
from kvsetup import Scenario, assert_close

pytestmark = pytest.mark.gpu


def _cases(n=20, seed=5150):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n:
        D = int(rng.choice([64, 128, 128, 256, 512]))
        n_kv = int(rng.choice([1, 2, 4]))
        group = int(rng.choice([1, 2, 4, 8]))
        bt = int(rng.choice([8, 16, 32, 64]))
        kv_type = emelk.KV_F16 if rng.random() < 0.5 else emelk.KV_Q8_0
        if kv_type == emelk.KV_Q8_0 and (bt * D) % 256 != 0:
            continue
        n_seq = int(rng.choice([1, 2, 3]))
        n_q = int(rng.choice([1, 7, 33, 64, 100]))
        prefix = int(rng.choice([0, 50, 300, 900, 2000]))
        q_starts = [int(x) for x in rng.integers(0, prefix + 1, size=n_seq)]
        # oracle cost: attended keys x heads x head_dim over every row
        while sum((s + n_q) * n_q for s in q_starts) * n_kv * group * D > 3e9:
            q_starts = [s // 2 for s in q_starts]
            if max(q_starts) == 0:
                n_q = max(1, n_q // 2)
        nan_pool = rng.random() < 0.3
        # an invalid page inside sequence 0's prefix (kept clear of the chunk)
        bad_page = int(rng.integers(0, q_starts[0] // bt)) if nan_pool and q_starts[0] >= 2 * bt else -1
        cases.append((D, n_kv, group, bt, kv_type, q_starts, n_q, nan_pool, bad_page,
                      int(rng.integers(1 << 30))))
    return cases


CASES = _cases()


@pytest.mark.parametrize("case", CASES, ids=[f"prefill{i}" for i in range(len(CASES))])
def test_prefill_shape_sweep(device, case):
    import torch
    D, n_kv, group, bt, kv_type, q_starts, n_q, nan_pool, bad_page, seed = case
    n_head = n_kv * group
    print(f"\n[gpu-case] prefill sweep D={D} n_kv={n_kv} G={group} bt={bt} type={kv_type} "
          f"q_starts={q_starts} n_q={n_q} nan_pool={nan_pool} bad_page={bad_page}", flush=True)
    lens = [s + n_q for s in q_starts]
    q8 = kv_type == emelk.KV_Q8_0
    sc = Scenario(n_layer=1, n_head=n_head, n_kv=n_kv, head_dim=D, block_tokens=bt, lens=lens,
                  seed=seed, kv_type=kv_type, pool_byte=0xFF if nan_pool else 0,
                  extra_blocks=6 if nan_pool else 3, outlier_frac=0.01 if q8 else 0.0)
    t = sc.tables_host.copy()
    if bad_page >= 0:
        t[0, bad_page] = 0xFFFF
        sc.tables = torch.from_numpy(np.ascontiguousarray(t).view(np.int16)).to(device)
    rng = np.random.default_rng(seed + 1)
    q = rng.standard_normal((sc.n_seq, n_q, n_head, D)).astype(np.float32)
    qd = torch.from_numpy(q).to(device)
    out = torch.full_like(qd, float("nan"))
    scale = 1.0 / np.sqrt(D)
    emelk.prefill_chunk(sc.g, sc.k_pool, sc.v_pool, 0, qd, out,
                        torch.tensor(q_starts, dtype=torch.int32, device=device), sc.tables, scale)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    kc, vc = sc.oracle_cache(0)
    stored = ((lambda r: oracle.dequantize_q8_0(oracle.quantize_q8_0(r))) if q8 else
              (lambda r: oracle.fp16_to_fp32(oracle.fp32_to_fp16(r))))
    for s in range(sc.n_seq):
        kf, vf = stored(sc.k_rows[0][s]), stored(sc.v_rows[0][s])
        for r in range(n_q):
            limit = q_starts[s] + r + 1
            keep = np.array([t[s, p // bt] != 0xFFFF for p in range(limit)])
            qr = oracle.fp16_to_fp32(oracle.fp32_to_fp16(q[s, r].ravel()))
            kk, vv, n = kf[:limit][keep], vf[:limit][keep], int(keep.sum())
            ideal = oracle.attention_f64(qr, kk, vv, n_head, n_kv, D, n, scale)
            atol = 2e-3
            if q8:  # the reference's own fp16 rounding of P, against the ideal only
                mag = oracle.attention_f64(qr, kk, np.abs(vv), n_head, n_kv, D, n, scale)
                atol = 2e-3 + 2.0 ** -10 * np.asarray(mag)
            g = got[s, r].ravel()
            assert_close(g, ideal, atol=atol, what=f"seq {s} row {r} vs fp64 ideal")
            if keep.all():
                fn = oracle.compute_attention_q8_0 if q8 else oracle.compute_attention_f16
                want = fn(q[s, r].ravel(), kc, vc, sc.tables_host[s], bt, n_head, n_kv, D, limit,
                          limit, scale)
                assert_close(g, want, what=f"seq {s} row {r} vs reference route")
