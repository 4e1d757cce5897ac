"""GPU parity of the fused step before append (emelk_kv_qkv_rope_append)
against the oracle's restatement of compute_layer_attention_residual's
norm -> RoPE -> store (text/generator/detail.hpp:3806-3825): roped q and the
pool bytes are bit-exact."""
import numpy as np
import pytest

import emelk
import oracle
from kvsetup import Scenario

pytestmark = pytest.mark.gpu


def banner(msg):
    print(f"\n[gpu-case] {msg}", flush=True)


CASES = [
    # kv_type, n_head, n_kv, D, bt, pairing, n_rot, freq_base, qk_norm, v_rms, lens
    (emelk.KV_F16, 16, 8, 128, 32, emelk.NEOX_PAIRING, 128, 1e6, True, False, [70, 9]),
    (emelk.KV_F16, 32, 8, 64, 16, emelk.NORMAL_PAIRING, 64, 5e5, False, False, [33, 1, 47]),
    (emelk.KV_Q8_0, 32, 8, 128, 32, emelk.NORMAL_PAIRING, 128, 5e5, False, False, [65, 40]),
    (emelk.KV_Q8_0, 8, 2, 128, 32, emelk.NEOX_PAIRING, 64, 1e4, True, True, [37, 96]),
    # launches of 65536 rows or more (prefill chunks) take the multi-row
    # kernel: its register route (adjacent pairs, no norms, f16; two
    # sequences, the second's table row 2 bytes off a 4-byte boundary as the
    # stride of 45 pages is odd) and its LDS route
    (emelk.KV_F16, 32, 8, 128, 32, emelk.NORMAL_PAIRING, 128, 5e5, False, False, [1370, 1370]),
    (emelk.KV_F16, 32, 8, 64, 16, emelk.NORMAL_PAIRING, 32, 5e5, False, False, [1400]),
    (emelk.KV_F16, 16, 8, 128, 32, emelk.NEOX_PAIRING, 128, 1e6, True, False, [2100]),
    (emelk.KV_Q8_0, 32, 8, 128, 32, emelk.NORMAL_PAIRING, 128, 5e5, False, False, [1400]),
    (emelk.KV_Q8_0, 8, 2, 128, 32, emelk.NEOX_PAIRING, 64, 1e4, True, True, [5500]),
]


@pytest.mark.parametrize("case", CASES, ids=[f"case{i}" for i in range(len(CASES))])
def test_qkv_rope_append_is_bit_exact(device, case):
    import torch
    kv_type, n_head, n_kv, D, bt, pairing, n_rot, base, qk_norm, v_rms, lens = case
    banner(f"qkv_rope_append kv_type={kv_type} H={n_head}/{n_kv} D={D} pairing={pairing} "
           f"n_rot={n_rot} qk_norm={qk_norm} v_rms={v_rms} lens={lens}")
    sc = Scenario(n_layer=2, n_head=n_head, n_kv=n_kv, head_dim=D, block_tokens=bt, lens=lens,
                  kv_type=kv_type, seed=23, fill=False,
                  outlier_frac=0.01 if kv_type == emelk.KV_Q8_0 else 0.0)
    rng = np.random.default_rng(99)
    eps = 1e-6
    qn = rng.standard_normal(D).astype(np.float32) if qk_norm else None
    kn = rng.standard_normal(D).astype(np.float32) if qk_norm else None
    q_rows = [[rng.standard_normal((n, n_head * D)).astype(np.float32) for n in lens]
              for _ in range(sc.n_layer)]
    rope = emelk.RopeTable(n_rot, D, max(lens) + 5, base, pairing)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    qn_d = dev(qn) if qk_norm else None
    kn_d = dev(kn) if qk_norm else None

    q_got = [[None] * sc.n_seq for _ in range(sc.n_layer)]
    for layer in range(sc.n_layer):
        # every token but the last, one chunked call per sequence
        for s, n in enumerate(lens):
            q_got[layer][s] = np.zeros((n, n_head * D), np.float32)
            if n == 1:
                continue
            q_in = dev(q_rows[layer][s][:n - 1]).view(1, n - 1, -1)
            q_out = torch.zeros_like(q_in)
            emelk.qkv_rope_append(sc.g, sc.k_pool, sc.v_pool, layer, q_in, q_out,
                                  dev(sc.k_rows[layer][s][:n - 1]).view(1, n - 1, -1),
                                  dev(sc.v_rows[layer][s][:n - 1]).view(1, n - 1, -1),
                                  torch.zeros(1, dtype=torch.int32, device=device),
                                  sc.tables[s:s + 1], rope, qn_d, kn_d, v_rms, eps)
            q_got[layer][s][:n - 1] = q_out.cpu().numpy().reshape(n - 1, -1)
        # the last token of every sequence in one batched decode-shaped call
        q_in = dev(np.stack([q_rows[layer][s][n - 1] for s, n in enumerate(lens)])).view(
            sc.n_seq, 1, -1)
        q_out = q_in.clone()  # q_out may alias q_in; use a copy to keep q_in for nothing else
        emelk.qkv_rope_append(sc.g, sc.k_pool, sc.v_pool, layer, q_out, q_out,
                              dev(np.stack([sc.k_rows[layer][s][n - 1] for s, n in
                                            enumerate(lens)])).view(sc.n_seq, 1, -1),
                              dev(np.stack([sc.v_rows[layer][s][n - 1] for s, n in
                                            enumerate(lens)])).view(sc.n_seq, 1, -1),
                              torch.tensor([n - 1 for n in lens], dtype=torch.int32,
                                           device=device),
                              sc.tables, rope, qn_d, kn_d, v_rms, eps)
        last = q_out.cpu().numpy().reshape(sc.n_seq, -1)
        for s, n in enumerate(lens):
            q_got[layer][s][n - 1] = last[s]
    torch.cuda.synchronize()

    # oracle: the same steps per token, then the plain store
    for layer in range(sc.n_layer):
        for s, n in enumerate(lens):
            for t in range(n):
                qo, ko, vo = oracle.qkv_rope_rows(q_rows[layer][s][t], sc.k_rows[layer][s][t],
                                                  sc.v_rows[layer][s][t], n_head, n_kv, D,
                                                  pairing, n_rot, base, t, q_norm=qn,
                                                  k_norm=kn, v_rms=v_rms, eps=eps)
                np.testing.assert_array_equal(q_got[layer][s][t].view(np.uint32),
                                              qo.view(np.uint32),
                                              err_msg=f"q layer {layer} seq {s} token {t}")
                sc.k_rows[layer][s][t] = ko
                sc.v_rows[layer][s][t] = vo
    for which, pool in (("k", sc.k_pool), ("v", sc.v_pool)):
        np.testing.assert_array_equal(pool.cpu().numpy(), sc.expected_pool(which),
                                      err_msg=f"{which} pool")
    rope.close()


def test_qkv_rope_append_skips_tokens_outside_table_and_pool(device):
    """Tokens past the rope table, past the block table or on an invalid page
    write nothing (q_out included)."""
    import torch
    banner("qkv_rope_append skips")
    sc = Scenario(n_layer=1, n_head=4, n_kv=2, head_dim=64, block_tokens=16, lens=[40],
                  seed=5, fill=False)
    rope = emelk.RopeTable(64, 64, 20, 1e4)  # positions [0, 20) only
    n = 40
    q = torch.randn(1, n, 4 * 64, device=device)
    q_out = torch.full_like(q, 7.0)
    k = torch.from_numpy(sc.k_rows[0][0]).to(device).view(1, n, -1)
    v = torch.from_numpy(sc.v_rows[0][0]).to(device).view(1, n, -1)
    pos = torch.zeros(1, dtype=torch.int32, device=device)
    emelk.qkv_rope_append(sc.g, sc.k_pool, sc.v_pool, 0, q, q_out, k, v, pos, sc.tables, rope)
    torch.cuda.synchronize()
    got = q_out.cpu().numpy()[0]
    assert np.all(got[20:] == 7.0)
    assert not np.any(got[:20] == 7.0)
    # pool: only tokens < 20 were written
    sc.lens = [20]
    sc.k_rows[0][0] = sc.k_rows[0][0][:20].copy()
    sc.v_rows[0][0] = sc.v_rows[0][0][:20].copy()
    for t in range(20):  # rows 0..19 after RoPE
        _, ko, vo = oracle.qkv_rope_rows(np.zeros(4 * 64, np.float32), sc.k_rows[0][0][t],
                                         sc.v_rows[0][0][t], 4, 2, 64, emelk.NORMAL_PAIRING, 64,
                                         1e4, t)
        sc.k_rows[0][0][t] = ko
        sc.v_rows[0][0][t] = vo
    for which, pool in (("k", sc.k_pool), ("v", sc.v_pool)):
        np.testing.assert_array_equal(pool.cpu().numpy(), sc.expected_pool(which))
    # an invalid page in the block table: the token is skipped
    bad = sc.tables.clone()
    bad[0, 0] = -1  # 0xFFFF
    q_out.fill_(7.0)
    emelk.qkv_rope_append(sc.g, sc.k_pool, sc.v_pool, 0, q[:, :1], q_out[:, :1], k[:, :1],
                          v[:, :1], pos, bad, rope)
    torch.cuda.synchronize()
    assert np.all(q_out.cpu().numpy()[0, 0] == 7.0)
    rope.close()


def test_qkv_rope_append_skips_in_a_multi_row_launch(device):
    """The same skips in a launch of 65536 rows or more (the multi-row
    kernel): tokens past the rope table, and the tokens of an invalid page,
    write neither q nor the pool; every other token is bit-exact."""
    import torch
    banner("qkv_rope_append skips, multi-row launch")
    n, H, HK, D, bt = 1400, 32, 8, 64, 16
    sc = Scenario(n_layer=1, n_head=H, n_kv=HK, head_dim=D, block_tokens=bt, lens=[n], seed=8,
                  fill=False)
    assert n * (H + 2 * HK) >= 65536
    rope = emelk.RopeTable(D, D, 1000, 1e4)  # positions [0, 1000) only
    bad = sc.tables.clone()
    bad[0, 3] = -1  # tokens 48..63: an invalid page
    rng = np.random.default_rng(9)
    q = rng.standard_normal((n, H * D)).astype(np.float32)
    q_out = torch.full((1, n, H * D), 7.0, device=device)
    emelk.qkv_rope_append(sc.g, sc.k_pool, sc.v_pool, 0, torch.from_numpy(q).to(device).view(1, n, -1),
                          q_out, torch.from_numpy(sc.k_rows[0][0]).to(device).view(1, n, -1),
                          torch.from_numpy(sc.v_rows[0][0]).to(device).view(1, n, -1),
                          torch.zeros(1, dtype=torch.int32, device=device), bad, rope)
    torch.cuda.synchronize()
    got = q_out.cpu().numpy()[0]
    skipped = [t >= 1000 or t // bt == 3 for t in range(n)]
    written = np.zeros((n, HK * D), bool)
    for t in range(n):
        if skipped[t]:
            assert np.all(got[t] == 7.0), t
            continue
        qo, ko, vo = oracle.qkv_rope_rows(q[t], sc.k_rows[0][0][t], sc.v_rows[0][0][t], H, HK, D,
                                          emelk.NORMAL_PAIRING, D, 1e4, t)
        np.testing.assert_array_equal(got[t].view(np.uint32), qo.view(np.uint32), err_msg=str(t))
        sc.k_rows[0][0][t], sc.v_rows[0][0][t] = ko, vo
        written[t] = True
    # the pool holds exactly the written tokens (expected_pool leaves the
    # others' bytes at zero, as the pool started)
    for which, pool in (("k", sc.k_pool), ("v", sc.v_pool)):
        rows = sc.k_rows if which == "k" else sc.v_rows
        rows[0][0] = np.where(written, rows[0][0], 0.0).astype(np.float32)
        np.testing.assert_array_equal(pool.cpu().numpy(), sc.expected_pool(which),
                                      err_msg=f"{which} pool")
    rope.close()


@pytest.mark.parametrize("kv_type,D,n_rot,pairing", [
    (emelk.KV_F16, 256, 256, emelk.NEOX_PAIRING),
    (emelk.KV_Q8_0, 512, 512, emelk.NORMAL_PAIRING),
    (emelk.KV_F16, 512, 128, emelk.NEOX_PAIRING),     # partial rotation
])
def test_qkv_rope_append_large_heads_bit_exact(device, kv_type, D, n_rot, pairing):
    """head_dim 256 and 512 (more rotation pairs than lanes): q and pool
    bytes bit-exact, with both norms."""
    case = (kv_type, 8, 2, D, 16, pairing, n_rot, 1e6, True, True, [21, 5])
    test_qkv_rope_append_is_bit_exact(device, case)
