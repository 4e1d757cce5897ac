"""Decode on contiguous caches (emelk_attn_decode_contiguous): each
sequence's pages in order, no block table.  The kernel is the paged one with
the page of a token computed instead of read, so every result must equal,
bit for bit, the paged entry points over the equivalent identity tables (the
paged route's own parity against the oracle is tested in
test_gpu_parity.py).  With one page spanning the capacity the pools are the
flash route's caches (make_flash_attn_request, text/generator/detail.hpp:
3232-3292), which the last test passes as they are."""
import numpy as np
import pytest

import emelk
from kvsetup import Scenario, banner

pytestmark = pytest.mark.gpu

# n_head, n_kv, D, bt, lens (every sequence the same page count), kv type
CASES = [
    (16, 8, 128, 16, [513], emelk.KV_F16),              # config 1 shape
    (16, 8, 128, 16, [1], emelk.KV_F16),
    (8, 2, 64, 32, [250, 256, 230], emelk.KV_F16),      # 8 pages each
    (32, 8, 128, 32, [1000, 993], emelk.KV_Q8_0),       # 32 pages each
    (8, 1, 256, 16, [300], emelk.KV_Q8_0),
    (16, 2, 128, 16, [4000], emelk.KV_F16),             # balanced plan off, many splits
]


def _scenario(case, seed):
    n_head, n_kv, D, bt, lens, kv_type = case
    pages = {-(-n // bt) for n in lens}
    assert len(pages) == 1, "every sequence must hold the same number of pages"
    sc = Scenario(n_layer=2, n_head=n_head, n_kv=n_kv, head_dim=D, block_tokens=bt, lens=lens,
                  seed=seed, identity=True, kv_type=kv_type,
                  outlier_frac=0.01 if kv_type == emelk.KV_Q8_0 else 0.0)
    pps = pages.pop()
    want = np.array([[s * pps + i for i in range(pps)] for s in range(len(lens))])
    assert np.array_equal(sc.tables_host[:, :pps], want), "identity placement"
    return sc, pps * bt


@pytest.mark.parametrize("case", CASES, ids=[f"contig{i}" for i in range(len(CASES))])
def test_contiguous_decode_equals_paged_decode(device, case):
    import torch
    banner(f"contiguous decode {case}")
    sc, stride = _scenario(case, 900 + len(case[4]))
    n_seq, mx = sc.n_seq, max(sc.lens)
    for layer in range(2):
        q = np.random.default_rng(layer).standard_normal((n_seq, sc.n_head * sc.D)).astype(np.float32)
        paged = sc.gpu_decode(layer, q)
        qd = torch.from_numpy(q).to(device).view(n_seq, sc.n_head, sc.D)
        out = torch.full_like(qd, float("nan"))
        ws = torch.zeros(emelk.decode_workspace_bytes(sc.g, n_seq, mx) // 4 + 1,
                         dtype=torch.float32, device=device)
        kl = torch.tensor(sc.lens, dtype=torch.int32, device=device)
        emelk.decode_contiguous(sc.g, sc.k_pool, sc.v_pool, layer, qd, out, kl, mx, stride,
                                float(1.0 / np.sqrt(sc.D)), ws)
        torch.cuda.synchronize()
        got = out.view(n_seq, -1).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), paged.view(np.uint32)), f"layer {layer}"


@pytest.mark.parametrize("case", [c for c in CASES if all(n % c[3] for n in c[4])],
                         ids=lambda c: f"H{c[0]}_D{c[2]}_bt{c[3]}_n{len(c[4])}_t{c[5]}")
def test_contiguous_decode_append_equals_paged_decode_append(device, case):
    # the step's token lands in each sequence's last page (no new page), so
    # the identity placement holds after it
    import torch
    banner(f"contiguous decode_append {case}")
    sc_a, stride = _scenario(case, 77)
    sc_b, _ = _scenario(case, 77)
    n_seq = sc_a.n_seq
    kv_lens = [n + 1 for n in sc_a.lens]
    for sc in (sc_a, sc_b):
        for s in range(n_seq):
            assert sc.actor.allocate_slots(s, 1)[0]
        sc.refresh_tables()
    assert np.array_equal(sc_a.tables_host, sc_b.tables_host)
    rng = np.random.default_rng(5)
    kd = sc_a.n_kv * sc_a.D
    nk = torch.from_numpy(rng.standard_normal((n_seq, kd)).astype(np.float32)).to(device)
    nv = torch.from_numpy(rng.standard_normal((n_seq, kd)).astype(np.float32)).to(device)
    q = torch.from_numpy(rng.standard_normal((n_seq, sc_a.n_head, sc_a.D)).astype(np.float32)).to(device)
    kl = torch.tensor(kv_lens, dtype=torch.int32, device=device)
    mx = max(kv_lens)
    scale = float(1.0 / np.sqrt(sc_a.D))
    ws = torch.zeros(emelk.decode_workspace_bytes(sc_a.g, n_seq, mx) // 4 + 1,
                     dtype=torch.float32, device=device)
    out_a = torch.full_like(q, float("nan"))
    out_b = torch.full_like(q, float("nan"))
    emelk.decode_append(sc_a.g, sc_a.k_pool, sc_a.v_pool, 1, nk, nv, q, out_a, kl, mx,
                        sc_a.tables, scale, ws)
    emelk.decode_contiguous(sc_b.g, sc_b.k_pool, sc_b.v_pool, 1, q, out_b, kl, mx, stride, scale,
                            ws, k_rows=nk, v_rows=nv)
    torch.cuda.synchronize()
    assert torch.equal(out_a.view(torch.int32), out_b.view(torch.int32))
    assert torch.equal(sc_a.k_pool, sc_b.k_pool) and torch.equal(sc_a.v_pool, sc_b.v_pool)


@pytest.mark.parametrize("cap,n,D,G", [(640, 513, 128, 2), (96, 1, 128, 2), (1024, 1000, 64, 4)])
def test_contiguous_decode_on_the_flash_route_caches(device, cap, n, D, G):
    """The reference's flash caches, [layer][kv_head][capacity][head_dim] f16
    (make_flash_attn_request's src1/src2 views, text/generator/detail.hpp:
    3258-3269), are the pool of a geometry with block_tokens = capacity and
    max_blocks = 1: passed as they are, the step stores its token at n - 1
    and attends over n tokens, held to the bar against the reference's flash
    route (f16 accumulator) and the fp64 ideal."""
    import torch
    import oracle
    from kvsetup import assert_close
    banner(f"contiguous decode on flash-layout caches cap={cap} n={n} D={D} G={G}")
    L, HK = 2, 4
    H = HK * G
    g = emelk.geometry(L, H, HK, D, cap, 1)
    rng = np.random.default_rng(cap + n)
    k16 = oracle.fp32_to_fp16(rng.standard_normal((L, HK, cap, D)).astype(np.float32))
    v16 = oracle.fp32_to_fp16(rng.standard_normal((L, HK, cap, D)).astype(np.float32))
    assert emelk.pool_bytes(g) == k16.nbytes
    k_pool = torch.from_numpy(k16.view(np.uint8).ravel().copy()).to(device)
    v_pool = torch.from_numpy(v16.view(np.uint8).ravel().copy()).to(device)
    layer = 1
    q = rng.standard_normal((1, H * D)).astype(np.float32)
    nk = rng.standard_normal((1, HK * D)).astype(np.float32)
    nv = rng.standard_normal((1, HK * D)).astype(np.float32)
    qd = torch.from_numpy(q).to(device).view(1, H, D)
    out = torch.full_like(qd, float("nan"))
    ws = torch.zeros(emelk.decode_workspace_bytes(g, 1, n) // 4 + 1, dtype=torch.float32,
                     device=device)
    kl = torch.tensor([n], dtype=torch.int32, device=device)
    scale = float(1.0 / np.sqrt(D))
    emelk.decode_contiguous(g, k_pool, v_pool, layer, qd, out, kl, n, cap, scale, ws,
                            k_rows=torch.from_numpy(nk).to(device),
                            v_rows=torch.from_numpy(nv).to(device))
    torch.cuda.synchronize()
    got = out.view(-1).cpu().numpy()
    # the store: row n - 1 of every head holds fp16 of the new rows
    k16[layer, :, n - 1] = oracle.fp32_to_fp16(nk.reshape(HK, D))
    v16[layer, :, n - 1] = oracle.fp32_to_fp16(nv.reshape(HK, D))
    assert np.array_equal(k_pool.cpu().numpy(), k16.view(np.uint8).ravel())
    assert np.array_equal(v_pool.cpu().numpy(), v16.view(np.uint8).ravel())
    flash = oracle.flash_attn_f16acc(q[0], np.ascontiguousarray(k16[layer]),
                                     np.ascontiguousarray(v16[layer]), D, H, HK, n, cap, scale)
    assert_close(got, flash, what="vs the reference's flash route (f16 accumulator)")
    rows = lambda x: oracle.fp16_to_fp32(x[layer, :, :n].transpose(1, 0, 2).reshape(n, HK * D))  # noqa: E731
    qr = oracle.fp16_to_fp32(oracle.fp32_to_fp16(q[0]))
    ideal = oracle.attention_f64(qr, rows(k16), rows(v16), H, HK, D, n, scale)
    assert_close(got, ideal, what="vs fp64 ideal")
