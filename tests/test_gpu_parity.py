"""GPU parity of the HIP path against the CPU oracle, through the C ABI.

Append, quantization, gather and page copies: bit-exact.  Attention:
|gpu - oracle| <= 2e-3 + 1e-2*|oracle| (max-abs 2e-3 / max-rel 1e-2, fp32
accumulation), also checked against the fp64 ideal.  Shapes are the
BASELINE.json configs with fewer layers/sequences where the CPU oracle would
be slow; full-size properties are checked separately."""
import numpy as np
import pytest

import emelk
import oracle
from kvsetup import Scenario, assert_close

pytestmark = pytest.mark.gpu


def banner(msg):
    print(f"\n[gpu-case] {msg}", flush=True)


# ---------------------------------------------------------------- append ----

@pytest.mark.parametrize("kv_type,D,bt,lens", [
    (emelk.KV_F16, 64, 16, [1, 17, 100]),
    (emelk.KV_F16, 128, 32, [33, 64, 5]),
    (emelk.KV_Q8_0, 128, 32, [31, 70]),
    (emelk.KV_Q8_0, 64, 16, [1, 48]),
])
def test_append_is_bit_exact(device, kv_type, D, bt, lens):
    banner(f"append kv_type={kv_type} D={D} bt={bt} lens={lens}")
    sc = Scenario(n_layer=2, n_head=8, n_kv=2, head_dim=D, block_tokens=bt, lens=lens,
                  kv_type=kv_type, seed=11, outlier_frac=0.01 if kv_type == emelk.KV_Q8_0 else 0)
    for which, pool in (("k", sc.k_pool), ("v", sc.v_pool)):
        got = pool.cpu().numpy()
        np.testing.assert_array_equal(got, sc.expected_pool(which))


def test_q8_0_append_matches_reference_golden_blocks(device):
    # the reference quantizer's own outputs (tests/golden/q8_0.npz) through
    # the device append: 68 rows of 1024 values = 8 kv heads x 128 dims
    banner("q8_0 golden rows through append")
    import os
    import torch
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "q8_0.npz"))
    x = g["x"]
    n = x.shape[0]
    geo = emelk.geometry(1, 8, 8, 128, 4, -(-n // 4) + 1, emelk.KV_Q8_0)
    pb = emelk.pool_bytes(geo)
    kp = torch.zeros(pb, dtype=torch.uint8, device=device)
    vp = torch.zeros(pb, dtype=torch.uint8, device=device)
    pages = -(-n // 4)
    table = torch.arange(pages, dtype=torch.int16, device=device).view(1, -1)
    rows = torch.from_numpy(x).to(device).view(1, n, 1024)
    emelk.append(geo, kp, vp, 0, rows, rows, torch.zeros(1, dtype=torch.int32, device=device),
                 table)
    lengths = torch.tensor([n], dtype=torch.int32, device=device)
    ko = torch.zeros(n * 8 * 4 * 34, dtype=torch.uint8, device=device)
    vo = torch.zeros_like(ko)
    emelk.gather(geo, kp, vp, 0, lengths, table, ko, vo, n)
    got = ko.cpu().numpy().reshape(8, n, 4 * 34).transpose(1, 0, 2).reshape(n, -1)
    np.testing.assert_array_equal(got, g["blocks"])


# ---------------------------------------------------------------- gather ----

@pytest.mark.parametrize("kv_type", [emelk.KV_F16, emelk.KV_Q8_0])
def test_gather_follows_block_table(device, kv_type):
    banner(f"gather kv_type={kv_type}")
    import torch
    sc = Scenario(n_layer=2, n_head=8, n_kv=2, head_dim=128, block_tokens=32, lens=[45, 1, 96],
                  kv_type=kv_type, seed=3)
    out_tokens = 100
    esz = 2 * 128 if kv_type == emelk.KV_F16 else 4 * 34
    lengths = torch.tensor(sc.lens, dtype=torch.int32, device=device)
    for layer in range(2):
        ko = torch.full((sc.n_seq * 2 * out_tokens * esz,), 7, dtype=torch.uint8, device=device)
        vo = torch.full_like(ko, 7)
        emelk.gather(sc.g, sc.k_pool, sc.v_pool, layer, lengths, sc.tables, ko, vo, out_tokens)
        for which, buf, rows in (("k", ko, sc.k_rows), ("v", vo, sc.v_rows)):
            got = buf.cpu().numpy().reshape(sc.n_seq, 2, out_tokens, esz)
            for s, n in enumerate(sc.lens):
                src = rows[layer][s].reshape(n, 2, 128)
                if kv_type == emelk.KV_F16:
                    want = oracle.fp32_to_fp16(src).transpose(1, 0, 2).view(np.uint8).reshape(2, n, esz)
                else:
                    want = oracle.quantize_q8_0(src).transpose(1, 0, 2).view(np.uint8).reshape(2, n, esz)
                np.testing.assert_array_equal(got[s, :, :n], want)
                assert not got[s, :, n:].any()  # past the length: zeros


# ------------------------------------------------------------- copy/compact -

def test_copy_blocks_and_compaction_are_bit_exact(device):
    banner("evict 25% + compact, f16")
    import torch
    lens = [4096 // 16, 300, 200]  # small variant of the chunked-prefill workload
    sc = Scenario(n_layer=3, n_head=8, n_kv=2, head_dim=64, block_tokens=16, lens=lens,
                  seed=5, extra_blocks=16)
    rng = np.random.default_rng(9)
    before = {}
    lengths = torch.tensor(sc.lens, dtype=torch.int32, device=device)
    out_tokens = max(lens)
    def gather_all():
        res = []
        for layer in range(sc.n_layer):
            ko = torch.zeros(sc.n_seq * 2 * out_tokens * 128, dtype=torch.uint8, device=device)
            vo = torch.zeros_like(ko)
            lengths = torch.tensor(sc.lens, dtype=torch.int32, device=device)
            emelk.gather(sc.g, sc.k_pool, sc.v_pool, layer, lengths, sc.tables, ko, vo, out_tokens)
            res.append((ko.cpu().numpy().reshape(sc.n_seq, 2, out_tokens, 128),
                        vo.cpu().numpy().reshape(sc.n_seq, 2, out_tokens, 128)))
        return res
    full = gather_all()
    kept = {}
    for s, n in enumerate(lens):
        nb = -(-n // 16)
        ev = sorted(rng.choice(nb - 1, size=max(1, nb // 4), replace=False).tolist())
        ok, err, removed = sc.actor.evict_blocks(s, ev)
        assert ok, err
        keep_tok = [t for t in range(n) if t // 16 not in ev]
        kept[s] = keep_tok
        sc.lens[s] = n - removed
        assert len(keep_tok) == sc.lens[s]
    ok, err, moves = sc.actor.compact()
    assert ok and len(moves) > 0
    mv = torch.tensor(moves, dtype=torch.int32, device=device)
    emelk.copy_blocks(sc.g, sc.k_pool, sc.v_pool, mv)
    torch.cuda.synchronize()
    sc.refresh_tables()
    n_live = sum(-(-n // 16) for n in sc.lens)
    assert int(sc.tables_host[sc.tables_host != 0xFFFF].max()) < n_live
    after = gather_all()
    for layer in range(sc.n_layer):
        for kv in range(2):
            for s in range(sc.n_seq):
                want = full[layer][kv][s][:, kept[s]]
                got = after[layer][kv][s][:, :sc.lens[s]]
                np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("kv_type,D,bt", [(emelk.KV_F16, 128, 32), (emelk.KV_Q8_0, 128, 32),
                                          (emelk.KV_Q8_0, 64, 16)])
def test_compaction_moves_exactly_the_listed_pages(device, kv_type, D, bt):
    """The whole pool after compaction, byte for byte: every (layer, moved
    page) holds its source page's bytes of before the call, K and V, and
    every other byte is unchanged (q8_0 pages move with their scale planes)."""
    banner(f"compaction, whole-pool check, kv_type={kv_type} D={D} bt={bt}")
    import torch
    lens = [20 * bt + 3, 9 * bt, 31 * bt + 1, 5]
    sc = Scenario(n_layer=3, n_head=8, n_kv=2, head_dim=D, block_tokens=bt, lens=lens,
                  kv_type=kv_type, seed=15, extra_blocks=8, outlier_frac=0.01)
    rng = np.random.default_rng(16)
    for s_, n in enumerate(lens):
        nb = -(-n // bt)
        if nb < 2:
            continue
        ev = sorted(rng.choice(nb - 1, size=max(1, nb // 4), replace=False).tolist())
        assert sc.actor.evict_blocks(s_, ev)[0]
    ok, err, moves = sc.actor.compact()
    assert ok and len(moves) > 0, err
    k_old = sc.k_pool.cpu().numpy()
    v_old = sc.v_pool.cpu().numpy()
    emelk.copy_blocks(sc.g, sc.k_pool, sc.v_pool, torch.tensor(moves, dtype=torch.int32,
                                                               device=device))
    torch.cuda.synchronize()
    pb = emelk.pool_bytes(sc.g)
    page = pb // (sc.n_layer * sc.max_blocks)
    mv = np.asarray(moves, np.int64).reshape(-1, 2)
    srcs, dsts = set(mv[:, 0].tolist()), set(mv[:, 1].tolist())
    assert not (srcs & dsts), "a move list never chains pages"
    for old, pool in ((k_old, sc.k_pool), (v_old, sc.v_pool)):
        want = old.reshape(sc.n_layer, sc.max_blocks, page).copy()
        for src, dst in mv:
            want[:, dst] = old.reshape(sc.n_layer, sc.max_blocks, page)[:, src]
        np.testing.assert_array_equal(pool.cpu().numpy().reshape(want.shape), want)


def test_copy_block_callback_splits_shared_tail(device):
    banner("copy_block callback through allocate_slots")
    import ctypes
    import os
    import torch
    g = emelk.geometry(2, 8, 2, 64, 16, 8)
    cache = ctypes.c_void_p()
    stream = torch.cuda.current_stream().cuda_stream
    assert emelk.lib.emelk_kv_cache_create(ctypes.byref(g), ctypes.c_void_p(stream),
                                           ctypes.byref(cache)) == 0
    try:
        kp = emelk.lib.emelk_kv_cache_k_pool(cache)
        vp = emelk.lib.emelk_kv_cache_v_pool(cache)
        a = emelk.KvActor()
        a.reserve(2, 8, 16)
        a.allocate_sequence(0)
        a.allocate_slots(0, 10)
        table = torch.from_numpy(a.export_block_tables([0], 4).view(np.int16)).to(device)
        rows = torch.randn(1, 10, 128, device=device)
        class P:  # minimal tensor-like wrapper for raw pointers
            def __init__(self, p): self.p = p
            def data_ptr(self): return self.p
        for layer in range(2):
            emelk.append(g, P(kp), P(vp), layer, rows, rows * 2,
                         torch.zeros(1, dtype=torch.int32, device=device), table)
        assert a.branch_sequence(0, 1)[0]
        fn = ctypes.cast(emelk.lib.emelk_kv_cache_copy_block, ctypes.c_void_p).value
        ok, err, cnt = a.allocate_slots(1, 1, copy_block=fn, copy_block_user_data=cache.value)
        assert ok and err == 0 and cnt == 1
        torch.cuda.synchronize()
        src, dst = a.lookup_kv_block(0, 0), a.lookup_kv_block(1, 0)
        assert src != dst
        pb = emelk.pool_bytes(g)
        hip = ctypes.CDLL("libamdhip64.so.7", mode=os.RTLD_NOLOAD)  # the loaded runtime
        for pool in (kp, vp):
            host = np.zeros(pb, dtype=np.uint8)
            assert hip.hipMemcpy(ctypes.c_void_p(host.ctypes.data), ctypes.c_void_p(pool),
                                 ctypes.c_size_t(pb), 2) == 0  # device -> host
            pages = host.reshape(2, 8, 2 * 16 * 64 * 2)
            np.testing.assert_array_equal(pages[:, dst], pages[:, src])
            assert pages[:, src].any()
    finally:
        emelk.lib.emelk_kv_cache_destroy(cache)


# ---------------------------------------------------------------- decode ----

def _decode_case(sc, layer, seed, scale=None):
    q = np.random.default_rng(seed).standard_normal((sc.n_seq, sc.n_head * sc.D)).astype(np.float32)
    got = sc.gpu_decode(layer, q, scale=scale)
    want = sc.oracle_decode(layer, q, scale=scale)
    err = assert_close(got, want, what="gpu vs reference route")
    ideal = sc.ideal_decode(layer, q, scale=scale)
    assert_close(got, ideal, what="gpu vs fp64 ideal")
    return err


def test_decode_config1_qwen3_contiguous(device):
    # Qwen3-0.6B shape: 16/8 heads, 128 dims, identity page map, 512 cached +
    # 1 appended token (513 attended); reference route here is the flash one.
    banner("decode config1 (qwen3, contiguous)")
    sc = Scenario(n_layer=2, n_head=16, n_kv=8, head_dim=128, block_tokens=16, lens=[513],
                  seed=1, identity=True)
    for layer in range(2):
        _decode_case(sc, layer, 100 + layer)
        q = np.random.default_rng(7 + layer).standard_normal((1, 16 * 128)).astype(np.float32)
        got = sc.gpu_decode(layer, q)
        k = oracle.fp32_to_fp16(sc.k_rows[layer][0]).reshape(513, 8, 128).transpose(1, 0, 2)
        v = oracle.fp32_to_fp16(sc.v_rows[layer][0]).reshape(513, 8, 128).transpose(1, 0, 2)
        flash = oracle.flash_attn_f16acc(q[0], np.ascontiguousarray(k), np.ascontiguousarray(v),
                                         128, 16, 8, 513, 513, 1 / np.sqrt(128))
        # the route the reference takes for an identity map (flash, f16
        # accumulator), held to the north-star bar: 2e-3 abs + 1e-2 rel
        dev = np.max(np.abs(got[0] - flash))
        print(f"[gpu-case] config1 layer {layer}: max |gpu - flash(f16 acc)| = {dev:.3e}")
        assert_close(got[0], flash, what="gpu vs reference flash route (f16 acc)")


def test_decode_config2_llama1b_ragged(device):
    banner("decode config2 (llama-3.2-1b, ragged U[1024,4096], 16-token pages)")
    lens = np.random.default_rng(2).integers(1024, 4097, size=4).tolist()
    sc = Scenario(n_layer=2, n_head=32, n_kv=8, head_dim=64, block_tokens=16, lens=lens, seed=2)
    for layer in range(2):
        _decode_case(sc, layer, 200 + layer)


def test_decode_config3_llama8b_shape(device):
    banner("decode config3 shape (llama-3-8b, ctx 8193, 32-token pages), 3 seqs")
    sc = Scenario(n_layer=1, n_head=32, n_kv=8, head_dim=128, block_tokens=32,
                  lens=[8193, 8193, 8193], seed=3)
    _decode_case(sc, 0, 300, scale=1.0 / np.sqrt(128))


def test_decode_config4_q8_0(device):
    banner("decode config4 (q8_0, ctx 16385, 1% x20 outliers), 2 seqs")
    sc = Scenario(n_layer=1, n_head=32, n_kv=8, head_dim=128, block_tokens=32,
                  lens=[16385, 9000], seed=4, kv_type=emelk.KV_Q8_0, outlier_frac=0.01)
    _decode_case(sc, 0, 400)


@pytest.mark.parametrize("n_head,n_kv,D,bt,lens,kv_type", [
    (8, 8, 64, 16, [1, 2, 3, 15, 16, 17], emelk.KV_F16),          # tiny, G=1
    (8, 1, 64, 16, [129, 128, 127], emelk.KV_F16),                # G=8
    (4, 2, 128, 32, [64, 65, 2047, 2048, 2049], emelk.KV_F16),    # tile/split edges
    (4, 2, 128, 32, [1, 33, 4097], emelk.KV_Q8_0),
    (16, 8, 128, 16, [1000], emelk.KV_Q8_0),                      # G=2 q8_0
    (8, 1, 128, 32, [129, 1000, 16], emelk.KV_Q8_0),              # G=8 q8_0
    (4, 4, 128, 12, [100, 7], emelk.KV_Q8_0),                     # G=1, pages not a multiple of 8
    (8, 2, 256, 16, [1, 40, 700], emelk.KV_Q8_0),                 # head_dim 256 q8_0, G=4
    (8, 2, 64, 16, [5, 300, 1100], emelk.KV_Q8_0),                # head_dim 64 q8_0, G=4
    (16, 8, 64, 8, [77, 3], emelk.KV_Q8_0),                       # G=2, pages not a multiple of 16
    # ragged batches: balanced splits (up to 64 sequences) and the fixed plan past 64
    (8, 2, 64, 16, [1 + (37 * i) % 700 for i in range(64)], emelk.KV_F16),
    (8, 2, 128, 32, [1 + (53 * i) % 500 for i in range(70)], emelk.KV_F16),
    (8, 2, 128, 16, [2000] + [1 + (29 * i) % 90 for i in range(40)], emelk.KV_Q8_0),
])
def test_decode_edge_shapes(device, n_head, n_kv, D, bt, lens, kv_type):
    banner(f"decode edges H={n_head} HK={n_kv} D={D} bt={bt} n_seq={len(lens)} "
           f"lens={lens[:6]} type={kv_type}")
    sc = Scenario(n_layer=1, n_head=n_head, n_kv=n_kv, head_dim=D, block_tokens=bt, lens=lens,
                  seed=sum(lens), kv_type=kv_type)
    _decode_case(sc, 0, 500 + sum(lens))


def test_decode_reused_workspace_across_shapes(device):
    """One workspace across calls whose split plans differ (other lengths and
    maximum length): every call matches the oracle, and repeating a call
    gives bit-identical output (the split merge has a fixed order)."""
    import torch
    banner("decode: one workspace, several shapes")
    lens = [3001, 700, 33, 1]
    sc = Scenario(n_layer=1, n_head=32, n_kv=8, head_dim=128, block_tokens=32, lens=lens,
                  seed=77)
    ws = torch.full((emelk.decode_workspace_bytes(sc.g, len(lens), max(lens)) // 4 + 1,),
                    float("nan"), dtype=torch.float32, device=device)
    rng = np.random.default_rng(78)
    q = rng.standard_normal((len(lens), 32 * 128)).astype(np.float32)
    scale = 1.0 / np.sqrt(128)
    first = None
    for i, ls in enumerate([lens, [64, 700, 1, 2], [1500, 1, 1, 1], lens]):
        got = sc.gpu_decode(0, q, lens=ls, ws=ws)
        assert_close(got, sc.oracle_decode(0, q, lens=ls, scale=scale),
                     what=f"call {i} lens {ls}")
        if i == 0:
            first = got
    assert np.array_equal(got.view(np.uint32), first.view(np.uint32))


def test_decode_step_append_then_attend(device):
    # One decode step as the generator runs it: allocate_slots(1) per
    # sequence, append the new token at position len, attend over len+1.
    banner("decode step: allocate 1, append, attend")
    import torch
    sc = Scenario(n_layer=2, n_head=32, n_kv=8, head_dim=128, block_tokens=32,
                  lens=[95, 96, 300], seed=8, extra_blocks=8)
    pos = torch.tensor(sc.lens, dtype=torch.int32, device=device)
    for s in range(sc.n_seq):
        ok, err, cnt = sc.actor.allocate_slots(s, 1)
        assert ok
    sc.refresh_tables()
    new_k = np.random.default_rng(1).standard_normal((2, sc.n_seq, 1, sc.kv_dim)).astype(np.float32)
    new_v = np.random.default_rng(2).standard_normal((2, sc.n_seq, 1, sc.kv_dim)).astype(np.float32)
    for layer in range(2):
        emelk.append(sc.g, sc.k_pool, sc.v_pool, layer, torch.from_numpy(new_k[layer]).to(device),
                     torch.from_numpy(new_v[layer]).to(device), pos, sc.tables)
        for s in range(sc.n_seq):
            sc.k_rows[layer][s] = np.concatenate([sc.k_rows[layer][s], new_k[layer][s]])
            sc.v_rows[layer][s] = np.concatenate([sc.v_rows[layer][s], new_v[layer][s]])
    sc.lens = [n + 1 for n in sc.lens]
    torch.cuda.synchronize()
    for which, pool in (("k", sc.k_pool), ("v", sc.v_pool)):
        np.testing.assert_array_equal(pool.cpu().numpy(), sc.expected_pool(which))
    for layer in range(2):
        _decode_case(sc, layer, 900 + layer)


@pytest.mark.parametrize("kv_type,n_head,n_kv,D,bt,lens,pool_byte", [
    (emelk.KV_F16, 32, 8, 128, 32, [95, 96, 300, 1], 0),
    (emelk.KV_F16, 32, 8, 64, 16, [15, 16, 1000], 0xFF),
    (emelk.KV_F16, 8, 8, 128, 12, [11, 40], 0),           # block_tokens not a multiple of 8
    (emelk.KV_Q8_0, 32, 8, 128, 32, [31, 32, 4000], 0xFF),
    (emelk.KV_Q8_0, 16, 8, 128, 16, [100, 1], 0),
    (emelk.KV_Q8_0, 8, 2, 64, 16, [17, 300], 0xFF),
    (emelk.KV_Q8_0, 8, 2, 256, 16, [2, 129], 0xFF),
])
def test_decode_append_is_append_then_decode(device, kv_type, n_head, n_kv, D, bt, lens,
                                             pool_byte):
    """emelk_attn_decode_append (store the token at kv_lens - 1 and attend,
    one launch) writes the same pool bytes as emelk_kv_append and gives the
    oracle's attention, including a new token on an invalid page."""
    banner(f"decode_append type={kv_type} H={n_head}/{n_kv} D={D} bt={bt} lens={lens}")
    import torch
    sc = Scenario(n_layer=2, n_head=n_head, n_kv=n_kv, head_dim=D, block_tokens=bt, lens=lens,
                  seed=sum(lens) + 3, extra_blocks=8, kv_type=kv_type, pool_byte=pool_byte)
    for s in range(sc.n_seq):
        assert sc.actor.allocate_slots(s, 1)[0]
    sc.refresh_tables()
    rng = np.random.default_rng(11)
    new_k = rng.standard_normal((2, sc.n_seq, sc.kv_dim)).astype(np.float32)
    new_v = rng.standard_normal((2, sc.n_seq, sc.kv_dim)).astype(np.float32)
    if kv_type == emelk.KV_Q8_0:
        new_k[np.abs(new_k) > 2.0] *= 20.0  # outliers set the block scales
    q = rng.standard_normal((2, sc.n_seq, n_head * D)).astype(np.float32)
    lens_now = [n + 1 for n in sc.lens]
    kl = torch.tensor(lens_now, dtype=torch.int32, device=device)
    mx = max(lens_now)
    ws = torch.zeros(emelk.decode_workspace_bytes(sc.g, sc.n_seq, mx) // 4 + 1,
                     dtype=torch.float32, device=device)
    for layer in range(2):
        out = torch.full((sc.n_seq, n_head, D), float("nan"), device=device)
        emelk.decode_append(sc.g, sc.k_pool, sc.v_pool, layer,
                            torch.from_numpy(new_k[layer]).to(device),
                            torch.from_numpy(new_v[layer]).to(device),
                            torch.from_numpy(q[layer]).to(device).view(sc.n_seq, n_head, D), out,
                            kl, mx, sc.tables, float(1 / np.sqrt(D)), ws)
        torch.cuda.synchronize()
        for s in range(sc.n_seq):
            sc.k_rows[layer][s] = np.concatenate([sc.k_rows[layer][s], new_k[layer][s][None]])
            sc.v_rows[layer][s] = np.concatenate([sc.v_rows[layer][s], new_v[layer][s][None]])
        got = out.view(sc.n_seq, -1).cpu().numpy()
        sc.lens = list(lens_now)  # the oracle's caches place the rows up to these lengths
        want = sc.oracle_decode(layer, q[layer], lens=lens_now)
        assert_close(got, want, what=f"decode_append layer {layer}")
    if pool_byte == 0:  # the oracle's pool image has zeros where nothing was written
        for which, pool in (("k", sc.k_pool), ("v", sc.v_pool)):
            np.testing.assert_array_equal(pool.cpu().numpy(), sc.expected_pool(which),
                                          err_msg=f"{which} pool after decode_append")
    # a new token on an invalid page is neither stored nor attended; the
    # page's other tokens drop out as in decode
    s0 = 0
    p = sc.lens[s0]
    t = sc.tables_host.copy()
    t[s0, p // bt] = 0xFFFF
    bad = torch.from_numpy(np.ascontiguousarray(t).view(np.int16)).to(device)
    kl2 = torch.tensor([n + 1 for n in sc.lens], dtype=torch.int32, device=device)
    ws2 = torch.zeros(emelk.decode_workspace_bytes(sc.g, sc.n_seq, mx + 1) // 4 + 1,
                      dtype=torch.float32, device=device)
    out = torch.full((sc.n_seq, n_head, D), float("nan"), device=device)
    nk = torch.randn(sc.n_seq, sc.kv_dim, device=device)
    emelk.decode_append(sc.g, sc.k_pool, sc.v_pool, 0, nk, nk.clone(),
                        torch.from_numpy(q[0]).to(device).view(sc.n_seq, n_head, D), out, kl2,
                        mx + 1, bad, float(1 / np.sqrt(D)), ws2)
    torch.cuda.synchronize()
    got = out.view(sc.n_seq, -1).cpu().numpy()
    if kv_type == emelk.KV_F16:
        stored = lambda r: oracle.fp16_to_fp32(oracle.fp32_to_fp16(r))  # noqa: E731
    else:
        stored = lambda r: oracle.dequantize_q8_0(oracle.quantize_q8_0(r))  # noqa: E731
    keep = np.array([pos // bt != p // bt for pos in range(p)])
    if keep.any():
        k = stored(sc.k_rows[0][s0])[keep]
        v = stored(sc.v_rows[0][s0])[keep]
        want = oracle.attention_f64(oracle.fp16_to_fp32(oracle.fp32_to_fp16(q[0][s0])), k, v,
                                    n_head, n_kv, D, int(keep.sum()), 1 / np.sqrt(D))
        assert_close(got[s0], want, what="new token on an invalid page")
    else:
        assert np.all(got[s0] == 0.0)


def test_decode_is_invariant_to_page_placement(device):
    # Same logical K/V under two different page permutations: bit-identical
    # outputs (size-independent property; run at config-3 head shape).
    banner("decode page-permutation invariance")
    a = Scenario(n_layer=1, n_head=32, n_kv=8, head_dim=128, block_tokens=32,
                 lens=[3000, 5000], seed=21)
    b = Scenario(n_layer=1, n_head=32, n_kv=8, head_dim=128, block_tokens=32,
                 lens=[3000, 5000], seed=21, identity=True)
    q = np.random.default_rng(4).standard_normal((2, 32 * 128)).astype(np.float32)
    assert not np.array_equal(a.tables_host, b.tables_host)
    np.testing.assert_array_equal(a.gpu_decode(0, q), b.gpu_decode(0, q))


# --------------------------------------------------------------- prefill ----

def _prefill_case(device, n_head, n_kv, D, bt, q_starts, n_q, seed):
    import torch
    lens = [s + n_q for s in q_starts]
    sc = Scenario(n_layer=1, n_head=n_head, n_kv=n_kv, head_dim=D, block_tokens=bt, lens=lens,
                  seed=seed)
    rng = np.random.default_rng(seed + 1)
    q = rng.standard_normal((sc.n_seq, n_q, n_head, D)).astype(np.float32)
    qd = torch.from_numpy(q).to(device)
    out = torch.full_like(qd, float("nan"))
    qs = torch.tensor(q_starts, dtype=torch.int32, device=device)
    scale = 1.0 / np.sqrt(D)
    emelk.prefill_chunk(sc.g, sc.k_pool, sc.v_pool, 0, qd, out, qs, sc.tables, scale)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    kc, vc = sc.oracle_cache(0)
    want = np.zeros_like(got)
    ideal = np.zeros_like(got)
    for s in range(sc.n_seq):
        kf = oracle.fp16_to_fp32(oracle.fp32_to_fp16(sc.k_rows[0][s]))
        vf = oracle.fp16_to_fp32(oracle.fp32_to_fp16(sc.v_rows[0][s]))
        for r in range(n_q):
            limit = q_starts[s] + r + 1  # row r attends causally to [0, q_start + r]
            want[s, r] = oracle.compute_attention_f16(
                q[s, r].ravel(), kc, vc, sc.tables_host[s], bt, n_head, n_kv, D, limit, limit,
                scale).reshape(n_head, D)
            qr = oracle.fp16_to_fp32(oracle.fp32_to_fp16(q[s, r].ravel()))
            ideal[s, r] = oracle.attention_f64(qr, kf[:limit], vf[:limit], n_head, n_kv, D, limit,
                                               scale).reshape(n_head, D)
    assert_close(got, want, what="prefill gpu vs reference per-row route")
    assert_close(got, ideal, what="prefill gpu vs fp64 ideal")


def test_prefill_chunk_config5_shape(device):
    # Llama-3-8B heads, 32-token pages; prefixes not multiples of the tile,
    # chunk of 96 rows (three 32-row blocks)
    banner("prefill chunk llama-3-8b heads, prefixes [200, 1000], 96 rows")
    _prefill_case(device, 32, 8, 128, 32, [200, 1000], 96, seed=31)


def test_prefill_chunk_edges(device):
    banner("prefill chunk edges: empty prefix, ragged rows, G=2 and G=1, D=64")
    _prefill_case(device, 8, 4, 64, 16, [0, 33], 40, seed=32)
    _prefill_case(device, 4, 4, 128, 16, [5], 7, seed=33)
    _prefill_case(device, 16, 2, 128, 32, [64], 33, seed=34)  # G=8


@pytest.mark.parametrize("n_head,n_kv,D,bt", [(8, 2, 128, 32), (8, 2, 128, 16),
                                               (8, 1, 512, 32), (8, 1, 512, 16)])
def test_prefill_masks_invalid_pages_and_never_reads_unwritten_slots(device, n_head, n_kv, D, bt):
    # Pools start as 0xFF bytes (f16 NaN), so any slot past a sequence's end
    # that reached P.V would poison the output.  Keys on invalid pages are
    # left out of the softmax, as decode does.  bt=32 takes the uniform-page
    # staging path, bt=16 the general one; head_dim 512 runs the 16-row
    # (M16) kernel with its own masking and V^T key order.  A second call
    # with a negative q_start for sequence 1 must write zeros for its rows
    # and leave sequence 0 unchanged.
    import torch
    banner(f"prefill on a NaN-filled pool with invalid pages, D={D} bt={bt}")
    n_q, q_starts = 40, [100, 37]
    lens = [q + n_q for q in q_starts]
    sc = Scenario(n_layer=1, n_head=n_head, n_kv=n_kv, head_dim=D, block_tokens=bt, lens=lens,
                  seed=44, pool_byte=0xFF, extra_blocks=6)
    t = sc.tables_host.copy()
    t[0, 1] = 0xFFFF  # keys bt..2bt-1 of sequence 0
    sc.tables = torch.from_numpy(np.ascontiguousarray(t).view(np.int16)).to(device)
    rng = np.random.default_rng(45)
    q = rng.standard_normal((2, n_q, n_head, D)).astype(np.float32)
    qd = torch.from_numpy(q).to(device)
    out = torch.full_like(qd, float("nan"))
    scale = 1 / np.sqrt(D)
    emelk.prefill_chunk(sc.g, sc.k_pool, sc.v_pool, 0, qd, out,
                        torch.tensor(q_starts, dtype=torch.int32, device=device), sc.tables, scale)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    for s_ in range(2):
        kf = oracle.fp16_to_fp32(oracle.fp32_to_fp16(sc.k_rows[0][s_]))
        vf = oracle.fp16_to_fp32(oracle.fp32_to_fp16(sc.v_rows[0][s_]))
        for r in range(n_q):
            limit = q_starts[s_] + r + 1
            keep = np.array([t[s_, p // bt] != 0xFFFF for p in range(limit)])
            qr = oracle.fp16_to_fp32(oracle.fp32_to_fp16(q[s_, r].ravel()))
            want = oracle.attention_f64(qr, kf[:limit][keep], vf[:limit][keep], n_head, n_kv, D,
                                        int(keep.sum()), scale)
            assert_close(got[s_, r].ravel(), want, what=f"D {D} bt {bt} seq {s_} row {r}")
    out2 = torch.full_like(qd, float("nan"))
    emelk.prefill_chunk(sc.g, sc.k_pool, sc.v_pool, 0, qd, out2,
                        torch.tensor([q_starts[0], -3], dtype=torch.int32, device=device),
                        sc.tables, scale)
    torch.cuda.synchronize()
    got2 = out2.cpu().numpy()
    np.testing.assert_array_equal(got2[0], got[0])
    np.testing.assert_array_equal(got2[1], np.zeros_like(got2[1]))


@pytest.mark.parametrize("kv_type,D", [("q8_0", 512), ("q8_0", 128), ("f16", 128)])
def test_prefill_negative_q_start_writes_zero_rows_on_every_route(device, kv_type, D):
    # q8_0 at head_dim 512 runs row by row through the decode kernel; the
    # others on the MFMA prefill kernel.  Each route must treat a negative
    # q_start as a sequence that attends to nothing: zero rows, and the other
    # sequence's rows unchanged.
    import torch
    banner(f"prefill with a negative q_start, {kv_type} D={D}")
    kt = emelk.KV_Q8_0 if kv_type == "q8_0" else emelk.KV_F16
    n_q, q_starts = 12, [40, 20]
    sc = Scenario(n_layer=1, n_head=4, n_kv=1, head_dim=D, block_tokens=16,
                  lens=[q + n_q for q in q_starts], seed=46, kv_type=kt)
    q = np.random.default_rng(47).standard_normal((2, n_q, 4, D)).astype(np.float32)
    qd = torch.from_numpy(q).to(device)
    outs = []
    for starts in (q_starts, [q_starts[0], -3]):
        out = torch.full_like(qd, float("nan"))
        emelk.prefill_chunk(sc.g, sc.k_pool, sc.v_pool, 0, qd, out,
                            torch.tensor(starts, dtype=torch.int32, device=device), sc.tables,
                            1 / np.sqrt(D))
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    assert np.isfinite(outs[0]).all()
    np.testing.assert_array_equal(outs[1][0], outs[0][0])
    np.testing.assert_array_equal(outs[1][1], np.zeros_like(outs[1][1]))


def test_decode_masks_invalid_pages_and_short_tables(device):
    # Tokens on pages marked EMELK_INVALID_KV_BLOCK (0xFFFF), or past the end
    # of the table row, are left out of the softmax instead of being read
    # from an arbitrary page.
    banner("decode with invalid pages in the block table")
    import torch
    sc = Scenario(n_layer=1, n_head=8, n_kv=2, head_dim=128, block_tokens=32,
                  lens=[300, 1000], seed=41)
    t = sc.tables_host.copy()
    t[0, 2] = 0xFFFF          # tokens 64..95 of sequence 0
    t[1, 5] = 0xFFFF          # tokens 160..191 of sequence 1
    t[1, 7] = 0xFFFF          # tokens 224..255
    sc.tables = torch.from_numpy(np.ascontiguousarray(t).view(np.int16)).to(device)
    q = np.random.default_rng(5).standard_normal((2, 8 * 128)).astype(np.float32)
    got = sc.gpu_decode(0, q)
    for s, n in enumerate(sc.lens):
        keep = np.array([t[s, p // 32] != 0xFFFF for p in range(n)])
        k = oracle.fp16_to_fp32(oracle.fp32_to_fp16(sc.k_rows[0][s]))[keep]
        v = oracle.fp16_to_fp32(oracle.fp32_to_fp16(sc.v_rows[0][s]))[keep]
        qr = oracle.fp16_to_fp32(oracle.fp32_to_fp16(q[s]))
        want = oracle.attention_f64(qr, k, v, 8, 2, 128, int(keep.sum()), 1 / np.sqrt(128))
        assert_close(got[s], want, what=f"seq {s} with invalid pages")
    # a kv_len reaching past the table row: only the covered tokens count
    sc2 = Scenario(n_layer=1, n_head=8, n_kv=2, head_dim=128, block_tokens=32, lens=[200],
                   seed=42)
    short = torch.from_numpy(np.ascontiguousarray(sc2.tables_host[:, :4]).view(np.int16)).to(device)
    sc2.tables = short  # covers 128 tokens
    got2 = sc2.gpu_decode(0, q[:1])
    k = oracle.fp16_to_fp32(oracle.fp32_to_fp16(sc2.k_rows[0][0]))[:128]
    v = oracle.fp16_to_fp32(oracle.fp32_to_fp16(sc2.v_rows[0][0]))[:128]
    qr = oracle.fp16_to_fp32(oracle.fp32_to_fp16(q[0]))
    assert_close(got2[0], oracle.attention_f64(qr, k, v, 8, 2, 128, 128, 1 / np.sqrt(128)),
                 what="short table")


@pytest.mark.parametrize("kv_type,n_head,n_kv,D,bt,lens", [
    (emelk.KV_F16, 32, 8, 128, 32, [300, 1000, 37, 1]),
    (emelk.KV_F16, 32, 8, 64, 16, [301, 77, 5]),
    (emelk.KV_F16, 8, 8, 128, 12, [100, 29]),       # block_tokens not a multiple of 8
    (emelk.KV_Q8_0, 32, 8, 128, 32, [300, 1000, 37, 1]),
    (emelk.KV_Q8_0, 16, 8, 128, 16, [333, 18]),
])
def test_decode_never_uses_unwritten_slots(device, kv_type, n_head, n_kv, D, bt, lens):
    """The pool starts as 0xFF bytes (NaN in every never-written f16 slot and
    q8_0 scale): masked tokens past a sequence's end, and tokens on an invalid
    page, must contribute nothing, not 0 * NaN."""
    banner(f"decode over a NaN-filled pool type={kv_type} H={n_head}/{n_kv} D={D} bt={bt} "
           f"lens={lens}")
    import torch
    sc = Scenario(n_layer=1, n_head=n_head, n_kv=n_kv, head_dim=D, block_tokens=bt, lens=lens,
                  seed=sum(lens) + D, kv_type=kv_type, pool_byte=0xFF)
    q = np.random.default_rng(9).standard_normal((sc.n_seq, n_head * D)).astype(np.float32)
    got = sc.gpu_decode(0, q)
    assert_close(got, sc.oracle_decode(0, q), what="NaN-filled pool")
    # an invalid page in the middle of sequence 0: its tokens are left out
    t = sc.tables_host.copy()
    t[0, 1] = 0xFFFF
    sc.tables = torch.from_numpy(np.ascontiguousarray(t).view(np.int16)).to(device)
    got = sc.gpu_decode(0, q)
    n = lens[0]
    keep = np.array([p // bt != 1 for p in range(n)])
    if kv_type == emelk.KV_F16:
        stored = lambda r: oracle.fp16_to_fp32(oracle.fp32_to_fp16(r))  # noqa: E731
    else:
        stored = lambda r: oracle.dequantize_q8_0(oracle.quantize_q8_0(r))  # noqa: E731
    k = stored(sc.k_rows[0][0])[keep]
    v = stored(sc.v_rows[0][0])[keep]
    want = oracle.attention_f64(oracle.fp16_to_fp32(oracle.fp32_to_fp16(q[0])), k, v, n_head,
                                n_kv, D, int(keep.sum()), 1 / np.sqrt(D))
    assert_close(got[0], want, what="NaN-filled pool, invalid page")


def test_decode_graph_replay_matches_eager(device):
    # One layer's append + decode captured in a HIP graph and replayed with
    # eager work and synchronisations in between: every replay must equal
    # the eager result bit for bit.
    banner("decode step in a HIP graph, replayed")
    import torch
    sc = Scenario(n_layer=1, n_head=32, n_kv=8, head_dim=128, block_tokens=32,
                  lens=[2000, 3000], seed=43, extra_blocks=4)
    for s in range(2):
        assert sc.actor.allocate_slots(s, 1)[0]
    sc.refresh_tables()
    pos = torch.tensor(sc.lens, dtype=torch.int32, device=device)
    kl = pos + 1
    newk = torch.randn(2, 1, 1024, device=device)
    newv = torch.randn(2, 1, 1024, device=device)
    q = torch.randn(2, 32, 128, device=device)
    out = torch.zeros_like(q)
    ws = torch.zeros(emelk.decode_workspace_bytes(sc.g, 2, 3001) // 4 + 1, device=device)

    def run():
        emelk.append(sc.g, sc.k_pool, sc.v_pool, 0, newk, newv, pos, sc.tables)
        emelk.decode(sc.g, sc.k_pool, sc.v_pool, 0, q, out, kl, 3001, sc.tables,
                     1 / np.sqrt(128), ws)

    run()
    torch.cuda.synchronize()
    eager = out.clone()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            run()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    for i in range(4):
        out.fill_(float("nan"))
        scratch = torch.randn(1 << 20, device=device) * 2  # unrelated eager work
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i} differs"
        del scratch


# ---- maximum sizes: a sequence spanning EMELK_MAX_BLOCKS_PER_SEQUENCE pages,
# a batch of EMELK_MAX_SEQUENCES sequences ----

@pytest.mark.parametrize("kv_type,n_head,n_kv,D,bt", [
    (emelk.KV_F16, 8, 1, 64, 16),     # 65,536 tokens, 8 query heads per KV head
    (emelk.KV_Q8_0, 4, 1, 128, 32),   # 131,072 tokens
])
def test_decode_at_the_per_sequence_page_limit(device, kv_type, n_head, n_kv, D, bt):
    n = 4096 * bt  # EMELK_MAX_BLOCKS_PER_SEQUENCE pages
    banner(f"decode at the page limit: {n} tokens type={kv_type} D={D} bt={bt}")
    sc = Scenario(n_layer=1, n_head=n_head, n_kv=n_kv, head_dim=D, block_tokens=bt,
                  lens=[n, 700], seed=61, kv_type=kv_type, outlier_frac=0.01)
    assert -(-n // bt) == 4096
    q = np.random.default_rng(62).standard_normal((2, n_head * D)).astype(np.float32)
    got = sc.gpu_decode(0, q)
    assert_close(got, sc.oracle_decode(0, q), what="decode at the page limit")


def test_prefill_at_the_end_of_a_page_limit_sequence(device):
    # 65,536 tokens in 4096 pages; the chunk is the last 40 rows
    banner("prefill chunk of 40 rows after a 65,496-token prefix (4096 pages)")
    _prefill_case(device, 8, 1, 64, 16, [65536 - 40], 40, seed=63)


def test_decode_at_the_sequence_limit(device):
    banner("decode of EMELK_MAX_SEQUENCES = 256 sequences, ragged")
    lens = np.random.default_rng(64).integers(1, 300, size=256).tolist()
    sc = Scenario(n_layer=1, n_head=8, n_kv=2, head_dim=64, block_tokens=16, lens=lens, seed=65)
    q = np.random.default_rng(66).standard_normal((256, 8 * 64)).astype(np.float32)
    got = sc.gpu_decode(0, q)  # one split per sequence: no combine kernel runs
    assert_close(got, sc.oracle_decode(0, q), what="256 sequences")
    # a sequence given no token to attend gets a zero output
    lens0 = list(lens)
    lens0[7] = 0
    got0 = sc.gpu_decode(0, q, lens=lens0)
    assert np.all(got0[7] == 0.0)
    keep = [s for s in range(256) if s != 7]
    np.testing.assert_array_equal(got0[keep], got[keep])


Q8_PREFILL_CASES = [
    # n_head, n_kv, D, bt, q_starts, n_q, invalid page (seq, page) or None
    (16, 4, 128, 32, [0, 100, 1000], 37, None),   # uniform 32-key sub-tiles
    (8, 2, 128, 16, [33, 5], 70, None),           # general staging (pages of 16)
    (8, 8, 64, 32, [64], 33, None),               # G=1, D=64
    (16, 2, 64, 8, [19, 0], 40, None),            # G=8, pages of 8
    (8, 2, 128, 32, [100, 37], 40, (0, 1)),       # NaN-filled pool, an invalid page
    (8, 2, 128, 16, [100, 37], 40, (1, 2)),
    (8, 1, 256, 16, [40], 9, None),               # head_dim 256: 4 waves, 32-key tiles
    (8, 2, 256, 32, [70, 3], 36, (0, 1)),         # head_dim 256, NaN pool, invalid page
    (8, 1, 512, 16, [30], 11, None),              # head_dim 512: row by row
]


@pytest.mark.parametrize("case", Q8_PREFILL_CASES, ids=[f"q8p{i}" for i in range(len(Q8_PREFILL_CASES))])
def test_prefill_chunk_q8_0(device, case):
    """q8_0 pools on the MFMA prefill kernel: K is dequantized while staged
    into two fp16 planes whose sum is exactly q * d, V into fp16(q * d) (one
    rounding of the exact product), checked against
    the oracle's q8_0 route of the reference's per-row loop and against the
    fp64 ideal over the dequantized values.  With pool_byte 0xFF every
    never-written scale is an fp16 NaN, so a slot past a sequence's end (or
    on an invalid page) that reached the softmax or P.V would poison rows."""
    import torch
    n_head, n_kv, D, bt, q_starts, n_q, bad = case
    banner(f"q8_0 prefill chunk H={n_head}/{n_kv} D={D} bt={bt} starts={q_starts} n_q={n_q} "
           f"invalid={bad}")
    lens = [s + n_q for s in q_starts]
    sc = Scenario(n_layer=1, n_head=n_head, n_kv=n_kv, head_dim=D, block_tokens=bt, lens=lens,
                  seed=71, kv_type=emelk.KV_Q8_0, outlier_frac=0.01,
                  pool_byte=0xFF if bad else 0, extra_blocks=6 if bad else 3)
    t = sc.tables_host.copy()
    if bad:
        t[bad[0], bad[1]] = 0xFFFF
        sc.tables = torch.from_numpy(np.ascontiguousarray(t).view(np.int16)).to(device)
    rng = np.random.default_rng(72)
    q = rng.standard_normal((sc.n_seq, n_q, n_head, D)).astype(np.float32)
    qd = torch.from_numpy(q).to(device)
    out = torch.full_like(qd, float("nan"))
    qs = torch.tensor(q_starts, dtype=torch.int32, device=device)
    scale = 1.0 / np.sqrt(D)
    emelk.prefill_chunk(sc.g, sc.k_pool, sc.v_pool, 0, qd, out, qs, sc.tables, scale)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    kc, vc = sc.oracle_cache(0)
    for s in range(sc.n_seq):
        kq = oracle.dequantize_q8_0(oracle.quantize_q8_0(sc.k_rows[0][s]))
        vq = oracle.dequantize_q8_0(oracle.quantize_q8_0(sc.v_rows[0][s]))
        for r in range(n_q):
            limit = q_starts[s] + r + 1  # row r attends causally to [0, q_start + r]
            qr = oracle.fp16_to_fp32(oracle.fp32_to_fp16(q[s, r].ravel()))
            if bad is None:
                want = oracle.compute_attention_q8_0(q[s, r].ravel(), kc, vc, sc.tables_host[s],
                                                     bt, n_head, n_kv, D, limit, limit, scale)
                assert_close(got[s, r].ravel(), want, what=f"q8_0 prefill seq {s} row {r}")
                keep = np.ones(limit, bool)
            else:
                keep = np.array([t[s, p // bt] != 0xFFFF for p in range(limit)])
            kk, vv, n = kq[:limit][keep], vq[:limit][keep], int(keep.sum())
            ideal = oracle.attention_f64(qr, kk, vv, n_head, n_kv, D, n, scale)
            # beyond the bar, the fp16 rounding of P (the reference's rounded
            # probabilities) and of the dequantized V, each <= 2^-11 of
            # sum_p p |v|: with x20 outliers that sum dwarfs a cancelling output
            mag = oracle.attention_f64(qr, kk, np.abs(vv), n_head, n_kv, D, n, scale)
            assert_close(got[s, r].ravel(), ideal, atol=2e-3 + 2.0 ** -10 * np.asarray(mag),
                         what=f"q8_0 prefill seq {s} row {r} vs ideal")


# ---- head_dim 256 and 512 (Gemma-4-sized heads: key_length 512, 256 on
# sliding-window layers, src/emel/model/gemma4/detail.cpp:26-29) ----

@pytest.mark.parametrize("kv_type,n_head,n_kv,D,bt,lens", [
    (emelk.KV_F16, 8, 2, 256, 16, [300, 1, 1025]),
    (emelk.KV_F16, 8, 1, 512, 32, [700, 33]),
    (emelk.KV_Q8_0, 8, 2, 256, 32, [513, 64]),
    (emelk.KV_Q8_0, 4, 4, 512, 16, [129, 3000]),
])
def test_decode_large_heads(device, kv_type, n_head, n_kv, D, bt, lens):
    banner(f"decode large heads type={kv_type} H={n_head}/{n_kv} D={D} bt={bt} lens={lens}")
    sc = Scenario(n_layer=1, n_head=n_head, n_kv=n_kv, head_dim=D, block_tokens=bt, lens=lens,
                  seed=sum(lens) + D, kv_type=kv_type, outlier_frac=0.01)
    _decode_case(sc, 0, 800 + D)


def test_decode_append_large_heads(device):
    import torch
    banner("decode_append at head_dim 256 (f16) and 512 (q8_0)")
    for kv_type, D in ((emelk.KV_F16, 256), (emelk.KV_Q8_0, 512)):
        sc = Scenario(n_layer=1, n_head=8, n_kv=2, head_dim=D, block_tokens=16, lens=[47, 200],
                      seed=D, extra_blocks=4, kv_type=kv_type)
        for s in range(sc.n_seq):
            assert sc.actor.allocate_slots(s, 1)[0]
        sc.refresh_tables()
        rng = np.random.default_rng(D + 1)
        nk = rng.standard_normal((sc.n_seq, sc.kv_dim)).astype(np.float32)
        nv = rng.standard_normal((sc.n_seq, sc.kv_dim)).astype(np.float32)
        q = rng.standard_normal((sc.n_seq, 8 * D)).astype(np.float32)
        lens_now = [n + 1 for n in sc.lens]
        kl = torch.tensor(lens_now, dtype=torch.int32, device=device)
        ws = torch.zeros(emelk.decode_workspace_bytes(sc.g, sc.n_seq, max(lens_now)) // 4 + 1,
                         device=device)
        out = torch.full((sc.n_seq, 8, D), float("nan"), device=device)
        emelk.decode_append(sc.g, sc.k_pool, sc.v_pool, 0, torch.from_numpy(nk).to(device),
                            torch.from_numpy(nv).to(device),
                            torch.from_numpy(q).to(device).view(sc.n_seq, 8, D), out, kl,
                            max(lens_now), sc.tables, float(1 / np.sqrt(D)), ws)
        torch.cuda.synchronize()
        for s in range(sc.n_seq):
            sc.k_rows[0][s] = np.concatenate([sc.k_rows[0][s], nk[s][None]])
            sc.v_rows[0][s] = np.concatenate([sc.v_rows[0][s], nv[s][None]])
        sc.lens = lens_now
        assert_close(out.view(sc.n_seq, -1).cpu().numpy(), sc.oracle_decode(0, q),
                     what=f"decode_append D={D}")
        for which, pool in (("k", sc.k_pool), ("v", sc.v_pool)):
            np.testing.assert_array_equal(pool.cpu().numpy(), sc.expected_pool(which),
                                          err_msg=f"{which} pool D={D}")


@pytest.mark.parametrize("n_head,n_kv,bt,q_starts,n_q", [
    (8, 2, 16, [0, 130], 21),      # G=4, general staging (pages of 16)
    (8, 8, 32, [33], 70),          # G=1: 4 row blocks per workgroup
    (8, 4, 32, [100, 0], 45),      # G=2
    (16, 2, 32, [64], 40),         # G=8: two workgroups per KV head
])
def test_prefill_chunk_head_dim_256(device, n_head, n_kv, bt, q_starts, n_q):
    """head_dim 256 (Gemma-4 sliding-window layers) on the MFMA kernel: 4
    waves per workgroup, 32-key tiles."""
    banner(f"prefill chunk at head_dim 256 H={n_head}/{n_kv} bt={bt} starts={q_starts} n_q={n_q}")
    _prefill_case(device, n_head, n_kv, 256, bt, q_starts, n_q, seed=81)


@pytest.mark.parametrize("n_head,n_kv,bt,q_starts,n_q", [
    (8, 2, 16, [0, 70], 13),       # G=4, general staging
    (8, 1, 32, [40], 50),          # G=8 (Gemma-4 global layers): two workgroups per row block
    (4, 4, 32, [9, 100], 35),      # G=1: 4 row blocks per workgroup
    (8, 4, 32, [64], 20),          # G=2
])
def test_prefill_chunk_head_dim_512(device, n_head, n_kv, bt, q_starts, n_q):
    """head_dim 512 on the MFMA kernel with 16 query rows per wave
    (v_mfma_f32_16x16x32_f16), 4 waves per workgroup."""
    banner(f"prefill chunk at head_dim 512 H={n_head}/{n_kv} bt={bt} starts={q_starts} n_q={n_q}")
    _prefill_case(device, n_head, n_kv, 512, bt, q_starts, n_q, seed=82)


def test_decode_straight_from_the_device_view(device):
    """emelk_kv_cache_upload_view puts the actor's capture_view snapshot in
    device memory byte for byte; its length values and block rows then serve
    as kv_lens and block_tables (stride MAX_BLOCKS_PER_SEQUENCE), and decode
    from them is bit-identical to decode from the exported tables."""
    import ctypes
    import torch
    banner("decode from the device snapshot (capture_view uploaded)")
    sc = Scenario(n_layer=2, n_head=8, n_kv=2, head_dim=128, block_tokens=32,
                  lens=[300, 77, 1000], seed=91)
    cache = emelk.KvCache(sc.g)
    view_dev = torch.zeros(ctypes.sizeof(emelk.Snapshot), dtype=torch.uint8, device=device)
    cache.upload_view(sc.actor, view_dev)
    torch.cuda.synchronize()
    host = emelk.Snapshot()
    ok, err = sc.actor.capture_view(host)
    assert ok and err == 0
    want = np.frombuffer(bytes(host), dtype=np.uint8)
    np.testing.assert_array_equal(view_dev.cpu().numpy(), want)
    lens, tables = emelk.KvCache.view_fields(view_dev, sc.n_seq)
    rng = np.random.default_rng(92)
    q = torch.from_numpy(rng.standard_normal((sc.n_seq, 8 * 128)).astype(np.float32)).to(device)
    ws = torch.empty(emelk.decode_workspace_bytes(sc.g, sc.n_seq, 1000), dtype=torch.uint8,
                     device=device)
    a = torch.full_like(q, float("nan"))
    b = torch.full_like(q, float("nan"))
    emelk.decode(sc.g, sc.k_pool, sc.v_pool, 1, q, a, lens, 1000, tables, 1 / np.sqrt(128), ws)
    exp_lens = torch.tensor(sc.lens, dtype=torch.int32, device=device)
    emelk.decode(sc.g, sc.k_pool, sc.v_pool, 1, q, b, exp_lens, 1000, sc.tables, 1 / np.sqrt(128),
                 ws)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(a.cpu().numpy(), b.cpu().numpy())
    assert np.isfinite(a.cpu().numpy()).all()
    cache.close()


@pytest.mark.parametrize("kv_type", [emelk.KV_F16, emelk.KV_Q8_0])
def test_prefill_config5_full_size_sampled_rows(device, kv_type):
    """The config-5 chunk at its full size: 8 sequences x (4096 cached + 512
    new rows), Llama-3-8B heads, 32-token pages on a seeded permutation.
    One layer runs on the GPU, and 24 seeded (sequence, row) samples, first
    and last rows included, are checked against the oracle's per-row route."""
    import torch
    banner(f"prefill chunk at the full config-5 size, kv_type={kv_type}")
    P0, NQ, B = 4096, 512, 8
    sc = Scenario(n_layer=1, n_head=32, n_kv=8, head_dim=128, block_tokens=32,
                  lens=[P0 + NQ] * B, seed=101, kv_type=kv_type,
                  outlier_frac=0.01 if kv_type == emelk.KV_Q8_0 else 0.0)
    rng = np.random.default_rng(102)
    q = rng.standard_normal((B, NQ, 32, 128)).astype(np.float32)
    qd = torch.from_numpy(q).to(device)
    out = torch.full_like(qd, float("nan"))
    qs = torch.full((B,), P0, dtype=torch.int32, device=device)
    scale = 1.0 / np.sqrt(128)
    emelk.prefill_chunk(sc.g, sc.k_pool, sc.v_pool, 0, qd, out, qs, sc.tables, scale)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    kc, vc = sc.oracle_cache(0)
    route = oracle.compute_attention_f16 if kv_type == emelk.KV_F16 else \
        oracle.compute_attention_q8_0
    samples = [(0, 0), (B - 1, NQ - 1)] + [(int(rng.integers(B)), int(rng.integers(NQ)))
                                           for _ in range(22)]
    for s, r in samples:
        limit = P0 + r + 1
        want = route(q[s, r].ravel(), kc, vc, sc.tables_host[s], 32, 32, 8, 128, limit, limit,
                     scale)
        assert_close(got[s, r].ravel(), want, what=f"seq {s} row {r}")
