"""GPU parity at the configs' production batches: one full layer of the
decode step (emelk_attn_decode_append: store the token at position
kv_lens - 1, then attend over kv_lens tokens) at the batch size, context and
page size of BASELINE configs 2, 3 and 4, so the launch runs the split plan
the bench runs (config 3: 64 sequences, about 4 splits each; config 2: 16
ragged sequences on the balanced device plan; config 4: 32 q8_0 sequences of
16385 tokens).  Every output row is checked against the oracle's reference
route (compute_attention, text/generator/detail.hpp:3153-3230; the q8_0
route for q8_0 pools) at the 2e-3 abs + 1e-2 rel bar, and the stored
token's bytes against the oracle's fp16 rounding / q8_0 quantizer
(bit-exact).  Pools are filled on the device (f16: torch's normal_; q8_0:
N(0,1) rows with 1% x20 outliers through the append kernel, whose bytes
other tests pin), then read back for the oracle."""
import numpy as np
import pytest

import emelk
import oracle
from kvsetup import assert_close, banner, pool_token_major

pytestmark = pytest.mark.gpu

# (label, n_head, n_kv, D, bt, kv_type, batch, ctx lengths before the step)
CASES = [
    ("config3_llama3-8b_b64_ctx8k", 32, 8, 128, 32, "f16", 64, "8192"),
    ("config2_llama3.2-1b_b16_ragged", 32, 8, 64, 16, "f16", 16, "U[1024,4096]"),
    ("config4_llama3-8b_q8_0_b32_ctx16k", 32, 8, 128, 32, "q8_0", 32, "16384"),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_decode_append_full_batch_matches_reference_route(device, case):
    import torch
    label, H, HK, D, BT, kvt, B, ctx_spec = case
    banner(f"production batch {label}: {B} sequences, ctx {ctx_spec}, {kvt}")
    q8 = kvt == "q8_0"
    rng = np.random.default_rng(20260)
    if ctx_spec.startswith("U"):
        ctx = rng.integers(1024, 4097, size=B).astype(np.int64)
    else:
        ctx = np.full(B, int(ctx_spec), np.int64)
    lens = ctx + 1
    pages_per_seq = -(-lens // BT)
    max_blocks = int(pages_per_seq.sum()) + 1
    actor = emelk.KvActor()
    assert actor.reserve(B, max_blocks, BT)[0]
    actor.set_free_order(rng.permutation(max_blocks).astype(np.uint16))
    for s in range(B):
        assert actor.allocate_sequence(s)[0]
        assert actor.allocate_slots(s, int(ctx[s]))[0]
    for s in range(B):
        assert actor.allocate_slots(s, 1)[0]  # the step's slot
    stride = int(pages_per_seq.max()) + 1
    tables_h = actor.export_block_tables(list(range(B)), stride)
    tables = torch.from_numpy(tables_h.view(np.int16)).to(device)
    g = emelk.geometry(1, H, HK, D, BT, max_blocks, emelk.KV_Q8_0 if q8 else emelk.KV_F16)
    pb = emelk.pool_bytes(g)
    k_pool = torch.zeros(pb, dtype=torch.uint8, device=device)
    v_pool = torch.zeros(pb, dtype=torch.uint8, device=device)
    gen = torch.Generator(device=device)
    gen.manual_seed(20261)
    if q8:
        for s0 in range(0, B, 4):
            s1 = min(B, s0 + 4)
            n = int(ctx.max())
            rows = []
            for _ in range(2):
                x = torch.randn((s1 - s0, n, HK * D), generator=gen, device=device)
                x = torch.where(torch.rand(x.shape, generator=gen, device=device) < 0.01,
                                x * 20.0, x)
                rows.append(x)
            emelk.append(g, k_pool, v_pool, 0, rows[0], rows[1],
                         torch.zeros(s1 - s0, dtype=torch.int32, device=device), tables[s0:s1])
            del rows
    else:
        k_pool.view(torch.float16).normal_(generator=gen)
        v_pool.view(torch.float16).normal_(generator=gen)
    q = torch.randn((B, H, D), generator=gen, device=device) / np.sqrt(D)
    new_k = torch.randn((B, HK * D), generator=gen, device=device)
    new_v = torch.randn((B, HK * D), generator=gen, device=device)
    if q8:
        for t in (new_k, new_v):
            t[torch.rand(t.shape, generator=gen, device=device) < 0.01] *= 20.0
    out = torch.full((B, H, D), float("nan"), dtype=torch.float32, device=device)
    kv_lens = torch.from_numpy(lens.astype(np.int32)).to(device)
    max_len = int(lens.max())
    ws = torch.zeros(emelk.decode_workspace_bytes(g, B, max_len) // 4 + 1, dtype=torch.float32,
                     device=device)
    plan = emelk.decode_plan(g, B, max_len)
    scale = float(1.0 / np.sqrt(D))
    emelk.decode_append(g, k_pool, v_pool, 0, new_k, new_v, q, out, kv_lens, max_len, tables,
                        scale, ws)
    torch.cuda.synchronize()
    got = out.view(B, H * D).cpu().numpy()
    assert np.isfinite(got).all()
    kc, vc = (pool_token_major(p, 0, 1, max_blocks, HK, BT, D, q8) for p in (k_pool, v_pool))
    # the stored token, bit-exact
    nk, nv = new_k.cpu().numpy(), new_v.cpu().numpy()
    phys = tables_h[np.arange(B), ctx // BT].astype(np.int64) * BT + ctx % BT
    for cache, rows in ((kc, nk), (vc, nv)):
        want = oracle.quantize_q8_0(rows) if q8 else oracle.fp32_to_fp16(rows)
        np.testing.assert_array_equal(cache[phys].view(np.uint8), want.view(np.uint8))
    # every sequence against the reference route
    want, _secs = oracle.attention_rows(kvt, q.view(B, H * D).cpu().numpy(), kc, vc, tables_h,
                                        lens.astype(np.int32), BT, H, HK, D, scale, 16)
    err = assert_close(got, want, what=f"{label} vs reference route")
    print(f"[gpu-case] {label}: max abs err {err:.3e} over {B} sequences, plan {plan}",
          flush=True)
