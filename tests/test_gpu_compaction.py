"""Eviction + compaction at the full config-5 geometry, bit-exact.

Config 5: Llama-3-8B KV shape (32 layers, 8 KV heads, head_dim 128,
32-token pages), 8 sequences of 4096 cached + 512 chunk tokens (144 pages
each); a seeded 25% of each sequence's pages is evicted and the survivors
are compacted to the front of the pool by the actor's move list, applied
with one emelk_kv_copy_blocks launch.  The reference's page move is
copy_attention_kv_block (src/emel/text/generator/detail.hpp:3334-3417).

Every byte of both pools is checked: the pool after the launch must equal
the pool before with each listed destination page replaced by its source
page (built independently with torch indexing on the device), and every
sequence must read, through its new block table, exactly the bytes it read
through its old one for the pages it kept."""
import numpy as np
import pytest

import emelk
from kvsetup import banner

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kv_type", [emelk.KV_F16, emelk.KV_Q8_0], ids=["f16", "q8_0"])
def test_compaction_config5_full_size_bit_exact(device, kv_type):
    import torch
    L, HK, D, BT, B, P0, NQ = 32, 8, 128, 32, 8, 4096, 512
    pages = (P0 + NQ) // BT
    max_blocks = B * pages + 1
    banner(f"compaction config5 full size kv_type={kv_type}: {B} x {pages} pages, {L} layers")
    rng = np.random.default_rng(5)
    actor = emelk.KvActor()
    assert actor.reserve(B, max_blocks, BT)[0]
    actor.set_free_order(rng.permutation(max_blocks).astype(np.uint16))
    for s in range(B):
        assert actor.allocate_sequence(s)[0]
        assert actor.allocate_slots(s, P0)[0]
    for s in range(B):
        assert actor.allocate_slots(s, NQ)[0]
    old_tables = actor.export_block_tables(list(range(B)), pages).astype(np.int64)
    g = emelk.geometry(L, 32, HK, D, BT, max_blocks, kv_type)
    pb = emelk.pool_bytes(g)
    page_bytes = pb // (L * max_blocks)
    gen = torch.Generator(device=device)
    gen.manual_seed(55)
    pools = [torch.randint(0, 256, (pb,), dtype=torch.uint8, device=device, generator=gen)
             for _ in range(2)]
    before = [p.clone() for p in pools]

    kept = []
    for s in range(B):
        ev = sorted(rng.choice(pages, size=pages // 4, replace=False).tolist())
        ok, err, removed = actor.evict_blocks(s, ev)
        assert ok and err == 0, (s, err)
        kept.append([lb for lb in range(pages) if lb not in set(ev)])
    ok, err, moves = actor.compact()
    assert ok and err == 0
    moves = np.asarray(moves, np.int64).reshape(-1, 2)
    n_live = sum(len(k) for k in kept)
    assert len(moves) > 0
    # survivors end at the front of the pool; sources and destinations disjoint
    assert set(moves[:, 1]).isdisjoint(set(moves[:, 0]))
    assert moves[:, 1].max() < n_live and moves[:, 0].min() >= n_live
    print(f"[gpu-case] {len(moves)} page moves x {L} layers x K,V; page {page_bytes} B", flush=True)

    emelk.copy_blocks(g, pools[0], pools[1],
                      torch.from_numpy(moves.astype(np.int32)).to(device))
    torch.cuda.synchronize()

    src = torch.from_numpy(moves[:, 0]).to(device)
    dst = torch.from_numpy(moves[:, 1]).to(device)
    new_tables = actor.export_block_tables(list(range(B)), pages).astype(np.int64)
    for which in range(2):
        got = pools[which].view(L, max_blocks, page_bytes)
        want = before[which].view(L, max_blocks, page_bytes).clone()
        want[:, dst] = before[which].view(L, max_blocks, page_bytes)[:, src]
        assert torch.equal(got, want), f"pool {'KV'[which]}: bytes differ from the move list"
        del want
        b = before[which].view(L, max_blocks, page_bytes)
        for s in range(B):
            k = np.asarray(kept[s])
            assert (new_tables[s, :len(k)] != 0xFFFF).all()
            oldp = torch.from_numpy(old_tables[s, k]).to(device)
            newp = torch.from_numpy(new_tables[s, :len(k)]).to(device)
            assert torch.equal(got[:, newp], b[:, oldp]), f"seq {s} pool {'KV'[which]}"
    del before
