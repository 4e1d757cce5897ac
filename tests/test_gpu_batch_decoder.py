"""GPU test of the multi-sequence step executor (emelk_batch_decoder) against
the reference's per-token flow restated by the oracle: norm + RoPE of the
projection rows at each token's position, the store, and attention over the
sequence's whole history (compute_layer_attention_residual,
text/generator/detail.hpp:3745-3840), for several sequences at once,
including a branch whose shared tail page is split on the device."""
import numpy as np
import pytest

import emelk
import oracle
from kvsetup import assert_close

pytestmark = pytest.mark.gpu

H, HKV, D, BT, L = 8, 2, 128, 16, 2
BASE = 1e4
SCALE = 1.0 / np.sqrt(D)


def banner(msg):
    print(f"\n[gpu-case] {msg}", flush=True)


def f16r(x):
    return oracle.fp16_to_fp32(oracle.fp32_to_fp16(np.asarray(x, np.float32)))


def q8r(x):
    x = np.asarray(x, np.float32)
    return oracle.dequantize_q8_0(oracle.quantize_q8_0(x.reshape(-1, x.shape[-1]))).reshape(x.shape)


class Model:
    """Oracle side: per sequence and layer, the stored (roped) K and V rows."""

    def __init__(self, kv_type=emelk.KV_F16):
        self.k = {}
        self.v = {}
        self.stored = f16r if kv_type == emelk.KV_F16 else q8r

    def ensure(self, seq):
        self.k.setdefault(seq, [[] for _ in range(L)])
        self.v.setdefault(seq, [[] for _ in range(L)])

    def branch(self, parent, child):
        self.k[child] = [list(x) for x in self.k[parent]]
        self.v[child] = [list(x) for x in self.v[parent]]

    def token(self, seq, layer, q, k, v, pos, qn, kn):
        qo, ko, vo = oracle.qkv_rope_rows(q, k, v, H, HKV, D, emelk.NEOX_PAIRING, D, BASE, pos,
                                          q_norm=qn, k_norm=kn, eps=1e-6)
        assert len(self.k[seq][layer]) == pos
        self.k[seq][layer].append(ko)
        self.v[seq][layer].append(vo)
        kk = self.stored(np.stack(self.k[seq][layer]))
        vv = self.stored(np.stack(self.v[seq][layer]))
        return oracle.attention_f64(f16r(qo), kk, vv, H, HKV, D, pos + 1, SCALE)


@pytest.mark.parametrize("kv_type", [emelk.KV_F16, emelk.KV_Q8_0])
def test_batch_decoder_prefill_decode_and_branch(device, kv_type):
    import torch
    banner(f"batch decoder: prefill, decode, branch with device tail split, kv_type={kv_type}")
    rng = np.random.default_rng(7)
    g = emelk.geometry(L, H, HKV, D, BT, 96, kv_type)
    actor = emelk.KvActor()
    assert actor.reserve(8, 96, BT)[0]
    actor.set_free_order(rng.permutation(96).astype(np.uint16))
    for s in range(3):
        assert actor.allocate_sequence(s)[0]
    cache = emelk.KvCache(g)
    rope = emelk.RopeTable(D, D, 512, BASE, emelk.NEOX_PAIRING)
    dec = emelk.BatchDecoder(g, actor, cache, rope, max_batch=4, max_kv_len=300)
    qn = rng.standard_normal(D).astype(np.float32)
    kn = rng.standard_normal(D).astype(np.float32)
    qn_d = torch.from_numpy(qn).to(device)
    kn_d = torch.from_numpy(kn).to(device)
    model = Model(kv_type)
    for s in range(3):
        model.ensure(s)

    def step(ids, n_tokens, what):
        pos = dec.begin_step(ids, n_tokens)
        for i, s in enumerate(ids):
            assert pos[i] == len(model.k[s][0]), f"{what}: position of seq {s}"
        n = len(ids)
        for layer in range(L):
            q = rng.standard_normal((n, n_tokens, H * D)).astype(np.float32)
            k = rng.standard_normal((n, n_tokens, HKV * D)).astype(np.float32)
            v = rng.standard_normal((n, n_tokens, HKV * D)).astype(np.float32)
            qd = torch.from_numpy(q).to(device)
            out = torch.full((n, n_tokens, H * D), float("nan"), device=device)
            dec.layer(layer, qd, qd, torch.from_numpy(k).to(device),
                      torch.from_numpy(v).to(device), out, SCALE, q_norm=qn_d, k_norm=kn_d)
            torch.cuda.synchronize()
            got = out.cpu().numpy()
            for i, s in enumerate(ids):
                for t in range(n_tokens):
                    want = model.token(s, layer, q[i, t], k[i, t], v[i, t], pos[i] + t, qn, kn)
                    assert_close(got[i, t], want,
                                 what=f"{what} layer {layer} seq {s} token {pos[i] + t}")

    step([0, 1, 2], 20, "prefill")
    step([0, 1, 2], 1, "decode 1")
    step([2, 0, 1], 1, "decode 2")           # any order of sequences
    # branch mid-page: seq 1 has 22 tokens, its second page is shared and
    # partly filled, so the first append of either branch splits it on the device
    assert actor.branch_sequence(1, 3)[0]
    model.branch(1, 3)
    model.ensure(3)
    step([1, 3], 1, "after branch 1")
    step([3, 1], 1, "after branch 2")
    step([0, 2], 5, "prefill chunk on the others")
    step([0, 1, 2, 3], 1, "all four")
    dec.close()


def test_batch_decoder_step_is_all_or_nothing(device):
    banner("batch decoder: a refused sequence rolls the step back")
    g = emelk.geometry(1, H, HKV, D, BT, 6, emelk.KV_F16)
    actor = emelk.KvActor()
    assert actor.reserve(4, 6, BT)[0]
    for s in range(2):
        assert actor.allocate_sequence(s)[0]
    cache = emelk.KvCache(g)
    rope = emelk.RopeTable(D, D, 256, BASE)
    dec = emelk.BatchDecoder(g, actor, cache, rope, max_batch=2, max_kv_len=200)
    dec.begin_step([0, 1], 40)               # 3 pages each: the pool of 6 is full
    dec.begin_step([1], 8)                   # seq 1: 48 tokens, its last page full
    free_before = emelk.lib.emelk_kv_free_count(actor.handle)
    assert free_before == 0
    with pytest.raises(RuntimeError):
        dec.begin_step([0, 1], 4)            # seq 0 fits in its tail page, seq 1 does not
    assert emelk.lib.emelk_kv_sequence_length(actor.handle, 0) == 40
    assert emelk.lib.emelk_kv_sequence_length(actor.handle, 1) == 48
    assert emelk.lib.emelk_kv_free_count(actor.handle) == free_before
    dec.close()


def test_batch_decoder_requires_the_cache_stream(device):
    """Tail-split page copies run on the cache's stream, so a decoder on any
    other stream would race them: creation is refused."""
    import torch
    banner("batch decoder: stream must be the cache's")
    g = emelk.geometry(1, H, HKV, D, BT, 8, emelk.KV_F16)
    actor = emelk.KvActor()
    assert actor.reserve(2, 8, BT)[0]
    cache = emelk.KvCache(g)
    rope = emelk.RopeTable(D, D, 64, BASE)
    other = torch.cuda.Stream()
    assert (emelk.lib.emelk_kv_cache_stream(cache.handle) or 0) == \
        torch.cuda.current_stream().cuda_stream
    with pytest.raises(RuntimeError):
        emelk.BatchDecoder(g, actor, cache, rope, max_batch=2, max_kv_len=64,
                           stream=other.cuda_stream)


@pytest.mark.parametrize("kv_type", [emelk.KV_F16, emelk.KV_Q8_0])
def test_batch_decoder_runs_an_equal_plan(device, kv_type):
    """Prompts of three sequences, their tokens interleaved in one batch,
    planned by the batch planner in equal mode (the same number of tokens
    from every sequence of a step, each sequence's tokens in order) and run
    step by step through the executor: each step's (sequences, tokens per
    sequence) is emelk_plan_step_sequences of the plan."""
    import torch
    banner(f"batch decoder driven by an equal-mode plan, kv_type={kv_type}")
    rng = np.random.default_rng(11)
    lens = [13, 7, 20]
    ids = np.concatenate([np.full(n, s, np.int32) for s, n in enumerate(lens)])
    rng.shuffle(ids)
    n = len(ids)
    plan = emelk.BatchPlan(rng.integers(0, 32000, size=n).astype(np.int32), n_steps=9,
                           mode=emelk.PLAN_EQUAL, seq_primary_ids=ids, equal_sequential=False,
                           output_all=True)
    assert plan.accepted, plan.error
    g = emelk.geometry(L, H, HKV, D, BT, 32, kv_type)
    actor = emelk.KvActor()
    assert actor.reserve(4, 32, BT)[0]
    actor.set_free_order(rng.permutation(32).astype(np.uint16))
    for s in range(3):
        assert actor.allocate_sequence(s)[0]
    cache = emelk.KvCache(g)
    rope = emelk.RopeTable(D, D, 64, BASE, emelk.NEOX_PAIRING)
    dec = emelk.BatchDecoder(g, actor, cache, rope, max_batch=3, max_kv_len=64)
    model = Model(kv_type)
    for s in range(3):
        model.ensure(s)
    # per token and layer: the projection rows
    q = rng.standard_normal((L, n, H * D)).astype(np.float32)
    k = rng.standard_normal((L, n, HKV * D)).astype(np.float32)
    v = rng.standard_normal((L, n, HKV * D)).astype(np.float32)
    shapes = []
    for step, tokens in enumerate(plan.steps):
        seqs, per = plan.step_sequences(step)
        shapes.append((tuple(seqs), per))
        pos = dec.begin_step(seqs, per)
        order = np.array(tokens).reshape(len(seqs), per)
        for i, s in enumerate(seqs):
            assert pos[i] == len(model.k[s][0])
            assert all(ids[t] == s for t in order[i])
        for layer in range(L):
            qd = torch.from_numpy(q[layer][order]).to(device)
            out = torch.full(qd.shape, float("nan"), device=device)
            dec.layer(layer, qd, qd, torch.from_numpy(k[layer][order]).to(device),
                      torch.from_numpy(v[layer][order]).to(device), out, SCALE)
            torch.cuda.synchronize()
            got = out.cpu().numpy()
            for i, s in enumerate(seqs):
                for j, t in enumerate(order[i]):
                    want = model.token(s, layer, q[layer, t], k[layer, t], v[layer, t],
                                       pos[i] + j, None, None)
                    assert_close(got[i, j], want, what=f"step {step} layer {layer} seq {s} tok {t}")
    assert [len(model.k[s][0]) for s in range(3)] == lens
    # the plan mixes multi-sequence prefill steps with steps of other shapes
    assert any(len(sq) == 3 for sq, _ in shapes) and any(p > 1 for _, p in shapes)
    dec.close()


def test_batch_decoder_decode_layers_replay_as_a_graph(device):
    """With graph-stable launches, one decode step's layer calls are captured
    in a HIP graph once and replayed for later steps: begin_step refreshes
    the device tables, positions and lengths outside the graph.  Every
    replay is checked against the oracle's per-token flow, with host work
    and synchronisation between replays."""
    import torch
    banner("batch decoder: decode layers captured once, replayed over steps")
    rng = np.random.default_rng(21)
    g = emelk.geometry(L, H, HKV, D, BT, 64, emelk.KV_F16)
    actor = emelk.KvActor()
    assert actor.reserve(4, 64, BT)[0]
    actor.set_free_order(rng.permutation(64).astype(np.uint16))
    ids = [0, 1, 2]
    for s in ids:
        assert actor.allocate_sequence(s)[0]
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        cache = emelk.KvCache(g, stream=side.cuda_stream)
        rope = emelk.RopeTable(D, D, 256, BASE, emelk.NEOX_PAIRING, stream=side.cuda_stream)
        dec = emelk.BatchDecoder(g, actor, cache, rope, max_batch=3, max_kv_len=200,
                                 stream=side.cuda_stream)
        dec.set_fixed_plan(True)
        model = Model()
        for s in ids:
            model.ensure(s)
        n = len(ids)
        # static buffers the graph reads and writes
        qb = torch.zeros((L, n, 1, H * D), device=device)
        kb = torch.zeros((L, n, 1, HKV * D), device=device)
        vb = torch.zeros((L, n, 1, HKV * D), device=device)
        qr = torch.zeros_like(qb)
        ob = torch.zeros_like(qb)

        def fill(step_rows):
            for layer in range(L):
                q, k, v = step_rows[layer]
                qb[layer].copy_(torch.from_numpy(q).view(n, 1, -1))
                kb[layer].copy_(torch.from_numpy(k).view(n, 1, -1))
                vb[layer].copy_(torch.from_numpy(v).view(n, 1, -1))

        def layers():
            for layer in range(L):
                dec.layer(layer, qb[layer], qr[layer], kb[layer], vb[layer], ob[layer], SCALE)

        def rows():
            return [(rng.standard_normal((n, H * D)).astype(np.float32),
                     rng.standard_normal((n, HKV * D)).astype(np.float32),
                     rng.standard_normal((n, HKV * D)).astype(np.float32)) for _ in range(L)]

        def check(step_rows, pos, what):
            side.synchronize()
            got = ob.cpu().numpy()
            for layer in range(L):
                q, k, v = step_rows[layer]
                for i, s in enumerate(ids):
                    want = model.token(s, layer, q[i], k[i], v[i], pos[i], None, None)
                    assert_close(got[layer, i, 0], want, what=f"{what} layer {layer} seq {s}")

        # a prompt of 30 tokens per sequence, eager
        pos = dec.begin_step(ids, 30)
        for layer in range(L):
            q = rng.standard_normal((n, 30, H * D)).astype(np.float32)
            k = rng.standard_normal((n, 30, HKV * D)).astype(np.float32)
            v = rng.standard_normal((n, 30, HKV * D)).astype(np.float32)
            out = torch.empty((n, 30, H * D), device=device)
            qd = torch.from_numpy(q).to(device)
            dec.layer(layer, qd, qd, torch.from_numpy(k).to(device), torch.from_numpy(v).to(device),
                      out, SCALE)
            for i, s in enumerate(ids):
                for t in range(30):
                    model.token(s, layer, q[i, t], k[i, t], v[i, t], pos[i] + t, None, None)
        side.synchronize()
        # step 1 eager (with the fixed plan), then capture step 2's layers
        r = rows()
        fill(r)
        pos = dec.begin_step(ids, 1)
        layers()
        check(r, pos, "eager step")
        r = rows()
        fill(r)
        pos = dec.begin_step(ids, 1)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            layers()
        graph.replay()
        check(r, pos, "first replay")
        for step in range(3):
            r = rows()
            fill(r)
            pos = dec.begin_step(ids, 1)
            graph.replay()
            check(r, pos, f"replay {step + 2}")
        dec.close()


def test_batch_decoder_sized_for_64_runs_small_steps_on_a_fixed_plan(device):
    """A decoder sized for 64 sequences must run steps of 3, 5, 6 and 7: with
    the graph-stable plan (planned for max_kv_len) a small batch takes more
    splits per sequence, and n_seq * splits exceeds 64 * splits(64) for
    these batch sizes.  The workspace must cover every smaller call."""
    import torch
    banner("batch decoder: max_batch 64, steps of 3/5/6/7 sequences on a fixed plan")
    rng = np.random.default_rng(17)
    max_kv = 2048
    g = emelk.geometry(L, H, HKV, D, BT, 256, emelk.KV_F16)
    actor = emelk.KvActor()
    assert actor.reserve(64, 256, BT)[0]
    for s in range(7):
        assert actor.allocate_sequence(s)[0]
    cache = emelk.KvCache(g)
    rope = emelk.RopeTable(D, D, max_kv, BASE, emelk.NEOX_PAIRING)
    dec = emelk.BatchDecoder(g, actor, cache, rope, max_batch=64, max_kv_len=max_kv)
    dec.set_fixed_plan(True)
    model = Model()
    for s in range(7):
        model.ensure(s)
    for ids, n_tok in (([0, 1, 2, 3, 4, 5, 6], 24), ([0, 1, 2], 1), ([0, 1, 2, 3, 4], 1),
                       ([5, 4, 3, 2, 1, 0], 1), ([0, 1, 2, 3, 4, 5, 6], 1)):
        pos = dec.begin_step(ids, n_tok)
        n = len(ids)
        for layer in range(L):
            q = rng.standard_normal((n, n_tok, H * D)).astype(np.float32)
            k = rng.standard_normal((n, n_tok, HKV * D)).astype(np.float32)
            v = rng.standard_normal((n, n_tok, HKV * D)).astype(np.float32)
            qd = torch.from_numpy(q).to(device)
            out = torch.full((n, n_tok, H * D), float("nan"), device=device)
            dec.layer(layer, qd, qd, torch.from_numpy(k).to(device),
                      torch.from_numpy(v).to(device), out, SCALE)
            torch.cuda.synchronize()
            got = out.cpu().numpy()
            for i, s in enumerate(ids):
                for t in range(n_tok):
                    want = model.token(s, layer, q[i, t], k[i, t], v[i, t], pos[i] + t, None, None)
                    assert_close(got[i, t], want, what=f"n={n} layer {layer} seq {s} tok {t}")
    dec.close()
