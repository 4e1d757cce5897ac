"""Shared scenario builder for the GPU parity tests: one KV actor with a
seeded page permutation, device pools filled through the append kernel, and
the oracle's token-major caches holding the same logical rows."""
from __future__ import annotations

import numpy as np

import emelk
import oracle


class Scenario:
    def __init__(self, *, n_layer, n_head, n_kv, head_dim, block_tokens, lens, kv_type=emelk.KV_F16,
                 seed=0, identity=False, outlier_frac=0.0, extra_blocks=3, device="cuda:0",
                 fill=True, pool_byte=0):
        import torch
        self.torch = torch
        self.n_layer, self.n_head, self.n_kv, self.D = n_layer, n_head, n_kv, head_dim
        self.bt = block_tokens
        self.lens = [int(x) for x in lens]
        self.n_seq = len(self.lens)
        self.kv_type = kv_type
        self.kv_dim = n_kv * head_dim
        self.rng = np.random.default_rng(seed)
        perm_rng = np.random.default_rng(seed + 7919)  # page placement only
        self.device = device
        need = sum(-(-n // block_tokens) for n in self.lens)
        self.max_blocks = need + extra_blocks
        self.actor = emelk.KvActor()
        ok, err = self.actor.reserve(max(self.n_seq, 1), self.max_blocks, block_tokens)
        assert ok, err
        if not identity:
            self.actor.set_free_order(perm_rng.permutation(self.max_blocks).astype(np.uint16))
        for s, n in enumerate(self.lens):
            assert self.actor.allocate_sequence(s)[0]
            ok, err, _ = self.actor.allocate_slots(s, n)
            assert ok, err
        self.stride = max(1, max(-(-n // block_tokens) for n in self.lens) + 2)
        self.g = emelk.geometry(n_layer, n_head, n_kv, head_dim, block_tokens, self.max_blocks,
                                kv_type)
        self.pool_bytes = emelk.pool_bytes(self.g)
        # pool_byte 0xFF makes every never-written f16 slot a NaN
        self.k_pool = torch.full((self.pool_bytes,), pool_byte, dtype=torch.uint8, device=device)
        self.v_pool = torch.full((self.pool_bytes,), pool_byte, dtype=torch.uint8, device=device)
        self.refresh_tables()
        # logical fp32 rows [layer][seq] -> [len, kv_dim]
        self.k_rows, self.v_rows = [], []
        for _layer in range(n_layer):
            kl, vl = [], []
            for n in self.lens:
                k = self.rng.standard_normal((n, self.kv_dim)).astype(np.float32)
                v = self.rng.standard_normal((n, self.kv_dim)).astype(np.float32)
                if outlier_frac > 0:
                    k[self.rng.random(k.shape) < outlier_frac] *= 20.0
                    v[self.rng.random(v.shape) < outlier_frac] *= 20.0
                kl.append(k)
                vl.append(v)
            self.k_rows.append(kl)
            self.v_rows.append(vl)
        if fill:
            self.append_all()

    def refresh_tables(self):
        t = self.actor.export_block_tables(list(range(self.n_seq)), self.stride)
        self.tables_host = t
        self.tables = self.torch.from_numpy(np.ascontiguousarray(t).view(np.int16)).to(self.device)

    def append_all(self):
        torch = self.torch
        for layer in range(self.n_layer):
            for s, n in enumerate(self.lens):
                if n == 0:
                    continue
                k = torch.from_numpy(self.k_rows[layer][s]).to(self.device).view(1, n, self.kv_dim)
                v = torch.from_numpy(self.v_rows[layer][s]).to(self.device).view(1, n, self.kv_dim)
                pos = torch.zeros(1, dtype=torch.int32, device=self.device)
                emelk.append(self.g, self.k_pool, self.v_pool, layer, k, v, pos,
                             self.tables[s:s + 1])
        torch.cuda.synchronize()

    # ---- oracle-side views of the same data ----
    def oracle_cache(self, layer):
        """Token-major paged caches as the reference lays them out
        (key_cache[phys][kv_dim], text/generator/detail.hpp:2984-3005)."""
        cap = self.max_blocks * self.bt
        if self.kv_type == emelk.KV_F16:
            kc = np.zeros((cap, self.kv_dim), np.uint16)
            vc = np.zeros_like(kc)
        else:
            kc = np.zeros((cap, self.kv_dim // 32), oracle.BLOCK_Q8_0)
            vc = np.zeros_like(kc)
        for s, n in enumerate(self.lens):
            if n == 0:
                continue
            pos = np.arange(n)
            phys = self.tables_host[s][pos // self.bt].astype(np.int64) * self.bt + pos % self.bt
            if self.kv_type == emelk.KV_F16:
                kc[phys] = oracle.fp32_to_fp16(self.k_rows[layer][s])
                vc[phys] = oracle.fp32_to_fp16(self.v_rows[layer][s])
            else:
                kc[phys] = oracle.quantize_q8_0(self.k_rows[layer][s])
                vc[phys] = oracle.quantize_q8_0(self.v_rows[layer][s])
        return kc, vc

    def expected_pool(self, which):
        """The device pool bytes the append kernel must produce (bit-exact),
        derived from the oracle's caches and the pool layout."""
        L, P, H, bt, D = self.n_layer, self.max_blocks, self.n_kv, self.bt, self.D
        if self.kv_type == emelk.KV_F16:
            pool = np.zeros((L, P, H, bt, D), np.uint16)
            for layer in range(L):
                kc, vc = self.oracle_cache(layer)
                c = kc if which == "k" else vc
                pool[layer] = c.reshape(P, bt, H, D).transpose(0, 2, 1, 3)
            return pool.view(np.uint8).reshape(-1)
        region = bt * D + bt * D // 16
        pool = np.zeros((L, P, H, region), np.uint8)
        for layer in range(L):
            kc, vc = self.oracle_cache(layer)
            c = (kc if which == "k" else vc).reshape(P, bt, H, D // 32)
            qs = c["qs"].transpose(0, 2, 1, 3, 4).reshape(P, H, bt * D).view(np.uint8)
            d = np.ascontiguousarray(c["d"].transpose(0, 2, 1, 3)).reshape(P, H, bt * D // 32)
            pool[layer, :, :, :bt * D] = qs
            pool[layer, :, :, bt * D:] = d.view(np.uint8).reshape(P, H, bt * D // 16)
        return pool.reshape(-1)

    def oracle_decode(self, layer, q, lens=None, scale=None):
        """Reference nonflash route per sequence (q: [n_seq, n_head*D])."""
        lens = self.lens if lens is None else lens
        scale = (1.0 / np.sqrt(self.D)) if scale is None else scale
        kc, vc = self.oracle_cache(layer)
        fn = oracle.compute_attention_f16 if self.kv_type == emelk.KV_F16 else \
            oracle.compute_attention_q8_0
        out = np.zeros((self.n_seq, self.n_head * self.D), np.float32)
        for s, n in enumerate(lens):
            out[s] = fn(q[s], kc, vc, self.tables_host[s], self.bt, self.n_head, self.n_kv, self.D,
                        n, n, scale)
        return out

    def ideal_decode(self, layer, q, scale=None):
        """fp64 attention on exactly the operands both routes consume: the
        stored K/V values and q rounded to fp16 (round_q_for_nonflash,
        text/generator/detail.hpp:2898-2903)."""
        scale = (1.0 / np.sqrt(self.D)) if scale is None else scale
        q = oracle.fp16_to_fp32(oracle.fp32_to_fp16(q))
        out = np.zeros((self.n_seq, self.n_head * self.D), np.float32)
        for s, n in enumerate(self.lens):
            if self.kv_type == emelk.KV_F16:
                k = oracle.fp16_to_fp32(oracle.fp32_to_fp16(self.k_rows[layer][s]))
                v = oracle.fp16_to_fp32(oracle.fp32_to_fp16(self.v_rows[layer][s]))
            else:
                k = oracle.dequantize_q8_0(oracle.quantize_q8_0(self.k_rows[layer][s]))
                v = oracle.dequantize_q8_0(oracle.quantize_q8_0(self.v_rows[layer][s]))
            out[s] = oracle.attention_f64(q[s], k, v, self.n_head, self.n_kv, self.D, n, scale)
        return out

    def gpu_decode(self, layer, q, lens=None, scale=None, ws=None):
        torch = self.torch
        lens = self.lens if lens is None else lens
        scale = (1.0 / np.sqrt(self.D)) if scale is None else scale
        qd = torch.from_numpy(np.ascontiguousarray(q, np.float32)).to(self.device).view(
            self.n_seq, self.n_head, self.D)
        out = torch.full_like(qd, float("nan"))
        kl = torch.tensor(lens, dtype=torch.int32, device=self.device)
        mx = max(lens)
        if ws is None:
            ws = torch.zeros(emelk.decode_workspace_bytes(self.g, self.n_seq, mx) // 4 + 1,
                             dtype=torch.float32, device=self.device)
        emelk.decode(self.g, self.k_pool, self.v_pool, layer, qd, out, kl, mx, self.tables,
                     float(scale), ws)
        torch.cuda.synchronize()
        return out.view(self.n_seq, -1).cpu().numpy()


def assert_close(got, want, atol=2e-3, rtol=1e-2, what=""):
    """The attention parity bar: |got - want| <= atol + rtol*|want|
    (max-abs 2e-3 / max-rel 1e-2, fp32 accumulation)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = np.abs(got - want)
    bad = err > atol + rtol * np.abs(want)
    assert not bad.any(), (f"{what}: {bad.sum()} of {bad.size} outside tolerance; "
                           f"max abs err {err.max():.3e}")
    return float(err.max())


def banner(msg):
    """Names the case on stdout before any GPU work, flushed."""
    print(f"\n[gpu-case] {msg}", flush=True)


def pool_token_major(pool, layer, n_layer, max_blocks, n_kv, bt, d, q8):
    """One layer of a device pool in the reference's token-major paged
    layout (key_cache[phys][kv_dim], text/generator/detail.hpp:2984-3005):
    uint16 halves for f16 pools, BLOCK_Q8_0 rows for q8_0 pools (whose
    regions hold values [bt][d] then scales [bt][d/32])."""
    lb = pool.numel() // n_layer
    raw = pool[layer * lb:(layer + 1) * lb].cpu().numpy().reshape(max_blocks, n_kv, -1)
    if not q8:
        h = raw.view(np.uint16).reshape(max_blocks, n_kv, bt, d)
        return np.ascontiguousarray(h.transpose(0, 2, 1, 3)).reshape(max_blocks * bt, n_kv * d)
    qs = raw[:, :, :bt * d].view(np.int8).reshape(max_blocks, n_kv, bt, d // 32, 32)
    ds = raw[:, :, bt * d:].view(np.uint16).reshape(max_blocks, n_kv, bt, d // 32)
    out = np.empty((max_blocks, bt, n_kv, d // 32), oracle.BLOCK_Q8_0)
    out["qs"] = qs.transpose(0, 2, 1, 3, 4)
    out["d"] = ds.transpose(0, 2, 1, 3)
    return out.reshape(max_blocks * bt, n_kv * d // 32)
