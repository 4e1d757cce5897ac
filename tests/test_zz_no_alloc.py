"""emelk_attn_decode_noalloc: the allocation-free decode entry point (split
partials in a static per-GPU device array) against the entry points that
take a caller workspace, through the C ABI.  Same kernels and split plan,
so outputs and pools must agree bit for bit; two calls in a row, the second
smaller, so the array's leftovers from the first call must not leak in."""
import ctypes

import numpy as np
import pytest

import emelk
from kvsetup import Scenario, assert_close, banner


def _noalloc(sc, layer, k_rows, v_rows, q, out, kl, mx, tables):
    import torch
    return emelk.lib.emelk_attn_decode_noalloc(
        ctypes.byref(sc.g), ctypes.c_void_p(sc.k_pool.data_ptr()),
        ctypes.c_void_p(sc.v_pool.data_ptr()), layer,
        None if k_rows is None else ctypes.c_void_p(k_rows.data_ptr()),
        None if v_rows is None else ctypes.c_void_p(v_rows.data_ptr()),
        ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(out.data_ptr()), int(q.shape[0]),
        ctypes.c_void_p(kl.data_ptr()), mx, ctypes.c_void_p(tables.data_ptr()),
        int(tables.shape[1]), ctypes.c_float(1.0 / np.sqrt(sc.D)),
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))


def test_noalloc_rejects_an_oversized_call_before_the_device():
    g = emelk.geometry(1, 32, 8, 128, 32, 64)
    tps, ns, need = emelk.decode_plan(g, 65535, 8192)
    assert need > (16 << 20)
    e = emelk.lib.emelk_attn_decode_noalloc(ctypes.byref(g), None, None, 0, None, None, None,
                                            None, 65535, None, 8192, None, 4, 0.1, None)
    assert e == emelk.ERR_OUT_OF_MEMORY
    e = emelk.lib.emelk_attn_decode_noalloc(ctypes.byref(g), None, None, 0, None, None, None,
                                            None, 4, None, 8192, None, 4, 0.1, None)
    assert e == emelk.ERR_INVALID_REQUEST  # null pools, after the size check passed


@pytest.mark.gpu
def test_noalloc_decode_matches_workspace_entry_points(device):
    import torch
    # call 1: plain decode, 8 ragged sequences at Llama-3-8B head geometry
    banner("noalloc decode call 1: 8 ragged sequences, D=128, plain decode")
    lens = [3001, 17, 1024, 2048, 1, 700, 2999, 64]
    sc = Scenario(n_layer=1, n_head=32, n_kv=8, head_dim=128, block_tokens=32, lens=lens, seed=91)
    rng = np.random.default_rng(92)
    q = torch.from_numpy(rng.standard_normal((8, 32, 128)).astype(np.float32)).to(device)
    kl = torch.tensor(lens, dtype=torch.int32, device=device)
    mx = max(lens)
    ws = torch.zeros(emelk.decode_workspace_bytes(sc.g, 8, mx) // 4 + 1, device=device)
    want = torch.full_like(q, float("nan"))
    emelk.decode(sc.g, sc.k_pool, sc.v_pool, 0, q, want, kl, mx, sc.tables, 1 / np.sqrt(128), ws)
    got = torch.full_like(q, float("nan"))
    assert _noalloc(sc, 0, None, None, q, got, kl, mx, sc.tables) == emelk.ERR_NONE
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.cpu().numpy(), want.cpu().numpy())
    assert_close(got.view(8, -1).cpu().numpy(), sc.oracle_decode(0, q.view(8, -1).cpu().numpy()),
                 what="noalloc vs reference route")

    # call 2: smaller, store + attend, on a q8_0 pool; compared with
    # emelk_attn_decode_append on an identical copy of the pools
    banner("noalloc decode call 2: 3 sequences, q8_0, store + attend")
    lens2 = [513, 40, 1200]
    sc2 = Scenario(n_layer=2, n_head=16, n_kv=4, head_dim=128, block_tokens=16, lens=lens2,
                   seed=93, kv_type=emelk.KV_Q8_0, outlier_frac=0.01)
    kp0, vp0 = sc2.k_pool.clone(), sc2.v_pool.clone()
    q2 = torch.from_numpy(rng.standard_normal((3, 16, 128)).astype(np.float32)).to(device)
    nk = torch.from_numpy(rng.standard_normal((3, 4 * 128)).astype(np.float32)).to(device)
    nv = torch.from_numpy(rng.standard_normal((3, 4 * 128)).astype(np.float32)).to(device)
    # attend over each sequence's rows plus one new token at position len - 1
    # (the last stored row is overwritten by the new one)
    kl2 = torch.tensor(lens2, dtype=torch.int32, device=device)
    mx2 = max(lens2)
    got2 = torch.full_like(q2, float("nan"))
    assert _noalloc(sc2, 1, nk, nv, q2, got2, kl2, mx2, sc2.tables) == emelk.ERR_NONE
    torch.cuda.synchronize()
    kp_got, vp_got = sc2.k_pool.clone(), sc2.v_pool.clone()
    sc2.k_pool.copy_(kp0)
    sc2.v_pool.copy_(vp0)
    ws2 = torch.zeros(emelk.decode_workspace_bytes(sc2.g, 3, mx2) // 4 + 1, device=device)
    want2 = torch.full_like(q2, float("nan"))
    emelk.decode_append(sc2.g, sc2.k_pool, sc2.v_pool, 1, nk, nv, q2, want2, kl2, mx2,
                        sc2.tables, 1 / np.sqrt(128), ws2)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got2.cpu().numpy(), want2.cpu().numpy())
    assert torch.equal(kp_got, sc2.k_pool) and torch.equal(vp_got, sc2.v_pool)
    assert np.isfinite(got2.cpu().numpy()).all()
