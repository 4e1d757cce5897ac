"""The C-ABI library loads and exports every symbol include/emelk.h declares;
host-side validation paths work without a GPU.  CPU only."""
import ctypes
import os
import re

import emelk

ROOT = os.path.normpath(os.path.join(os.path.dirname(__file__), ".."))


def header_symbols():
    text = open(os.path.join(ROOT, "include", "emelk.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = set(re.findall(r"\b(emelk_\w+)\s*\(", text))
    # function-pointer typedef/field names are not exported symbols
    return {n for n in names if not n.endswith("_fn")}


def test_every_declared_symbol_is_exported():
    declared = header_symbols()
    assert declared, "no declarations parsed"
    lib = ctypes.CDLL(emelk.LIB_PATH)
    missing = [n for n in sorted(declared) if not hasattr(lib, n)]
    assert not missing, missing
    assert declared == set(emelk.SYMBOLS)


def test_pool_bytes_matches_layout():
    g = emelk.geometry(32, 32, 8, 128, 32, 16448, emelk.KV_F16)
    assert emelk.pool_bytes(g) == 32 * 16448 * 8 * 32 * 128 * 2
    g8 = emelk.geometry(32, 32, 8, 128, 32, 16448, emelk.KV_Q8_0)
    assert emelk.pool_bytes(g8) == 32 * 16448 * 8 * (32 * 128 + 32 * 4 * 2)


def test_invalid_geometry_is_rejected():
    out = ctypes.c_uint64(0)
    for bad in [emelk.geometry(1, 6, 4, 128, 16, 8),        # n_head % n_head_kv
                emelk.geometry(1, 8, 8, 96, 16, 8),         # head_dim
                emelk.geometry(1, 8, 8, 1024, 16, 8),       # head_dim above 512
                emelk.geometry(1, 8, 8, 64, 2, 8, emelk.KV_Q8_0),  # q8_0 page too small
                emelk.geometry(1, 8, 8, 64, 16, 40000),     # max_blocks
                emelk.geometry(1, 8, 8, 64, 16, 8, 3)]:     # kv_type
        assert emelk.lib.emelk_kv_pool_bytes(ctypes.byref(bad), ctypes.byref(out)) == \
            emelk.ERR_INVALID_REQUEST


def test_kernel_entry_points_validate_before_touching_the_gpu():
    g = emelk.geometry(2, 8, 2, 64, 16, 64)
    # null pools / bad layer are rejected on the host
    assert emelk.lib.emelk_kv_append(ctypes.byref(g), None, None, 0, None, None, 1, 1, None, None,
                                     4, None) == emelk.ERR_INVALID_REQUEST
    assert emelk.lib.emelk_attn_decode(ctypes.byref(g), None, None, 5, None, None, 1, None, 10,
                                       None, 4, 0.1, None, 0, None) == emelk.ERR_INVALID_REQUEST
    assert emelk.lib.emelk_kv_copy_blocks(ctypes.byref(g), None, None, None, 0, None) == \
        emelk.ERR_INVALID_REQUEST
    ws = emelk.decode_workspace_bytes(g, 4, 1000)
    assert ws > 0 and ws % 4 == 0
    bad_cb = ctypes.c_int32(0)
    assert not emelk.lib.emelk_kv_cache_copy_block(0, 1, 16, None, ctypes.byref(bad_cb))
    assert bad_cb.value == emelk.ERR_INVALID_REQUEST


def test_contiguous_decode_validates_its_layout_before_touching_the_gpu():
    g = emelk.geometry(2, 8, 2, 64, 16, 64)
    fake = ctypes.c_void_p(256)  # never dereferenced: every call below is refused first
    f = emelk.lib.emelk_attn_decode_contiguous

    def call(n_seq=2, max_len=100, stride=128, k_rows=None, v_rows=None):
        return f(ctypes.byref(g), fake, fake, 0, k_rows, v_rows, fake, fake, n_seq, fake,
                 max_len, stride, 0.1, fake, 1 << 20, None)

    assert call(stride=120) == emelk.ERR_INVALID_REQUEST           # not whole pages
    assert call(max_len=129) == emelk.ERR_INVALID_REQUEST          # context past the stride
    assert call(n_seq=9) == emelk.ERR_INVALID_REQUEST              # 9 x 8 pages > 64
    assert call(stride=0) == emelk.ERR_INVALID_REQUEST
    assert call(k_rows=fake) == emelk.ERR_INVALID_REQUEST          # k_rows without v_rows
    assert call(n_seq=0) == emelk.ERR_INVALID_REQUEST


def test_rope_table_rejects_bad_pairings_before_touching_the_gpu():
    h = ctypes.c_void_p(None)

    def create(n_rot, pairing, head_dim=128, max_pos=16, base=1e4):
        p = emelk.RopeParams(n_rot, *pairing, base)
        return emelk.lib.emelk_rope_table_create(ctypes.byref(p), head_dim, max_pos, None,
                                                 ctypes.byref(h))

    # overlapping pairs (p, p+1): the reference would chain them, the kernel cannot
    assert create(128, (1, 1, 1, 0)) == emelk.ERR_INVALID_REQUEST
    # pairs leaving the head
    assert create(128, (4, 4, 1, 0)) == emelk.ERR_INVALID_REQUEST
    assert create(128, (1, 1, 0, 2)) == emelk.ERR_INVALID_REQUEST
    # bad base, head or positions
    assert create(128, emelk.NORMAL_PAIRING, base=0.0) == emelk.ERR_INVALID_REQUEST
    assert create(128, emelk.NORMAL_PAIRING, head_dim=1024) == emelk.ERR_INVALID_REQUEST
    assert create(128, emelk.NORMAL_PAIRING, max_pos=0) == emelk.ERR_INVALID_REQUEST
    assert not h.value
    # rot_dim <= 1 rotates nothing: a table with no device memory is valid
    assert create(1, emelk.NORMAL_PAIRING) == emelk.ERR_NONE and h.value
    emelk.lib.emelk_rope_table_destroy(h)
    # the fused append validates its arguments first
    g = emelk.geometry(1, 4, 2, 64, 16, 4)
    assert emelk.lib.emelk_kv_qkv_rope_append(ctypes.byref(g), None, None, 0, None, None, None,
                                              None, 1, 1, None, None, 1, None, None, None, 0,
                                              1e-6, None) == emelk.ERR_INVALID_REQUEST


def test_plain_c_client_builds_and_runs(tmp_path):
    """include/emelk.h compiles as C11 with warnings as errors, and a C
    program linked against libemelk.so drives the actor through the
    kv_binding table and plans prompts (tests/cpp/abi_consumer.c)."""
    import subprocess
    exe = str(tmp_path / "abi_consumer")
    libdir = os.path.dirname(emelk.LIB_PATH)
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Wextra", "-Werror", "-I",
                    os.path.join(ROOT, "include"), os.path.join(ROOT, "tests", "cpp",
                                                                "abi_consumer.c"),
                    "-L", libdir, "-lemelk", f"-Wl,-rpath,{libdir}", "-o", exe], check=True)
    res = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert res.returncode == 0 and res.stdout.strip() == "ok", res.stdout + res.stderr


def test_workspace_size_covers_every_smaller_call():
    """A workspace sized for (n_seq, max_kv_len) must serve every call with
    fewer sequences or shorter contexts: an executor sizes it once for its
    largest step.  The split count rises as the batch shrinks, so the exact
    need (emelk_attn_decode_plan) is not monotone in n_seq."""
    lens = [1, 31, 32, 33, 500, 1023, 1024, 1025, 4096, 8191, 8192]
    for g in (emelk.geometry(32, 32, 8, 128, 32, 16448),
              emelk.geometry(16, 32, 8, 64, 16, 32768),
              emelk.geometry(28, 16, 8, 128, 32, 64, emelk.KV_Q8_0),
              emelk.geometry(4, 8, 1, 512, 16, 2048)):
        exact = {(n, L): emelk.decode_plan(g, n, L)[2] for n in range(1, 65) for L in lens}
        non_monotone = any(exact[(n, 8192)] > exact[(64, 8192)] for n in range(1, 64))
        for n_max in (1, 3, 16, 64):
            for L_max in (33, 1024, 8192):
                ws = emelk.decode_workspace_bytes(g, n_max, L_max)
                need = max(v for (n, L), v in exact.items() if n <= n_max and L <= L_max)
                assert ws >= need, (g.head_dim, n_max, L_max, ws, need)
        if g.head_dim == 128 and g.n_head_kv == 8 and g.kv_type == emelk.KV_F16:
            assert non_monotone  # the case the bound exists for


def test_decode_plan_splits_cover_the_context():
    g = emelk.geometry(32, 32, 8, 128, 32, 16448)
    for n, L in [(1, 512), (3, 8192), (16, 4096), (64, 8192), (64, 1)]:
        tps, ns, b = emelk.decode_plan(g, n, L)
        assert tps > 0 and ns >= 1 and (ns - 1) * tps < L <= ns * tps
        assert b == n * 32 * ns * (128 + 2) * 4


class _FakeDev:
    """Stands in for a device tensor so the checks can be driven on the CPU;
    every case below must raise before any device call."""

    def __init__(self, t, cuda=True):
        self.t, self.is_cuda, self.dtype, self.shape = t, cuda, t.dtype, t.shape
        self.device = "cuda:0" if cuda else "cpu"

    def is_contiguous(self):
        return self.t.is_contiguous()

    def dim(self):
        return self.t.dim()

    def numel(self):
        return self.t.numel()

    def element_size(self):
        return self.t.element_size()

    def data_ptr(self):
        raise AssertionError("validation let a bad call through to the library")


def test_python_helpers_reject_bad_tensors_before_any_launch():
    import pytest
    import torch
    g = emelk.geometry(2, 8, 2, 64, 16, 64)
    pb = emelk.pool_bytes(g)
    F = _FakeDev
    kp, vp = F(torch.zeros(pb, dtype=torch.uint8)), F(torch.zeros(pb, dtype=torch.uint8))
    q = F(torch.zeros(3, 8, 64))
    out = F(torch.zeros(3, 8, 64))
    lens = F(torch.zeros(3, dtype=torch.int32))
    tables = F(torch.zeros(3, 4, dtype=torch.int16))
    ws = F(torch.zeros(64))
    cases = [
        dict(k_pool=F(torch.zeros(pb - 1, dtype=torch.uint8))),     # pool too small
        dict(q=F(torch.zeros(3, 8, 64), cuda=False)),               # host tensor
        dict(q=F(torch.zeros(3, 8, 64, dtype=torch.float64))),      # dtype
        dict(q=F(torch.zeros(64, 8, 3).transpose(0, 2))),           # not contiguous
        dict(out=F(torch.zeros(3, 8, 32))),                         # shape
        dict(kv_lens=F(torch.zeros(3, dtype=torch.int64))),         # index dtype
        dict(kv_lens=F(torch.zeros(2, dtype=torch.int32))),         # one length short
        dict(block_tables=F(torch.zeros(2, 4, dtype=torch.int16))),  # one row short
        dict(block_tables=F(torch.zeros(3, 4, dtype=torch.int32))),  # table dtype
        dict(workspace=None),
    ]
    base = dict(k_pool=kp, v_pool=vp, q=q, out=out, kv_lens=lens, block_tables=tables,
                workspace=ws)
    for case in cases:
        a = dict(base, **case)
        with pytest.raises((ValueError, TypeError)):
            emelk.decode(g, a["k_pool"], a["v_pool"], 0, a["q"], a["out"], a["kv_lens"], 10,
                         a["block_tables"], 0.125, a["workspace"])
    rows = F(torch.zeros(3, 5, 2 * 64))
    pos = F(torch.zeros(3, dtype=torch.int32))
    with pytest.raises(ValueError):
        emelk.append(g, kp, vp, 0, rows, F(torch.zeros(3, 5, 64)), pos, tables)
    with pytest.raises(ValueError):
        emelk.prefill_chunk(g, kp, vp, 0, F(torch.zeros(3, 5, 8, 64)), F(torch.zeros(3, 5, 8, 64)),
                            F(torch.zeros(2, dtype=torch.int32)), tables, 0.125)
    with pytest.raises(ValueError):
        emelk.copy_blocks(g, kp, vp, F(torch.zeros(4, 3, dtype=torch.int32)))
    # contiguous decode: the same tensor checks, and its stored rows come in pairs
    krow = F(torch.zeros(3, 2 * 64))
    for case in cases[:7] + [dict(workspace=None)]:
        a = dict(base, **case)
        with pytest.raises((ValueError, TypeError)):
            emelk.decode_contiguous(g, a["k_pool"], a["v_pool"], 0, a["q"], a["out"],
                                    a["kv_lens"], 10, 16, 0.125, a["workspace"])
    with pytest.raises(ValueError):
        emelk.decode_contiguous(g, kp, vp, 0, q, out, lens, 10, 16, 0.125, ws, k_rows=krow)
    with pytest.raises(ValueError):
        emelk.decode_contiguous(g, kp, vp, 0, q, out, lens, 10, 16, 0.125, ws, k_rows=krow,
                                v_rows=F(torch.zeros(3, 64)))
