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
