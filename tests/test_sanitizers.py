"""The host side under AddressSanitizer and UndefinedBehaviorSanitizer, as
the reference runs its tests (scripts/test_with_sanitizers.sh:49-59):
kv_actor.cpp, capi.cpp and batch_planner.cpp are compiled with
-fsanitize=address,undefined -fno-sanitize-recover=all together with each C
or C++ client of the boundary (tests/cpp/abi_consumer.c drives the actor
through the kv_binding table and plans prompts; tests/cpp/actor_whitebox.cpp
drives the allocate effect on hand-built state; tests/cpp/ref_layout.cpp
drives the actor through the reference's own event types where the
reference checkout is present), and each client must run clean.  CPU only:
no device code is built."""
import os
import subprocess

import pytest

ROOT = os.path.normpath(os.path.join(os.path.dirname(__file__), ".."))
CSRC = os.path.join(ROOT, "emel.cpp_amd", "csrc")
REF = "/root/reference"
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer",
       "-g", "-O1"]
HOST_SRC = ["kv_actor.cpp", "capi.cpp", "batch_planner.cpp"]


@pytest.fixture(scope="module")
def host_objs(tmp_path_factory):
    d = tmp_path_factory.mktemp("asan")
    objs = []
    for src in HOST_SRC:
        o = str(d / (src + ".o"))
        subprocess.run(["g++", "-std=c++20", *SAN, "-Wall", "-I", CSRC, "-I",
                        os.path.join(ROOT, "include"), "-c", os.path.join(CSRC, src), "-o", o],
                       check=True)
        objs.append(o)
    return objs


def _run(exe):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    res = subprocess.run([exe], capture_output=True, text=True, timeout=120, env=env)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "runtime error" not in res.stderr and "AddressSanitizer" not in res.stderr, res.stderr
    return res


def test_c_client_under_sanitizers(tmp_path, host_objs):
    obj = str(tmp_path / "abi_consumer.o")
    subprocess.run(["gcc", "-std=c11", *SAN, "-Wall", "-Wextra", "-Werror", "-I",
                    os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "cpp", "abi_consumer.c"), "-c", "-o", obj],
                   check=True)
    exe = str(tmp_path / "abi_consumer")
    subprocess.run(["g++", *SAN, obj, *host_objs, "-o", exe], check=True)
    assert _run(exe).stdout.strip() == "ok"


def test_actor_whitebox_under_sanitizers(tmp_path, host_objs):
    exe = str(tmp_path / "actor_whitebox")
    subprocess.run(["g++", "-std=c++20", *SAN, "-I", CSRC, "-I", os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "cpp", "actor_whitebox.cpp"), *host_objs,
                    "-o", exe], check=True)
    _run(exe)


@pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "src", "emel", "memory")),
                    reason="reference checkout absent")
def test_reference_event_driver_under_sanitizers(tmp_path, host_objs):
    from test_ref_layout import _binding_block
    ctx = open(os.path.join(REF, "src", "emel", "memory", "hybrid", "context.hpp")).read()
    hdr = tmp_path / "ref_kv_binding.inc"
    hdr.write_text(_binding_block(ctx))
    exe = str(tmp_path / "ref_layout")
    subprocess.run(["g++", "-std=c++20", *SAN, "-Wall", "-Wextra", "-Werror",
                    "-I", os.path.join(REF, "src"), "-I", os.path.join(ROOT, "include"),
                    "-I", CSRC, f'-DREF_KV_BINDING_HEADER="{hdr}"',
                    os.path.join(ROOT, "tests", "cpp", "ref_layout.cpp"), *host_objs,
                    "-o", exe], check=True)
    assert "ref layout ok" in _run(exe).stdout
