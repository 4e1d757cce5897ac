"""The drop-in boundary's layout, pinned against the reference's own headers
(src/emel/memory/events.hpp:9-62, view.hpp:59-117, hybrid/context.hpp:11-30).

Builds tests/cpp/ref_layout.cpp with -Werror: its static_asserts compare
sizeof/alignof/offsetof of every event, the snapshot and kv_binding, and its
main() drives the actor through the reference's kv_binding and event types.
Skipped where the reference checkout is absent (the GPU box).  CPU only."""
import os
import re
import subprocess

import pytest

ROOT = os.path.normpath(os.path.join(os.path.dirname(__file__), ".."))
REF = "/root/reference"


def _binding_block(text):
    """The dispatch typedefs and struct kv_binding of hybrid/context.hpp."""
    start = text.index("using kv_reserve_dispatch_fn")
    m = re.compile(r"struct kv_binding \{.*?\};", re.S).search(text, start)
    assert m, "struct kv_binding not found"
    return text[start:m.end()] + "\n"


@pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "src", "emel", "memory")),
                    reason="reference checkout absent")
def test_boundary_layout_matches_reference_headers(tmp_path):
    ctx = open(os.path.join(REF, "src", "emel", "memory", "hybrid", "context.hpp")).read()
    hdr = tmp_path / "ref_kv_binding.inc"
    hdr.write_text(_binding_block(ctx))
    csrc = os.path.join(ROOT, "emel.cpp_amd", "csrc")
    exe = str(tmp_path / "ref_layout")
    subprocess.run(["g++", "-std=c++20", "-O1", "-Wall", "-Wextra", "-Werror",
                    "-I", os.path.join(REF, "src"), "-I", os.path.join(ROOT, "include"),
                    "-I", csrc, f'-DREF_KV_BINDING_HEADER="{hdr}"',
                    os.path.join(ROOT, "tests", "cpp", "ref_layout.cpp"),
                    os.path.join(csrc, "kv_actor.cpp"), os.path.join(csrc, "capi.cpp"),
                    "-o", exe], check=True)
    res = subprocess.run([exe], capture_output=True, text=True)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "ref layout ok" in res.stdout
