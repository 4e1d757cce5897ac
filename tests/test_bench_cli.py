"""bench.py's host-side contract, on the CPU: more than one GPU is refused
with a message, and the parity gate finds every `within_tolerance: false`
of a result line (the run then exits with status 3)."""
import json
import os
import subprocess
import sys

ROOT = os.path.normpath(os.path.join(os.path.dirname(__file__), ".."))


def test_more_than_one_gpu_is_refused_with_a_message():
    res = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=120)
    assert res.returncode == 2
    msg = json.loads(res.stdout.strip().splitlines()[-1])
    assert "one GPU" in msg["error"]


def test_parity_gate_finds_every_red_leg():
    sys.path.insert(0, ROOT)
    import bench
    line = {"parity_full_size": {"within_tolerance": True},
            "configs": {"a": {"parity_sample": {"within_tolerance": False}},
                        "b": {"parity_full_size": {"within_tolerance": True}},
                        "c": [{"within_tolerance": False}]}}
    assert sorted(bench.parity_failures(line)) == ["/configs/a/parity_sample", "/configs/c/0"]
    assert bench.parity_failures({"parity_full_size": {"within_tolerance": True}}) == []
