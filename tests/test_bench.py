"""CPU tier: bench.py's contract pieces that need no GPU.

- `--gpus N` above 1 exits with a message (one GPU per box; no multi-GPU path);
- without a GPU it exits non-zero instead of timing anything on the CPU;
- every kernel entry bench.py prices HBM traffic with exists in the committed
  rocprof summary (profiles/traffic.json), with positive byte counts and the
  copy calibration it was scaled by.
"""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def _run(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args],
                          capture_output=True, text=True, timeout=300)


def test_more_than_one_gpu_exits_with_message():
    r = _run("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_no_gpu_exits_nonzero():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    r = _run("--workload", "prefill", "--steps", "1", "--warmup", "0")
    assert r.returncode != 0
    assert r.stdout == ""


def test_traffic_entries_present():
    import bench
    with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
        t = json.load(f)
    cal = t["_calibration"]
    assert cal["fetch_factor"] > 0 and cal["write_factor"] > 0
    for name, key in bench.TRAFFIC_KEY.items():
        keys = key if isinstance(key, tuple) else (key,)
        for k in keys:
            assert k in t, f"{name}: {k} missing from profiles/traffic.json"
            assert t[k]["fetch_bytes"] > 0 and t[k]["write_bytes"] > 0, k
        assert bench._traffic(key) > 0
