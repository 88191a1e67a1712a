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
        assert key in t, f"{name}: {key} missing from profiles/traffic.json"
        assert t[key]["kernels"], key
        assert t[key]["fetch_bytes"] > 0 and t[key]["write_bytes"] > 0, key
        assert bench._traffic(key) > 0


def test_traffic_json_sums_a_steps_kernels(tmp_path):
    """--traffic-json: per kernel the mean counter value per dispatch, summed
    over the step's kernels, scaled by the copy calibration; kernels outside
    the step are left out."""
    import bench
    hdr = "Kernel_Name,Counter_Name,Counter_Value\n"

    def put(run, rows):
        d = tmp_path / run
        d.mkdir()
        (d / "run_counter_collection.csv").write_text(hdr + "".join(f"{a},{b},{c}\n" for a, b, c in rows))
    put("copy_fetch", [("__amd_rocclr_copyBuffer", "FETCH_SIZE", 1 << 20)])        # 2 GiB read as 1 GiB
    put("copy_write", [("__amd_rocclr_copyBuffer", "WRITE_SIZE", 2 << 20)])
    for w in bench.TRAFFIC_WORKLOADS:
        put(w + "_fetch", [("void ca::split_kernel<1>(int)", "FETCH_SIZE", 100), ("void ca::split_kernel<1>(int)", "FETCH_SIZE", 300),
                           ("void ca::merge_kernel(int)", "FETCH_SIZE", 10), ("void ca::stream_read_kernel(int)", "FETCH_SIZE", 9999),
                           ("void ca::prefill_x(int)", "FETCH_SIZE", 7)])
        put(w + "_write", [("void ca::split_kernel<1>(int)", "WRITE_SIZE", 4), ("void ca::merge_kernel(int)", "WRITE_SIZE", 6),
                           ("void ca::stream_read_kernel(int)", "WRITE_SIZE", 1), ("void ca::prefill_x(int)", "WRITE_SIZE", 1)])
    out = tmp_path / "t.json"
    bench.traffic_json(str(tmp_path), str(out))
    t = json.load(open(out))
    assert t["_calibration"]["fetch_factor"] == 2.0 and t["_calibration"]["write_factor"] == 1.0
    d = t["decode_fp8"]                               # stream_read left out
    assert d["kernels"] == ["ca::merge_kernel", "ca::prefill_x", "ca::split_kernel<1>"]
    assert d["fetch_bytes"] == (200 + 10 + 7) * 1024 * 2 and d["write_bytes"] == (4 + 6 + 1) * 1024
    b = t["backward"]                                 # the forward's kernel left out
    assert "ca::prefill_x" not in b["kernels"] and "ca::stream_read_kernel" in b["kernels"]
