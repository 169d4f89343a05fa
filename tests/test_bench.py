"""bench.py's contract: the options it refuses (CPU) and its one JSON line
on the GPU (the fields the driver reads, the roofline object, the timing
figures beside the headline)."""
import json
import os
import subprocess
import sys

import pytest

from tests.conftest import ROOT, say

BENCH = os.path.join(ROOT, "bench.py")


def run_bench(*args, timeout=300):
    return subprocess.run([sys.executable, BENCH, *args], capture_output=True, text=True,
                          timeout=timeout, cwd=ROOT)


def test_bench_refuses_more_than_one_gpu():
    # each box has one GPU: --gpus above 1 exits with a message saying so,
    # before anything touches a GPU
    p = run_bench("--gpus", "2", timeout=120)
    assert p.returncode == 2
    assert "--gpus 2 is not supported" in p.stderr and "one GPU" in p.stderr
    assert p.stdout == ""


def test_bench_refuses_bad_step_counts():
    for args in (("--steps", "0"), ("--warmup", "-1"), ("--min-warmup-ms", "-5")):
        p = run_bench(*args, timeout=120)
        assert p.returncode == 2, args
        assert "--steps must be > 0" in p.stderr, args


@pytest.mark.gpu
def test_bench_json_line_under_the_drivers_flags():
    say("[gpu] bench.py --steps 20 --warmup 5 --no-cpu-baseline")
    p = run_bench("--steps", "20", "--warmup", "5", "--no-cpu-baseline")
    assert p.returncode == 0, p.stderr[-2000:]
    lines = [ln for ln in p.stdout.splitlines() if ln.strip()]
    line = json.loads(lines[-1])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
                "roofline", "cpu_baseline"):
        assert key in line, key
    assert line["n_gpus"] == 1 and line["steps"] == 20 and line["warmup"] == 5
    assert line["unit"] == "TOPS" and line["higher_is_better"] is True
    assert line["cpu_baseline"] is None
    cfg = line["config"]
    assert cfg["workload"].startswith("cfg2_resnet_3x3_s1")
    assert cfg["ops_per_step"] == 7398752256
    # value is the layer's ops over the headline time per launch
    tops = cfg["ops_per_step"] / (line["ms_per_step"] * 1e-3) / 1e12
    assert abs(tops - line["value"]) <= 0.01 * line["value"]
    # the figures beside the headline time the same launches
    for key in ("event_bracketed_ms_per_step", "graph_ms_per_step", "stamped_ms_per_step"):
        assert 0.5 * line["ms_per_step"] < cfg[key] < 3.0 * line["ms_per_step"], key
    roof = line["roofline"]
    assert roof["bound"] == "hbm" and roof["unit"] == "GB/s" and roof["peak"] == 8000.0
    achieved = cfg["algorithmic_bytes_per_step"] / (line["ms_per_step"] * 1e-3) / 1e9
    assert abs(achieved - roof["achieved"]) <= 0.01 * achieved
    assert abs(roof["frac"] - roof["achieved"] / roof["peak"]) < 1e-3
    assert roof["traffic"] is None or roof["traffic"] >= cfg["algorithmic_bytes_per_step"]
