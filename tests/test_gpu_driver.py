"""GPU runs of the C++ host driver (conv_lab): oracle check before timing,
CSV row with the reference's columns first, exit code contract."""
import csv
import io
import os
import subprocess
import sys

import pytest

# torch before the library's first GPU call: both load libamdhip64.so.7, and
# the first copy loaded serves the process; torch's own (the version it was
# built for) must be that one for torch.cuda to see the GPU
try:
    import torch  # noqa: F401
except ImportError:  # pragma: no cover - torch is part of the image
    torch = None

from tests.conftest import DRIVER, ROOT, say

REF_COLUMNS = ["case", "n", "h", "w", "c", "k", "r", "s", "out_h", "out_w", "eligible_strip",
               "generic_ms", "strip_ms", "winner", "generic_correct", "strip_correct"]


def run_driver(*args, timeout=120):
    return subprocess.run([DRIVER, *args], capture_output=True, text=True, timeout=timeout)


@pytest.mark.gpu
def test_driver_all_kernels_csv_on_smoke():
    say("[gpu] conv_lab --strategy all --csv --case cfg1_smoke")
    p = run_driver("--strategy", "all", "--csv", "--case", "cfg1_smoke", "--warmup", "2",
                   "--iterations", "5")
    assert p.returncode == 0, p.stderr
    rows = list(csv.DictReader(io.StringIO(p.stdout)))
    assert len(rows) == 1
    row = rows[0]
    header = p.stdout.splitlines()[0].split(",")
    assert header[:len(REF_COLUMNS)] == REF_COLUMNS  # conv_lab.cu:223-224 prefix
    for k in ("generic", "strip", "halo", "splitk"):
        assert row[f"{k}_correct"] == "1"
        assert float(row[f"{k}_ms"]) > 0
    assert row["winner"] in ("generic", "strip", "halo", "splitk")
    assert row["out_h"] == "16" and row["out_w"] == "16"


@pytest.mark.gpu
def test_driver_reference_strategy_both_on_stride2():
    # strip is ineligible at stride 2: its column stays -1, as in the
    # reference (conv_lab.cu:180-181, 197), and the winner is generic
    say("[gpu] conv_lab --strategy both --csv --case cfg3_down_3x3_s2")
    p = run_driver("--strategy", "both", "--csv", "--case", "cfg3_down_3x3_s2", "--warmup", "2",
                   "--iterations", "5")
    assert p.returncode == 0, p.stderr
    row = next(csv.DictReader(io.StringIO(p.stdout)))
    assert row["eligible_strip"] == "0"
    assert float(row["strip_ms"]) == -1
    assert row["winner"] == "generic"


@pytest.mark.gpu
def test_driver_human_line_and_reference_value_range():
    say("[gpu] conv_lab --range reference --case cfg4b_k36_tail")
    p = run_driver("--range", "reference", "--case", "cfg4b_k36_tail", "--strategy", "dispatch",
                   "--warmup", "1", "--iterations", "3")
    assert p.returncode == 0, p.stderr
    assert p.stdout.startswith("cfg4b_k36_tail:") and "winner" in p.stdout


@pytest.mark.gpu
def test_sweep_over_reference_cases(tmp_path):
    # the sweep (sweep.py:10-62): one row per case, rewritten after each case
    out = tmp_path / "sweep.csv"
    say("[gpu] sweep over smoke,nonmultiple8_k63,batch8_asymmetric_1x3")
    p = subprocess.run([sys.executable, "-m", "int8_kernel_lab_amd.sweep", "--cases",
                        "smoke,nonmultiple8_k63,batch8_asymmetric_1x3", "--iterations", "3",
                        "--warmup", "1", "--output", str(out)],
                       capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert p.returncode == 0, p.stdout + p.stderr
    rows = list(csv.DictReader(out.open()))
    assert [r["case"] for r in rows] == ["smoke", "nonmultiple8_k63", "batch8_asymmetric_1x3"]
    for r in rows:
        assert r["generic_correct"] == "1" and r["winner"] != "none"
        assert r["dispatch"] in ("generic", "strip", "halo", "splitk")


@pytest.mark.gpu
def test_vendor_miopen_matches_dispatched_kernel():
    # MIOpen's int8 convolution (an independent implementation) must write
    # the same int32 output as the dispatched kernel on the same data
    from int8_kernel_lab_amd import vendor
    for case in ("cfg1_smoke", "cfg4b_k36_tail"):
        say(f"[gpu] vendor_lab --case {case}")
        row = vendor.miopen_row(os.path.join(ROOT, "int8_kernel_lab_amd", "workloads",
                                             "baseline.csv"), case, warmup=1, iterations=3)
        assert row["vendor_correct"] == "1", row
        assert float(row["vendor_ms"]) > 0 and float(row["dispatch_ms"]) > 0


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["small", "darknet_res_13_reduce"])
def test_vendor_hipblaslt_gemm_matches_dispatched_kernel(case):
    # darknet_res_13_reduce (1x1, C = 1024) dispatches split-K, whose
    # launch needs a workspace of partial sums
    import int8_kernel_lab_amd as lab
    from int8_kernel_lab_amd import vendor
    if case == "small":
        shape = lab.ConvShape(2, 28, 28, 64, 96, 1, 1, 0, 0, 1, 1, 1, 1)
    else:
        shape = lab.load_case(os.path.join(lab.WORKLOADS_DIR, "reference.csv"), case)
        assert lab.workspace_bytes(lab.dispatch(shape), shape) > 0
    say(f"[gpu] torch._int_mm vs dispatch on {shape}")
    got = vendor.hipblaslt_gemm(shape, warmup=1, iterations=3)
    assert got["hipblaslt_correct"] == 1, got
    assert got["hipblaslt_ms"] > 0
