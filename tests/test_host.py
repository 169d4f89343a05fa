"""CPU tests of the host side: the data generator, the kernels' exact
division, the workload-table readers, the C++ driver's command line and the
sweep script's argument handling.  No GPU is touched: every driver run below
exits on an argument or table error before its first HIP call.
"""
import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest

import int8_kernel_lab_amd as lab
from int8_kernel_lab_amd import sweep

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "int8_kernel_lab_amd", "csrc")
DRIVER = os.path.join(ROOT, "int8_kernel_lab_amd", "conv_lab")

# Published SplitMix64 outputs for seed 1234567 (the reference test vector of
# Vigna's splitmix64.c, reproduced by common ports of the generator).
SPLITMIX_1234567 = [6457827717110365317, 3203168211198807973, 9817491932198370423,
                    4593380528125082431, 16408922859458223821]


# ---- data generator ---------------------------------------------------------

def test_splitmix64_known_answers():
    # span 2^32 maps next() to its low 32 bits: value = lo + (next mod 2^32)
    state = ctypes.c_uint64(1234567)
    got = lab.fill_int32(5, -(1 << 31), (1 << 31) - 1, state)
    want = [(v & 0xFFFFFFFF) - (1 << 31) for v in SPLITMIX_1234567]
    assert got.tolist() == want
    # the state advanced by five golden-ratio increments
    assert state.value == (1234567 + 5 * 0x9E3779B97F4A7C15) % (1 << 64)
    state = ctypes.c_uint64(1234567)
    got8 = lab.fill_int8(5, -128, 127, state)
    assert got8.tolist() == [(v % 256) - 128 for v in SPLITMIX_1234567]


def test_generator_order_and_ranges():
    shape = lab.ConvShape(1, 4, 4, 16, 8, 3, 3, 1, 1)
    x, w, b = lab.make_case_data(shape, seed=99)
    state = ctypes.c_uint64(99)
    assert np.array_equal(x.reshape(-1), lab.fill_int8(x.size, -128, 127, state))
    assert np.array_equal(w.reshape(-1), lab.fill_int8(w.size, -128, 127, state))
    assert np.array_equal(b, lab.fill_int32(b.size, -(1 << 20), 1 << 20, state))
    xr, _, br = lab.make_case_data(shape, seed=99, value_range=(-4, 4), bias_range=(-31, 31))
    assert xr.min() >= -4 and xr.max() <= 4 and br.min() >= -31 and br.max() <= 31
    assert set(np.unique(xr).tolist()) == set(range(-4, 5))


# ---- exact division used by every kernel's index math -------------------------

def test_fastdiv_is_exact(tmp_path):
    exe = tmp_path / "fastdiv_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-I", CSRC, "-I", os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "fastdiv_check.cpp"), "-o", str(exe)],
                   check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    assert out.stdout.startswith("ok ")


def test_lds_layouts_are_conflict_free(tmp_path):
    # the fragment-read layouts (swz128, swz64, the row kernel's pixel pitch)
    # permute chunks, invert, and satisfy the measured ds_read_b128 bank rule
    exe = tmp_path / "layout_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-I", CSRC, "-I", os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "layout_check.cpp"), "-o", str(exe)],
                   check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    assert out.stdout.startswith("ok ")


# ---- workload tables (gen_case.py:15-36) ------------------------------------

def test_workload_loader_errors(tmp_path):
    bad = tmp_path / "bad.csv"
    bad.write_text("name,n,h,w,c,k,r,s\nx,1,8,8,16,16,3,3\n")
    with pytest.raises(SystemExit, match="missing columns: pad_h"):
        lab.load_workloads(str(bad))
    with pytest.raises(SystemExit, match="unknown case 'nope'"):
        lab.load_case(os.path.join(lab.WORKLOADS_DIR, "baseline.csv"), "nope")
    assert lab.load_case(os.path.join(lab.WORKLOADS_DIR, "reference.csv"), "big_3x3_s1") == \
        lab.ConvShape(16, 256, 256, 256, 256, 3, 3, 1, 1, 1, 1, 1, 1)


# ---- conv_lab command line (conv_lab.cu:112-145 defaults and errors) --------

def run_driver(*args):
    return subprocess.run([DRIVER, *args], capture_output=True, text=True, timeout=60)


@pytest.mark.parametrize("args", [
    ["--bogus"], ["--iterations"], ["--warmup", "abc"],
])
def test_driver_usage_errors(args):
    r = run_driver(*args)
    assert r.returncode != 0 and "usage: conv_lab" in r.stderr


@pytest.mark.parametrize("args", [
    ["--strategy", "cudnn"], ["--iterations", "0"], ["--warmup", "-1"],
    ["--range", "wide"], ["--threads", "-2"],
])
def test_driver_invalid_options(args):
    r = run_driver(*args)
    assert r.returncode != 0 and "invalid benchmark options" in r.stderr


def test_driver_table_errors(tmp_path):
    r = run_driver("--case", "nope")
    assert r.returncode != 0 and "unknown case 'nope'" in r.stderr
    bad = tmp_path / "bad.csv"
    bad.write_text("name,n,h,w,c,k,r,s,pad_h,pad_w,stride_h,stride_w,dilation_h\n"
                   "x,1,8,8,16,16,3,3,1,1,1,1,1\n")
    r = run_driver("--config", str(bad), "--case", "x")
    assert r.returncode != 0 and "missing columns: dilation_w" in r.stderr
    r = run_driver("--config", str(tmp_path / "absent.csv"))
    assert r.returncode != 0 and "cannot open" in r.stderr
    odd = tmp_path / "odd.csv"
    odd.write_text("name,n,h,w,c,k,r,s,pad_h,pad_w,stride_h,stride_w,dilation_h,dilation_w\n"
                   "c24,1,8,8,24,16,3,3,1,1,1,1,1,1\n")
    r = run_driver("--config", str(odd), "--case", "c24")
    assert r.returncode != 0 and "divisible by 16" in r.stderr


# ---- sweep (sweep.py:10-62) --------------------------------------------------

def test_sweep_rejects_unknown_cases_before_running():
    with pytest.raises(SystemExit, match="unknown cases: nope, zzz"):
        sweep.main(["--cases", "smoke,nope,zzz", "--driver", sys.executable])


def test_sweep_defaults():
    a = sweep.parse_args([])
    assert a.configs.name == "reference.csv" and a.iterations == 101 and a.warmup == 20
    assert a.strategy == "all"
    assert len(sweep.requested_cases(a.configs, None)) == 41


# ---- vendor comparison columns (sweep.py:44-56's --with-cudnn) --------------

FAKE_CONV_LAB = '''#!{py}
import sys
print("case,n,winner,dispatch,tops")
print(sys.argv[sys.argv.index("--case") + 1] + ",1,halo,halo,1.5")
'''

FAKE_VENDOR_LAB = '''#!{py}
import sys
case = sys.argv[sys.argv.index("--case") + 1]
print("case,dispatch,dispatch_ms,dispatch_batched_ms,vendor,vendor_algo,vendor_ms,"
      "vendor_batched_ms,vendor_over_dispatch,vendor_correct,comparison_contract")
print(case + ",halo,0.01,0.008,miopen,direct,0.5,0.49,50,1,\\"fake contract\\"")
'''


def _script(path, text):
    path.write_text(text.format(py=sys.executable))
    path.chmod(0o755)
    return path


def test_sweep_with_vendor_adds_comparison_columns(tmp_path):
    conv = _script(tmp_path / "conv_lab", FAKE_CONV_LAB)
    vend = _script(tmp_path / "vendor_lab", FAKE_VENDOR_LAB)
    out = tmp_path / "sweep.csv"
    assert sweep.main(["--cases", "smoke,batch16_bottleneck_reduce", "--driver", str(conv),
                       "--with-vendor", "--vendor-driver", str(vend), "--output", str(out)]) == 0
    import csv
    rows = list(csv.DictReader(out.open()))
    assert [r["case"] for r in rows] == ["smoke", "batch16_bottleneck_reduce"]
    for r in rows:
        assert float(r["dispatch_ms"]) == 0.01 and float(r["miopen_ms"]) == 0.5
        assert float(r["miopen_over_dispatch"]) == pytest.approx(50.0)
        assert r["miopen_correct"] == "1" and r["comparison_contract"] == "fake contract"
    # 3x3 smoke is not a plain GEMM; the 1x1 bottleneck is, but there is no GPU here
    assert rows[0]["hipblaslt_contract"].startswith("not a plain gemm")
    assert rows[1]["hipblaslt_contract"] == "no gpu" and rows[1]["hipblaslt_ms"] == ""


def test_vendor_plain_gemm_predicate():
    from int8_kernel_lab_amd import vendor
    assert vendor.is_plain_gemm(lab.ConvShape(64, 56, 56, 256, 64, 1, 1, 0, 0, 1, 1, 1, 1))
    assert not vendor.is_plain_gemm(lab.ConvShape(1, 16, 16, 64, 64, 3, 3, 1, 1, 1, 1, 1, 1))
    assert not vendor.is_plain_gemm(lab.ConvShape(1, 16, 16, 64, 64, 1, 1, 0, 0, 2, 2, 1, 1))
    assert not vendor.is_plain_gemm(lab.ConvShape(1, 16, 16, 64, 64, 1, 1, 1, 1, 1, 1, 1, 1))


def test_vendor_driver_is_built_and_links():
    # the MIOpen comparison driver links against libi8conv and MIOpen; its
    # usage error needs no GPU
    from int8_kernel_lab_amd import vendor
    assert vendor.VENDOR_DRIVER.exists()
    r = subprocess.run([str(vendor.VENDOR_DRIVER), "--bogus"], text=True, capture_output=True)
    assert r.returncode != 0 and "usage: vendor_lab" in r.stderr
