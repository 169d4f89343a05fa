#!/usr/bin/env python3
"""Measure every candidate kernel over a workload table (the counterpart of
the reference's scripts/sweep.py:10-62).

The reference compiled one binary per case (gen_case.py + make) and ran it;
here one prebuilt driver (conv_lab, next to this file) reads the case from
the CSV at run time.  For each requested case it runs

    conv_lab --config CONFIGS --case NAME --strategy STRATEGY --iterations N --csv

which checks every candidate against the CPU INT32 oracle before timing it
and exits nonzero on a wrong result; the sweep then prints the driver's
output and stops (the reference's check=True, sweep.py:37-41).  After every case the output CSV is rewritten with all rows
so far (sweep.py:55-59).  Unknown case names abort before anything runs
(sweep.py:26-29).

    python -m int8_kernel_lab_amd.sweep --configs int8_kernel_lab_amd/workloads/reference.csv \
        --output gpurun_out/dispatch_measurements.csv
"""
from __future__ import annotations

import argparse
import csv
import os
import subprocess
import sys
from pathlib import Path
from typing import List, Optional

HERE = Path(__file__).resolve().parent
DRIVER = HERE / "conv_lab"


def parse_args(argv: Optional[List[str]] = None) -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--configs", type=Path, default=HERE / "workloads" / "reference.csv")
    p.add_argument("--cases", help="comma-separated case names; default all")
    p.add_argument("--output", type=Path, default=Path("sweep_out/dispatch_measurements.csv"))
    p.add_argument("--iterations", type=int, default=101)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--strategy", default="all",
                   help="generic|strip|halo|splitk|both|all|dispatch (conv_lab --strategy)")
    p.add_argument("--range", default="baseline", choices=("baseline", "reference"),
                   help="data range: int8 full range (baseline) or U[-4,4] (reference)")
    p.add_argument("--driver", type=Path, default=DRIVER)
    p.add_argument("--with-vendor", action="store_true",
                   help="add vendor-library columns (sweep.py:44-56's --with-cudnn): MIOpen for "
                        "every case (vendor_lab), hipBLASLt int8 GEMM for plain-GEMM layers")
    p.add_argument("--vendor-driver", type=Path, default=None,
                   help="vendor_lab binary (default: next to this file)")
    return p.parse_args(argv)


def vendor_columns(args, configs: Path, case: str) -> dict:
    """The comparison columns of one case: dispatch_ms (the dispatched
    kernel, timed in the vendor driver's process), miopen_ms and its ratio,
    and for plain-GEMM layers hipblaslt_ms and its ratio; *_correct says
    whether the vendor output equals the dispatched kernel's."""
    from . import vendor

    driver = args.vendor_driver or vendor.VENDOR_DRIVER
    row = vendor.miopen_row(configs, case, args.warmup, args.iterations, driver)
    dispatch_ms = float(row["dispatch_ms"])
    miopen_ms = float(row["vendor_ms"])
    out = {"dispatch_ms": dispatch_ms,
           "miopen_algo": row["vendor_algo"],
           "miopen_ms": miopen_ms if miopen_ms > 0 else "",
           "miopen_over_dispatch": miopen_ms / dispatch_ms if miopen_ms > 0 else "",
           "miopen_correct": row["vendor_correct"],
           "comparison_contract": row["comparison_contract"]}
    from . import load_case
    gemm = vendor.hipblaslt_gemm(load_case(str(configs), case), args.warmup, args.iterations)
    out.update(gemm)
    hb = gemm["hipblaslt_ms"]
    out["hipblaslt_over_dispatch"] = float(hb) / dispatch_ms if hb != "" else ""
    return out


def requested_cases(configs: Path, cases: Optional[str]) -> List[str]:
    with configs.open(newline="") as stream:
        rows = list(csv.DictReader(stream))
    names = [row["name"] for row in rows]
    requested = cases.split(",") if cases else names
    unknown = sorted(set(requested) - set(names))
    if unknown:
        raise SystemExit(f"unknown cases: {', '.join(unknown)}")
    return requested


def main(argv: Optional[List[str]] = None) -> int:
    args = parse_args(argv)
    if not args.driver.exists():
        raise SystemExit(f"{args.driver} missing: build with `make -C int8_kernel_lab_amd/csrc`")
    configs = args.configs.resolve()
    cases = requested_cases(configs, args.cases)
    args.output.parent.mkdir(parents=True, exist_ok=True)
    rows = []
    for case in cases:
        cmd = [str(args.driver), "--config", str(configs), "--case", case,
               "--strategy", args.strategy, "--iterations", str(args.iterations),
               "--warmup", str(args.warmup), "--range", args.range, "--csv"]
        print(f"{case}: running", flush=True)
        result = subprocess.run(cmd, text=True, capture_output=True)
        if result.returncode != 0:
            sys.stderr.write(result.stdout + result.stderr)
            raise SystemExit(f"{case}: conv_lab exited with {result.returncode}")
        rows.append(next(csv.DictReader(result.stdout.splitlines())))
        if args.with_vendor:
            rows[-1].update(vendor_columns(args, configs, case))
        with args.output.open("w", newline="") as stream:
            writer = csv.DictWriter(stream, fieldnames=list(rows[0].keys()))
            writer.writeheader()
            writer.writerows(rows)
        r = rows[-1]
        extra = (f"; miopen x{float(r['miopen_over_dispatch']):.1f}" if r.get("miopen_over_dispatch")
                 else "")
        print(f"{case}: winner {r['winner']} dispatch {r['dispatch']} "
              f"({r['tops']} TOPS){extra}; wrote {args.output}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
