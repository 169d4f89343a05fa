#!/usr/bin/env python3
"""Headline benchmark: effective INT8 TOPS of the dispatched kernel on the
BASELINE configuration 2 layer (N=32, 28x28, C=K=128, 3x3, stride 1, pad 1;
the layer the >=50%-of-peak target is quoted on), on one GPU.

A step = one convolution of the whole layer (7.40 GOP) with input, filter,
bias and output resident in HBM.  Before timing, the GPU output is checked
bit-exact against the CPU oracle (the reference's check-before-time
contract, conv_lab.cu:193-194).  Timing: the K steps are launched as
replays of a HIP graph of 100 launches (a serving loop's form: the host
enqueues one graph per 100 convolutions): W warmup launches, synchronize,
then exactly K back-to-back launches between one pair of HIP events on the
graph's stream; the output is checked again after them.  Beside it: the same
K launches enqueued one by one on a stream, and the reference's per-launch
median (conv_lab.cu:88-110).

Prints one JSON line.  --gpus N > 1 is not supported (one GPU per box).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_INT8_TOPS = 5000.0   # MI355X dense INT8 MFMA, published
PEAK_HBM_GBPS = 8000.0    # MI355X HBM3E, published
WORKLOAD = "cfg2_resnet_3x3_s1"


def cpu_baseline(shape, x, w, b, threads: int, min_cpu_seconds: float = 10.0):
    """The oracle (a port of conv_lab.cu:39-66) on the host cores, repeated
    over the full layer until about `min_cpu_seconds` of CPU work."""
    from oracle import oracle
    reps, t_total = 0, 0.0
    while True:
        t0 = time.perf_counter()
        oracle.conv(shape, x, w, b, threads=threads)
        t_total += time.perf_counter() - t0
        reps += 1
        if t_total * threads >= min_cpu_seconds or reps >= 50:
            break
    tops = shape.ops() * reps / t_total / 1e12
    return {"value": round(tops, 6), "unit": "TOPS", "cores": threads, "kind": "port",
            "sample": f"oracle.conv over the full {WORKLOAD} layer x{reps} "
                      f"({reps * shape.ops() / 1e9:.1f} GOP, {t_total:.2f} s wall)"}


def copy_calibration(mib: int, steps: int) -> int:
    """A kernel of known HBM traffic: y = -x over MIB MiB of int32, with x and
    y distinct buffers far larger than the L2 and the MALL, so each launch
    reads and writes exactly MIB MiB of HBM."""
    import torch
    n = mib * (1 << 20) // 4
    x = torch.ones(n, dtype=torch.int32, device="cuda")
    y = torch.empty_like(x)
    for _ in range(steps):
        torch.neg(x, out=y)
    torch.cuda.synchronize()
    assert int(y[0]) == -1 and int(y[-1]) == -1
    print(json.dumps({"copy_calibration_bytes_read": n * 4, "copy_calibration_bytes_written": n * 4,
                      "launches": steps}), flush=True)
    return 0


def write_floor(workload: str, steps: int, warmup: int) -> int:
    """Times torch's fill kernel over exactly the layer's output bytes (the
    NHWK int32 tensor every candidate must store), back to back between two
    events on the current stream: no convolution can finish faster."""
    import torch
    import int8_kernel_lab_amd as lab
    shape = lab.load_case(os.path.join(lab.WORKLOADS_DIR, "baseline.csv"), workload)
    y = torch.empty(shape.geometry().output_elements, dtype=torch.int32, device="cuda")
    for _ in range(warmup):
        y.fill_(7)
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        y.fill_(7)
    stop.record()
    torch.cuda.synchronize()
    us = start.elapsed_time(stop) * 1e3 / steps
    print(json.dumps({"write_floor_workload": workload, "bytes": y.numel() * 4,
                      "us_per_launch": round(us, 3),
                      "tops_if_conv_took_this_long": round(shape.ops() / (us * 1e-6) / 1e12, 1),
                      "launches": steps}), flush=True)
    return 0


def requant_bench(workload: str, steps: int, warmup: int) -> int:
    """The same layer with requantized int8 output (i8conv_launch_requant:
    the dispatched kernel's fused epilogue where it has one, else the int32
    convolution into a workspace and a requantizing pass), checked against
    the oracle, then timed like the headline (i8conv_measure_requant: events
    around `steps` back-to-back launches on the launch stream, in C++).  A
    separate line, not the headline: the reference's contract is int32
    output."""
    import numpy as np
    import int8_kernel_lab_amd as lab
    from oracle import oracle

    shape = lab.load_case(os.path.join(lab.WORKLOADS_DIR, "baseline.csv"), workload)
    g = shape.geometry()
    x, w, b = lab.make_case_data(shape)
    rng = np.random.default_rng(1)
    mult = rng.integers(2 ** 30, 2 ** 31, size=shape.k).astype(np.int32)
    shift = rng.integers(50, 54, size=shape.k).astype(np.int32)
    bufs = [lab.DeviceBuffer.from_array(a) for a in (x, w, b, mult, shift)]
    yb = lab.DeviceBuffer(g.output_elements)
    ws_n = lab.requant_workspace_bytes(shape)
    ws = lab.DeviceBuffer(ws_n) if ws_n else None
    yb.fill(0xA5)
    lab.launch_requant(shape, *bufs, 3, yb, ws, ws_n)
    lab.synchronize()
    got = yb.download(np.int8, g.output_elements).reshape(shape.output_shape)
    if not np.array_equal(got, oracle.requantize(oracle.conv(shape, x, w, b), mult, shift, 3)):
        print(f"bench.py: requantized output differs from the oracle on {workload}", file=sys.stderr)
        return 1
    median_ms, mean_ms = lab.measure_requant(shape, *bufs, 3, yb, ws, ws_n, warmup=warmup,
                                             iterations=steps)
    us = mean_ms * 1e3
    nbytes = shape.algorithmic_bytes() - 4 * g.output_elements + g.output_elements + 8 * shape.k
    print(json.dumps({"requant_workload": workload, "fused": lab.requant_fused(shape),
                      "us_per_launch": round(us, 3),
                      "per_launch_median_us": round(median_ms * 1e3, 3),
                      "tops": round(shape.ops() / (us * 1e-6) / 1e12, 1),
                      "pct_int8_mfma_peak": round(100 * shape.ops() / (us * 1e-6) / 1e12
                                                  / PEAK_INT8_TOPS, 2),
                      "algorithmic_bytes": nbytes,
                      "gbps": round(nbytes / (us * 1e-6) / 1e9, 1), "launches": steps}), flush=True)
    for buf in bufs + [yb, ws]:
        if buf is not None:
            buf.close()
    return 0


def traffic_record(workload: str, kernel: str):
    """HBM bytes per launch of `kernel` on `workload` from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (profiles/hbm_traffic.json),
    scaled by the same counters' reading for the copy kernel; None when that
    pair was not profiled."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        table = json.load(f)
    rec = table.get("kernels", {}).get(f"{workload}/{kernel}")
    return None if rec is None else int(rec["traffic_bytes"])


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    # the clocks settle after ~20 ms of back-to-back launches: 10000 warmup
    # launches (~65 ms) before the 5000 timed ones (~33 ms)
    ap.add_argument("--steps", type=int, default=5000)
    ap.add_argument("--warmup", type=int, default=10000)
    ap.add_argument("--kernel", default="dispatch",
                    help="dispatch (default) or one of generic|strip|halo|splitk")
    ap.add_argument("--workload", default=WORKLOAD)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="instead of the benchmark, run a plain device copy of MIB MiB "
                         "(int32 negate: reads and writes MIB MiB) --steps times, to scale "
                         "rocprofv3 FETCH_SIZE/WRITE_SIZE readings")
    ap.add_argument("--write-floor", action="store_true",
                    help="instead of the benchmark, time a plain fill kernel writing exactly "
                         "the workload's int32 output bytes (the store traffic alone)")
    ap.add_argument("--requant", action="store_true",
                    help="instead of the benchmark, time the same layer with requantized int8 "
                         "output (a separate line; the headline contract is int32 output)")
    args = ap.parse_args()
    if args.requant:
        return requant_bench(args.workload, args.steps, args.warmup)
    if args.copy_calibration:
        return copy_calibration(args.copy_calibration, args.steps)
    if args.write_floor:
        return write_floor(args.workload, args.steps, args.warmup)
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this lab measures one GPU "
              "(each box has one MI355X; the layer is not sharded across GPUs)", file=sys.stderr)
        return 2
    if args.steps <= 0 or args.warmup < 0:
        print("bench.py: --steps must be > 0 and --warmup >= 0", file=sys.stderr)
        return 2

    import numpy as np
    import int8_kernel_lab_amd as lab
    from oracle import oracle

    shape = lab.load_case(os.path.join(lab.WORKLOADS_DIR, "baseline.csv"), args.workload)
    kernel = lab.dispatch(shape) if args.kernel == "dispatch" else args.kernel
    g = shape.geometry()
    x, w, b = lab.make_case_data(shape)
    xb, wb, bb = (lab.DeviceBuffer.from_array(a) for a in (x, w, b))
    yb = lab.DeviceBuffer(4 * g.output_elements)
    ws_n = lab.workspace_bytes(kernel, shape)
    ws = lab.DeviceBuffer(ws_n) if ws_n else None

    # correctness before timing: full output vs the CPU oracle
    yb.fill(0xA5)
    lab.launch(kernel, shape, xb, wb, bb, yb, ws, ws_n)
    lab.synchronize()
    got = yb.download(np.int32, g.output_elements).reshape(shape.output_shape)
    expected = oracle.conv(shape, x, w, b)
    if not np.array_equal(got, expected):
        print(f"bench.py: {kernel} output differs from the oracle on {args.workload}",
              file=sys.stderr)
        return 1

    median_ms, stream_ms = lab.measure(kernel, shape, xb, wb, bb, yb, ws, ws_n,
                                       warmup=args.warmup, iterations=args.steps)
    per_graph = 100 if args.steps % 100 == 0 else 1
    yb.fill(0xA5)
    mean_ms = lab.measure_graph(kernel, shape, xb, wb, bb, yb, ws, ws_n, warmup=args.warmup,
                                iterations=args.steps, launches_per_graph=per_graph)
    got = yb.download(np.int32, g.output_elements).reshape(shape.output_shape)
    if not np.array_equal(got, expected):
        print(f"bench.py: {kernel} output after the graph replays differs from the oracle",
              file=sys.stderr)
        return 1
    ops = shape.ops()
    nbytes = shape.algorithmic_bytes()
    tops = ops / (mean_ms * 1e-3) / 1e12
    gbps = nbytes / (mean_ms * 1e-3) / 1e9
    info = lab.device_info()
    threads = min(16, os.cpu_count() or 1)
    cpu = None if args.no_cpu_baseline else cpu_baseline(shape, x, w, b, threads)

    line = {
        "metric": "effective INT8 TOPS per conv layer + % of MI355X dense INT8 MFMA peak",
        "value": round(tops, 3),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(mean_ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 (int32 accumulate)",
        "data": "synthetic (SplitMix64 seed 20260925: int8 U[-128,127], bias U[-2^20,2^20])",
        "config": {
            "workload": f"{args.workload}: N={shape.n} H=W={shape.h} C={shape.c} K={shape.k} "
                        f"{shape.r}x{shape.s} stride {shape.stride_h} pad {shape.pad_h}",
            "kernel": kernel,
            "gemm_mnk": [g.gemm_m, g.gemm_n, g.gemm_k],
            "ops_per_step": ops,
            "algorithmic_bytes_per_step": nbytes,
            "pct_int8_mfma_peak": round(100.0 * tops / PEAK_INT8_TOPS, 2),
            "per_launch_median_ms": round(median_ms, 6),
            "timing": f"HIP graph of {per_graph} launches replayed; "
                      f"{args.steps} launches enqueued one by one on a stream: "
                      f"{stream_ms * 1e3:.3f} us per launch "
                      f"({ops / (stream_ms * 1e-3) / 1e12:.1f} TOPS)",
            "stream_ms_per_step": round(stream_ms, 6),
            "device": info["arch"],
            "compute_units": info["compute_units"],
            "parallelism": "single GPU",
        },
        # op/B = 457 < ridge 625 (5.0 POPS / 8 TB/s): HBM is the binding roof
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbps, 1),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(gbps / PEAK_HBM_GBPS, 4),
            "traffic": traffic_record(args.workload, kernel),
        },
        "cpu_baseline": cpu,
    }
    for buf in (xb, wb, bb, yb, ws):
        if buf is not None:
            buf.close()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
