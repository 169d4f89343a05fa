#!/usr/bin/env python3
"""Headline benchmark: effective INT8 TOPS of the dispatched kernel on the
BASELINE configuration 2 layer (N=32, 28x28, C=K=128, 3x3, stride 1, pad 1;
the layer the >=50%-of-peak target is quoted on), on one GPU.

A step = one convolution of the whole layer (7.40 GOP) with input, filter,
bias and output resident in HBM.  Before timing, the GPU output is checked
bit-exact against the CPU oracle (the reference's check-before-time
contract, conv_lab.cu:193-194).  Timing (i8conv_measure_graph): a warmup
of at least W launches AND at least --min-warmup-ms of wall time (back-to-
back launches need some tens of ms to bring the clocks to their steady
state), replayed from a HIP graph, ends in ~5 ms of replays the host does
not wait for; the timed launches are enqueued behind them, so the GPU does
not idle between the warmup and the timed launches.  The headline
(ms_per_step) is the K steps as K back-to-back launches enqueued one by one
on the stream (stream region), like the reference's launches
(conv_lab.cu:88-110) but batched, timed by events that the launches
themselves carry (hipExtLaunchKernel: the start of the first launch's first
kernel to the end of the last launch's last kernel); the output is poisoned
right before them and checked against the oracle after them.  The same
launches between two HIP events recorded on the stream around them
(config.event_bracketed_ms_per_step) also hold the two event packets'
overhead, ~10 us on 28x28x128, which weighs on short runs (about 0.5 us
per launch at K = 20; none at K = 2000, where both agree).  Beside it, the
same K launches as replays of a HIP graph of K launches (K <= 10000; larger K:
graphs of 10000 and a remainder) between events (config.graph_ms_per_step):
each graph replay begins some microseconds after the previous one ends, a
gap the graph region holds once per replay, which weighs on short runs
(28x28x128: about 0.4 us per launch at K = 20, 0.004 us at K = 2000); and
the same graphs between device clock stamps captured inside them
(config.stamped_ms_per_step, without that gap).  Also the reference's
per-launch median (conv_lab.cu:88-110).
The CPU baseline is the C oracle (a port of conv_lab.cu:39-66) timed on
this host, single-threaded and on all threads of the box's CPU share.

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


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def host_threads() -> int:
    """Threads of this process's CPU share: the CPUs it may run on, at most
    16 (a one-GPU box's share of its host, whatever the host has)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def time_oracle(shape, x, w, b, threads: int, min_cpu_seconds: float, max_reps: int = 50):
    """oracle.conv over the full layer on `threads` threads, repeated until
    about `min_cpu_seconds` of CPU work (threads x wall); (TOPS, reps,
    wall seconds)."""
    from oracle import oracle
    reps, t_total = 0, 0.0
    while True:
        t0 = time.perf_counter()
        oracle.conv(shape, x, w, b, threads=threads)
        t_total += time.perf_counter() - t0
        reps += 1
        if t_total * threads >= min_cpu_seconds or reps >= max_reps:
            break
    return shape.ops() * reps / t_total / 1e12, reps, t_total


def cpu_baseline(shape, x, w, b):
    """The oracle (a port of conv_lab.cu:39-66: bias, then fy -> fx -> c per
    output, int32) on this host's cores, in the same run as the GPU timing:
    single-threaded (the reference's oracle is single-threaded) and on all
    threads of the process's CPU share (`value`, `cores`).  Bounded samples
    of the same workload: about 6 s of CPU work single-threaded and 12 s of
    CPU work (threads x wall) on all threads."""
    from oracle import oracle
    threads = host_threads()
    one, one_reps, one_s = time_oracle(shape, x, w, b, 1, 6.0)
    many, many_reps, many_s = time_oracle(shape, x, w, b, threads, 12.0)
    return {"value": round(many, 6), "unit": "TOPS", "cores": threads, "kind": "port",
            "sample": f"oracle.conv over the full {WORKLOAD} layer x{many_reps} on {threads} "
                      f"threads ({many_reps * shape.ops() / 1e9:.1f} GOP, {many_s:.2f} s wall)",
            "single_thread": {"value": round(one, 6), "unit": "TOPS", "cores": 1,
                              "sample": f"the same layer x{one_reps} on 1 thread "
                                        f"({one_reps * shape.ops() / 1e9:.1f} GOP, "
                                        f"{one_s:.2f} s wall)"},
            "hardware_concurrency": os.cpu_count(),
            "cpu_model": cpu_model(),
            "build": oracle.build_info()}


def copy_calibration(mib: int, steps: int) -> int:
    """A kernel of known HBM traffic: y = -x over MIB MiB of int32, with x and
    y distinct buffers far larger than the L2 and the MALL, so each launch
    reads and writes exactly MIB MiB of HBM."""
    import torch
    n = mib * (1 << 20) // 4
    x = torch.ones(n, dtype=torch.int32, device="cuda")
    y = torch.empty_like(x)
    torch.neg(x, out=y)  # one untimed launch
    # the launches run on torch's current stream, so torch's events time them
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        torch.neg(x, out=y)
    stop.record()
    torch.cuda.synchronize()
    assert int(y[0]) == -1 and int(y[-1]) == -1
    us = start.elapsed_time(stop) * 1e3 / steps
    print(json.dumps({"copy_calibration_bytes_read": n * 4, "copy_calibration_bytes_written": n * 4,
                      "launches": steps, "us_per_launch": round(us, 3),
                      "gbps_read_plus_written": round(2 * n * 4 / (us * 1e-6) / 1e9, 1)}),
          flush=True)
    return 0


def write_floor(workload: str, steps: int, warmup: int, min_warmup_ms: float) -> int:
    """The store floor of the workload's dispatched row kernel: the lab's
    store-only kernel (i8conv_measure_store_floor) writing exactly the
    layer's int32 output bytes with the row kernel's 16-byte write-through
    stores, in its launch shape (workgroups x 512 threads, the same dynamic
    LDS), timed like the headline (stream launches timed by the events the
    first and last of them carry); beside it, an empty kernel of the same
    shape (the dispatch floor) and ordinary stores."""
    import numpy as np
    import int8_kernel_lab_amd as lab
    shape = lab.load_case(os.path.join(lab.WORKLOADS_DIR, "baseline.csv"), workload)
    nbytes = 4 * shape.geometry().output_elements
    plan = lab.describe(lab.dispatch(shape), shape)
    grid = int(plan.split("grid ")[1].split()[0]) if "grid " in plan else 256
    lds = int(plan.split("LDS ")[1].split()[0]) * 1024 if "copy waves" in plan else 0
    y = lab.DeviceBuffer(nbytes)
    out = {"write_floor_workload": workload, "bytes": nbytes, "workgroups": grid,
           "threads": 512, "lds_bytes": lds, "launches": steps}
    for key, n, through in (("write_through", nbytes, True), ("ordinary", nbytes, False),
                            ("empty", 0, True)):
        t = lab.measure_store_floor(y, n, grid, 512, lds, through, warmup=warmup,
                                    min_warmup_ms=min_warmup_ms, iterations=steps,
                                    launches_per_graph=min(steps, 100))
        us = t["kernel_ms"] * 1e3  # timed like the headline
        out[f"{key}_us_per_launch"] = round(us, 3)
        if n:
            units = y.download(np.int32, n // 4).reshape(-1, 4)
            if not (units == np.arange(units.shape[0], dtype=np.int32)[:, None]).all():
                print(f"bench.py: the store floor kernel ({key}) left wrong bytes", file=sys.stderr)
                return 1
    us = out["write_through_us_per_launch"]
    out["tops_if_conv_took_this_long"] = round(shape.ops() / (us * 1e-6) / 1e12, 1)
    out["pct_int8_mfma_peak_at_floor"] = round(100 * shape.ops() / (us * 1e-6) / 1e12
                                               / PEAK_INT8_TOPS, 2)
    y.close()
    print(json.dumps(out), flush=True)
    return 0


def lds_probe(steps: int, warmup: int, min_warmup_ms: float) -> int:
    """The LDS read probe in each pattern (i8conv_measure_lds_probe): 256
    workgroups x 512 threads, 4097 16-byte reads per lane, timed like the
    headline, each thread's XOR checked against the host's restatement.
    Prints the time per launch and the LDS read rate per compute unit at the
    2.4 GHz peak clock; under rocprofv3 --pmc the same launches give the
    bank-conflict counters of a known pattern."""
    import numpy as np
    import int8_kernel_lab_amd as lab
    workgroups, threads, reads = 256, 512, 4097
    sink = lab.DeviceBuffer(4 * workgroups * threads)
    out = {"lds_probe_workgroups": workgroups, "threads": threads, "reads_per_lane": reads,
           "bytes_per_launch": 16 * reads * workgroups * threads, "launches": steps}
    for pattern in lab.LDS_PROBE_PATTERNS:
        t = lab.measure_lds_probe(pattern, sink, workgroups, threads, reads, warmup=warmup,
                                  min_warmup_ms=min_warmup_ms, iterations=steps,
                                  launches_per_graph=min(steps, 100))
        got = sink.download(np.int32, workgroups * threads).reshape(workgroups, threads)
        if not (got == lab.lds_probe_expected(pattern, threads, reads)[None, :]).all():
            print(f"bench.py: the LDS probe ({pattern}) stored wrong values", file=sys.stderr)
            return 1
        us = t["mean_ms"] * 1e3
        out[f"{pattern}_us_per_launch"] = round(us, 3)
        out[f"{pattern}_bytes_per_clk_per_cu"] = round(
            out["bytes_per_launch"] / (us * 1e-6) / 256 / 2.4e9, 1)
    sink.close()
    print(json.dumps(out), flush=True)
    return 0


def dispatch_floor(steps: int, warmup: int, min_warmup_ms: float) -> int:
    """The dispatch floor over launch shapes: an empty kernel (the lab's
    store-only kernel with nothing to store, i8conv_measure_store_floor) in
    64, 256, 512 and 768 threads per workgroup x 128, 256, 512 and 1024
    workgroups, with no dynamic LDS and with 160 KB, and beside each
    (threads, workgroups) pair the same kernel writing config 2's 12.85 MB
    int32 output with 16-byte write-through stores; every figure timed like
    the headline.  One JSON line."""
    import numpy as np
    import int8_kernel_lab_amd as lab
    nbytes = 12845056
    y = lab.DeviceBuffer(nbytes)
    rows = []

    def timed(n, wg, threads, lds):
        t = lab.measure_store_floor(y, n, wg, threads, lds, True, warmup=warmup,
                                    min_warmup_ms=min_warmup_ms, iterations=steps,
                                    launches_per_graph=min(steps, 100))
        return round(t["kernel_ms"] * 1e3, 3)

    try:
        for threads in (64, 256, 512, 768):
            for wg in (128, 256, 512, 1024):
                row = {"threads": threads, "workgroups": wg,
                       "empty_us": timed(0, wg, threads, 0),
                       "empty_160kb_lds_us": timed(0, wg, threads, 160 * 1024),
                       "write_12_85mb_us": timed(nbytes, wg, threads, 0)}
                units = y.download(np.int32, nbytes // 4).reshape(-1, 4)
                if not (units == np.arange(units.shape[0], dtype=np.int32)[:, None]).all():
                    print("bench.py: the store floor kernel left wrong bytes", file=sys.stderr)
                    return 1
                rows.append(row)
    finally:
        y.close()
    empty = [r[k] for r in rows for k in ("empty_us", "empty_160kb_lds_us")]
    extra = [r["write_12_85mb_us"] - r["empty_us"] for r in rows]
    print(json.dumps({"dispatch_floor": rows, "launches": steps,
                      "empty_us_min": min(empty), "empty_us_max": max(empty),
                      "write_minus_empty_us_min": round(min(extra), 3),
                      "write_minus_empty_us_max": round(max(extra), 3)}), flush=True)
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
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[1])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--min-warmup-ms", type=float, default=100.0,
                    help="wall time the warmup lasts at least, whatever --warmup says "
                         "(the clocks settle after some tens of ms of back-to-back launches)")
    ap.add_argument("--kernel", default="dispatch",
                    help="dispatch (default) or one of generic|strip|halo|splitk")
    ap.add_argument("--workload", default=WORKLOAD)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="instead of the benchmark, run a plain device copy of MIB MiB "
                         "(int32 negate: reads and writes MIB MiB) --steps times, to scale "
                         "rocprofv3 FETCH_SIZE/WRITE_SIZE readings")
    ap.add_argument("--write-floor", action="store_true",
                    help="instead of the benchmark, time the lab's store-only kernel writing "
                         "exactly the workload's int32 output bytes in the dispatched row "
                         "kernel's launch shape (and an empty kernel of that shape)")
    ap.add_argument("--dispatch-floor", action="store_true",
                    help="instead of the benchmark, time an empty kernel (and one writing "
                         "config 2's output) over a grid of launch shapes")
    ap.add_argument("--lds-probe", action="store_true",
                    help="instead of the benchmark, time the LDS read probe in its four "
                         "patterns (the control for the LDS bank-conflict counters)")
    ap.add_argument("--requant", action="store_true",
                    help="instead of the benchmark, time the same layer with requantized int8 "
                         "output (a separate line; the headline contract is int32 output)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this lab measures one GPU "
              "(each box has one MI355X; the layer is not sharded across GPUs)", file=sys.stderr)
        return 2
    if args.steps <= 0 or args.warmup < 0 or args.min_warmup_ms < 0:
        print("bench.py: --steps must be > 0, --warmup and --min-warmup-ms >= 0", file=sys.stderr)
        return 2
    if args.requant:
        return requant_bench(args.workload, args.steps, args.warmup)
    if args.copy_calibration:
        return copy_calibration(args.copy_calibration, args.steps)
    if args.lds_probe:
        return lds_probe(args.steps, args.warmup, args.min_warmup_ms)
    if args.write_floor:
        return write_floor(args.workload, args.steps, args.warmup, args.min_warmup_ms)
    if args.dispatch_floor:
        return dispatch_floor(args.steps, args.warmup, args.min_warmup_ms)

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
    if not np.array_equal(got, expected) or lab.wait_expired():
        print(f"bench.py: {kernel} output differs from the oracle on {args.workload}",
              file=sys.stderr)
        return 1

    # the timed steps (stream region, the headline; graph and stamped
    # figures beside it); the output is poisoned right before the stream
    # region, so the check afterwards covers exactly the timed launches
    per_graph = min(args.steps, 10000)
    t = lab.measure_graph(kernel, shape, xb, wb, bb, yb, ws, ws_n, warmup=args.warmup,
                          min_warmup_ms=args.min_warmup_ms, iterations=args.steps,
                          launches_per_graph=per_graph, poison_byte=0xA5)
    mean_ms = t["kernel_ms"]
    got = yb.download(np.int32, g.output_elements).reshape(shape.output_shape)
    if not np.array_equal(got, expected):
        print(f"bench.py: {kernel} output after the timed replays differs from the oracle",
              file=sys.stderr)
        return 1
    # beside it, right after (the clocks are warm): the reference's
    # per-launch median (each launch between its own events, synchronized)
    median_ms, _ = lab.measure(kernel, shape, xb, wb, bb, yb, ws, ws_n,
                               warmup=args.warmup, iterations=args.steps)
    if lab.wait_expired():
        print(f"bench.py: a bounded wait of {kernel} gave up during the timed launches",
              file=sys.stderr)
        return 1
    ops = shape.ops()
    nbytes = shape.algorithmic_bytes()
    tops = ops / (mean_ms * 1e-3) / 1e12
    gbps = nbytes / (mean_ms * 1e-3) / 1e9
    info = lab.device_info()
    cpu = None if args.no_cpu_baseline else cpu_baseline(shape, x, w, b)
    graphs = f"{t['full_replays']} replay(s) of a HIP graph of {t['launches_per_graph']} launches"
    if t["remainder_launches"]:
        graphs += f" + a graph of {t['remainder_launches']}"

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
            "plan": lab.describe(kernel, shape),
            "gemm_mnk": [g.gemm_m, g.gemm_n, g.gemm_k],
            "ops_per_step": ops,
            "algorithmic_bytes_per_step": nbytes,
            "pct_int8_mfma_peak": round(100.0 * tops / PEAK_INT8_TOPS, 2),
            "timing": f"{args.steps} back-to-back launches enqueued one by one on a stream, "
                      f"timed from the start of the first launch's kernel to the end of the last "
                      f"one's by events the launches carry, after {t['warmup_launches']} warmup "
                      f"launches over {t['warmup_ms']:.0f} ms whose last ~5 ms the host does not "
                      f"wait for (the timed launches are enqueued behind them: no idle GPU between "
                      f"warmup and timing); output poisoned before and checked after the timed "
                      f"launches",
            # the same launches between two events recorded on the stream
            # around them (adds the event packets' overhead)
            "event_bracketed_ms_per_step": round(t["stream_ms"], 6),
            "warmup_launches_run": t["warmup_launches"],
            "warmup_ms": round(t["warmup_ms"], 1),
            # the same K launches as graph replays, between events
            # (holds one graph-start gap per replay)
            "graph_ms_per_step": round(t["mean_ms"], 6),
            "graph_timing": graphs,
            # the same graphs between device clock stamps captured inside
            # them: the launches plus one stamp dispatch, without that gap
            "stamped_ms_per_step": round(t["stamped_ms"], 6),
            "per_launch_median_ms": round(median_ms, 6),
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
