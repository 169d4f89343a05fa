"""python -m int8_kernel_lab_amd.timeline build
python -m int8_kernel_lab_amd.timeline run [LAYER] [--steps K] [--requant] [--json PATH]

build: compiles the stamped copies of the row kernel with copy waves and the
deep-channel split-K into timeline/_build/libi8conv_timeline.so (the library
itself must be built first: make -C int8_kernel_lab_amd/csrc).

run: on the GPU, launches LAYER (a row of workloads/baseline.csv, default
cfg2_resnet_3x3_s1) with its dispatched kernel through the stamped library,
checks it bit-exact against the oracle, times it like bench.py (graph region,
then K launches enqueued on a stream, whose last launch leaves the stamps;
with --requant, int8 output timed like bench.py --requant) and prints each
stamp's spread over waves: min / median / max microseconds after the
launch's first wave started.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import subprocess
import sys

from . import instrument

ROOT = os.path.dirname(os.path.dirname(instrument.PKG))
MAX_WORKGROUPS = 4096


def _spread(values, t0):
    import numpy as np
    v = values[values > 0]
    if v.size == 0:
        return None
    return [round(float(z), 3) for z in np.percentile((v - t0) / 100.0, [0, 50, 100])]


def _analyse(stamps, kernel_file):
    """Per-stamp spreads of one launch: stamps is [workgroups][WAVES][SLOTS]."""
    import numpy as np
    a = stamps.astype(np.int64)
    started = a[:, :, 0] > 0
    if not started.any():
        return None
    t0 = a[:, :, 0][started].min()
    out = {"workgroups": int(started.any(axis=1).sum()), "stamps_us": {}}
    if kernel_file == "kernel_rowpass.hip":
        copy = [w for w in range(instrument.WAVES) if (a[:, w, 2] > 0).any()]
        mfma = [w for w in range(instrument.WAVES) if (a[:, w, 27] > 0).any()]
        names = instrument.ROWPASS_SLOTS
        for g in range(2):
            for r in range(10):
                names = dict(names)
                names[4 + g * 10 + r] = f"MFMA wave: group {g} input row {r} ready"
    else:
        copy = [w for w in range(instrument.WAVES) if (a[:, w, 3] > 0).any()]
        mfma = [w for w in range(instrument.WAVES) if (a[:, w, 21] > 0).any()]
        names = instrument.DEEPK_SLOTS
    out["copy_waves"], out["mfma_waves"] = copy, mfma
    for slot, name in sorted(names.items()):
        if name.startswith("copy wave"):
            waves = copy
        elif name.startswith("MFMA wave"):
            waves = mfma
        else:
            waves = copy + mfma
        s = _spread(a[:, waves, slot], t0)
        if s is not None:
            out["stamps_us"][f"{slot:2d} {name}"] = s
    if kernel_file == "kernel_deepk.hip":
        for slot, name in sorted(instrument.DEEPK_FRAG_SLOTS.items()):
            s = _spread(a[:, mfma, slot], t0)
            if s is not None:
                out["stamps_us"][f"{slot:2d} {name}"] = s
    else:
        c0, c1 = instrument.ROWPASS_CYCLES
        cyc = a[:, mfma, c1] - a[:, mfma, c0]
        rt = (a[:, mfma, 29] - a[:, mfma, 27]) / 100.0
        ok = (cyc > 0) & (rt > 0)
        if ok.any():
            out["walk_us_median"] = round(float(np.median(rt[ok])), 3)
            out["walk_clock_ghz_median"] = round(float(np.median(cyc[ok] / rt[ok] / 1e3)), 3)
        r4, r8 = a[:, mfma, 8], a[:, mfma, 12]
        ok = (r4 > 0) & (r8 > 0)
        if ok.any():
            out["row_step_us_median"] = round(float(np.median((r8 - r4)[ok] / 400.0)), 3)
    return out


def _child(args):
    import numpy as np

    sys.path.insert(0, ROOT)
    import int8_kernel_lab_amd as lab
    from int8_kernel_lab_amd import _lib
    from oracle import oracle

    if os.path.realpath(_lib.LIB_PATH) != os.path.realpath(instrument.LIBRARY):
        raise SystemExit(f"timeline: loaded {_lib.LIB_PATH}, not the stamped library")
    shape = lab.load_case(os.path.join(lab.WORKLOADS_DIR, "baseline.csv"), args.layer)
    kernel = lab.dispatch(shape)
    g = shape.geometry()
    x, w, b = lab.make_case_data(shape)
    expected = oracle.conv(shape, x, w, b)
    xb, wb, bb = (lab.DeviceBuffer.from_array(v) for v in (x, w, b))
    if args.requant:
        # bench.py --requant's multipliers, shifts and zero point
        rng = np.random.default_rng(1)
        mult = rng.integers(2 ** 30, 2 ** 31, size=shape.k).astype(np.int32)
        shift = rng.integers(50, 54, size=shape.k).astype(np.int32)
        expected = oracle.requantize(expected, mult, shift, 3)
        mb, sb = lab.DeviceBuffer.from_array(mult), lab.DeviceBuffer.from_array(shift)
        yb = lab.DeviceBuffer(g.output_elements)
        ws_n = lab.requant_workspace_bytes(shape)
    else:
        mb = sb = None
        yb = lab.DeviceBuffer(4 * g.output_elements)
        ws_n = lab.workspace_bytes(kernel, shape)
    ws = lab.DeviceBuffer(ws_n) if ws_n else None
    count = MAX_WORKGROUPS * instrument.WAVES * instrument.SLOTS
    tl = lab.DeviceBuffer(8 * count)
    tl.fill(0)
    setter = _lib.lib().i8conv_timeline_set
    setter.argtypes, setter.restype = [ctypes.c_void_p, ctypes.c_int], None
    setter(ctypes.c_void_p(tl.ptr), MAX_WORKGROUPS)
    print(f"timeline: {args.layer} {shape} kernel={kernel} ({lab.describe(kernel, shape)})",
          flush=True)
    yb.fill(0xA5)
    if args.requant:
        lab.launch_requant(shape, xb, wb, bb, mb, sb, 3, yb, ws, ws_n)
    else:
        lab.launch(kernel, shape, xb, wb, bb, yb, ws, ws_n)
    lab.synchronize()
    got = yb.download(np.int8 if args.requant else np.int32,
                      g.output_elements).reshape(shape.output_shape)
    exact = bool(np.array_equal(got, expected))
    expired = lab.wait_expired()
    print(f"bit-exact vs oracle: {exact}; a bounded wait gave up: {expired}", flush=True)
    result = {"layer": args.layer, "kernel": kernel, "output": "int8" if args.requant else "int32",
              "bit_exact": exact, "wait_gave_up": expired, "steps": args.steps}
    if args.requant:
        # events around K back-to-back launches (bench.py --requant)
        _, mean_ms = lab.measure_requant(shape, xb, wb, bb, mb, sb, 3, yb, ws, ws_n, warmup=20,
                                         iterations=args.steps)
        result["stream_us_per_launch"] = round(mean_ms * 1e3, 3)
    else:
        t = lab.measure_graph(kernel, shape, xb, wb, bb, yb, ws, ws_n, warmup=20,
                              min_warmup_ms=100, iterations=args.steps,
                              launches_per_graph=args.steps, poison_byte=0xA5)
        result["graph_us_per_launch"] = round(t["mean_ms"] * 1e3, 3)
        result["stream_us_per_launch"] = round(t["stream_ms"] * 1e3, 3)
    lab.synchronize()
    stamps = tl.download(np.uint64, count).reshape(MAX_WORKGROUPS, instrument.WAVES,
                                                    instrument.SLOTS)
    for name in ("kernel_rowpass.hip", "kernel_deepk.hip"):
        a = _analyse(stamps, name)
        # the two kernels' stamps differ in which slots the MFMA waves set
        if a is not None and a["mfma_waves"] and a["copy_waves"]:
            result["stamped_kernel"] = name
            result.update(a)
            break
    for buf in (xb, wb, bb, yb, ws, tl, mb, sb):
        if buf is not None:
            buf.close()
    print(f"graph {result.get('graph_us_per_launch', '-')} us/launch, stream "
          f"{result['stream_us_per_launch']} us/launch (K = {args.steps})")
    if "stamped_kernel" not in result:
        print("no stamps: the dispatched kernel is neither stamped kernel, or its grid "
              f"exceeds {MAX_WORKGROUPS} workgroups")
    else:
        print(f"{result['stamped_kernel']}: {result['workgroups']} workgroups, copy waves "
              f"{result['copy_waves']}, MFMA waves {result['mfma_waves']}")
        for name, (lo, med, hi) in result["stamps_us"].items():
            print(f"  {name:44s} {lo:7.3f} {med:7.3f} {hi:7.3f}")
        for key in ("walk_us_median", "walk_clock_ghz_median", "row_step_us_median"):
            if key in result:
                print(f"  {key}: {result[key]}")
    if args.json:
        with open(args.json, "w") as f:
            json.dump(result, f, indent=1)
    return 0 if exact and not expired else 1


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(prog="python -m int8_kernel_lab_amd.timeline")
    sub = ap.add_subparsers(dest="cmd", required=True)
    sub.add_parser("build")
    run = sub.add_parser("run")
    run.add_argument("layer", nargs="?", default="cfg2_resnet_3x3_s1")
    run.add_argument("--steps", type=int, default=20)
    run.add_argument("--json")
    run.add_argument("--requant", action="store_true",
                     help="int8 output (launch_requant), timed like bench.py --requant")
    run.add_argument("--child", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args(argv)
    if args.cmd == "build":
        print(instrument.build())
        return 0
    if args.child:
        return _child(args)
    if not os.path.exists(instrument.LIBRARY):
        raise SystemExit(f"timeline: {instrument.LIBRARY} is missing: run the build step first")
    # The package binds its library at import: a child process loads the
    # stamped one (this process has not touched the GPU).
    path = os.pathsep.join(p for p in (ROOT, os.environ.get("PYTHONPATH")) if p)
    env = dict(os.environ, I8CONV_LIBRARY=instrument.LIBRARY, PYTHONPATH=path)
    cmd = [sys.executable, "-u", "-m", "int8_kernel_lab_amd.timeline", "run", args.layer,
           "--steps", str(args.steps), "--child"] + (["--requant"] if args.requant else [])
    if args.json:
        cmd += ["--json", os.path.abspath(args.json)]
    return subprocess.run(cmd, env=env).returncode


if __name__ == "__main__":
    sys.exit(main())
