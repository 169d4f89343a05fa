"""MI355X (gfx950) INT8 implicit-GEMM convolution lab: Python host interface.

Mirrors the reference's host-side contract (pthodima/int8_kernel_lab):

* ``ConvShape``            - conv_shape.cuh:5-36 (runtime instead of template)
* ``launch_generic``       - generic_implicit_gemm.cuh:155-165
* ``launch_spatial_strip`` - spatial_strip.cuh:289-301
* ``spatial_strip_eligible`` - kSpatialStripEligible, spatial_strip.cuh:11-15
  (re-derived for the gfx950 strip tile)
* ``DeviceBuffer``         - conv_lab.cu:24-37
* ``measure``              - conv_lab.cu:88-110
* ``load_case``            - gen_case.py:15-36 (case lookup by name)

plus the candidates the reference does not have (``halo``, ``splitk``), the
dispatch policy and a one-call ``conv2d``.  Tensors are NHWC int8 input, KRSC
int8 filter, K int32 bias, NHWK int32 output.  Every GPU call goes through
libi8conv.so; nothing here computes a convolution on the CPU.
"""
from __future__ import annotations

import csv
import ctypes
import os
from dataclasses import dataclass, fields
from typing import Dict, Optional, Tuple

import numpy as np

from . import _lib
from ._lib import I8ConvError, check, lib

__all__ = [
    "ConvShape", "DeviceBuffer", "I8ConvError", "KERNELS", "conv2d", "describe", "dispatch",
    "eligible", "fill_int8", "fill_int32", "kernel_names", "launch",
    "launch_generic", "launch_spatial_strip", "load_case", "load_workloads",
    "make_case_data", "measure", "spatial_strip_eligible", "workspace_bytes",
    "WORKLOADS_DIR", "BASELINE_SEED", "device_count", "device_info", "set_device",
    "synchronize", "requantize", "requant_fused", "requant_workspace_bytes", "launch_requant",
    "conv2d_requant", "measure_requant", "nchw_to_nhwc", "nhwc_to_nchw", "nhwk_to_nkhw",
    "pack_vect_c", "unpack_vect_c", "measure_graph", "measure_store_floor", "measure_lds_probe", "wait_expired", "launch_noalloc",
    "set_wait_spin_limit", "wait_spin_limit", "DEFAULT_WAIT_SPIN_LIMIT",
]

KERNELS = ("generic", "strip", "halo", "splitk")
WORKLOADS_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "workloads")
BASELINE_SEED = 20260925  # the reference's seed (conv_lab.cu:149)
SHAPE_FIELDS = ("n", "h", "w", "c", "k", "r", "s", "pad_h", "pad_w",
                "stride_h", "stride_w", "dilation_h", "dilation_w")


@dataclass(frozen=True)
class ConvShape:
    """Convolution geometry; the 13 ConvShape template parameters."""

    n: int
    h: int
    w: int
    c: int
    k: int
    r: int
    s: int
    pad_h: int = 0
    pad_w: int = 0
    stride_h: int = 1
    stride_w: int = 1
    dilation_h: int = 1
    dilation_w: int = 1

    def c_struct(self) -> _lib.CShape:
        return _lib.CShape(*[int(getattr(self, f)) for f in SHAPE_FIELDS])

    def geometry(self) -> _lib.CGeometry:
        """Derived sizes; ValueError where the reference's static_asserts
        (conv_shape.cuh:34-35) or this ABI's size limits reject the shape."""
        g = _lib.CGeometry()
        status = lib().i8conv_derive(ctypes.byref(self.c_struct()), ctypes.byref(g))
        if status != _lib.OK:
            raise ValueError(f"bad shape {self}: {lib().i8conv_last_error().decode()}")
        return g

    @property
    def out_h(self) -> int:
        return self.geometry().out_h

    @property
    def out_w(self) -> int:
        return self.geometry().out_w

    @property
    def gemm_m(self) -> int:
        return self.geometry().gemm_m

    @property
    def gemm_n(self) -> int:
        return self.geometry().gemm_n

    @property
    def gemm_k(self) -> int:
        return self.geometry().gemm_k

    @property
    def input_elements(self) -> int:
        return self.geometry().input_elements

    @property
    def filter_elements(self) -> int:
        return self.geometry().filter_elements

    @property
    def output_elements(self) -> int:
        return self.geometry().output_elements

    @property
    def output_shape(self) -> Tuple[int, int, int, int]:
        g = self.geometry()
        return (self.n, g.out_h, g.out_w, self.k)

    def ops(self) -> int:
        """2*M*N*K, counting padded taps (the metric's op count)."""
        g = self.geometry()
        return 2 * g.gemm_m * g.gemm_n * g.gemm_k

    def algorithmic_bytes(self) -> int:
        """int8 input + int8 filter + int32 bias + int32 output, once each."""
        g = self.geometry()
        return g.input_elements + g.filter_elements + 4 * self.k + 4 * g.output_elements


# ---- workload tables (schema of the reference's workloads.csv:1) ----------

def load_workloads(path: str) -> Dict[str, ConvShape]:
    """All cases of a workload CSV, by name.  Raises SystemExit for missing
    columns, like gen_case.py:25-27."""
    with open(path, newline="") as stream:
        rows = list(csv.DictReader(stream))
    out: Dict[str, ConvShape] = {}
    for row in rows:
        missing = [f for f in SHAPE_FIELDS if f not in row]
        if "name" not in row or missing:
            raise SystemExit(f"{path} is missing columns: {', '.join((['name'] if 'name' not in row else []) + missing)}")
        out[row["name"]] = ConvShape(*[int(row[f]) for f in SHAPE_FIELDS])
    return out


def load_case(path: str, name: str) -> ConvShape:
    """One case by name (gen_case.py:20-27): SystemExit for an unknown case."""
    cases = load_workloads(path)
    if name not in cases:
        raise SystemExit(f"unknown case {name!r} in {path}")
    return cases[name]


# ---- registry / policy ----------------------------------------------------

def kernel_names() -> Tuple[str, ...]:
    n = lib().i8conv_kernel_count()
    return tuple(lib().i8conv_kernel_name(i).decode() for i in range(n))


def _kernel_id(name: str) -> int:
    kid = lib().i8conv_kernel_id(name.encode())
    if kid < 0:
        raise ValueError(f"unknown kernel {name!r}; known: {kernel_names()}")
    return kid


def eligible(name: str, shape: ConvShape) -> bool:
    return bool(lib().i8conv_eligible(_kernel_id(name), ctypes.byref(shape.c_struct())))


def spatial_strip_eligible(shape: ConvShape) -> bool:
    return bool(lib().i8conv_spatial_strip_eligible(ctypes.byref(shape.c_struct())))


def workspace_bytes(name: str, shape: ConvShape) -> int:
    return int(lib().i8conv_workspace_bytes(_kernel_id(name), ctypes.byref(shape.c_struct())))


def describe(name: str, shape: ConvShape) -> str:
    """One-line description of the tile plan `name` would launch for `shape`."""
    buf = ctypes.create_string_buffer(256)
    check(lib().i8conv_describe(_kernel_id(name), ctypes.byref(shape.c_struct()), buf, 256),
          f"describe {name}")
    return buf.value.decode()


def dispatch(shape: ConvShape) -> str:
    kid = lib().i8conv_dispatch(ctypes.byref(shape.c_struct()))
    if kid < 0:
        shape.geometry()  # raises with the reason
        raise ValueError(f"no kernel for {shape}")
    return lib().i8conv_kernel_name(kid).decode()


# ---- device memory (DeviceBuffer, conv_lab.cu:24-37) -----------------------

class DeviceBuffer:
    """Owned device allocation, freed on close()/garbage collection."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        ptr = ctypes.c_void_p()
        check(lib().i8conv_device_alloc(ctypes.byref(ptr), self.nbytes), "device alloc")
        self.ptr = ptr.value

    @classmethod
    def from_array(cls, array: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(array)
        buf = cls(a.nbytes)
        buf.upload(a)
        return buf

    def upload(self, array: np.ndarray) -> None:
        a = np.ascontiguousarray(array)
        if a.nbytes > self.nbytes:
            raise ValueError("array larger than buffer")
        check(lib().i8conv_copy_to_device(self.ptr, a.ctypes.data, a.nbytes), "copy to device")

    def download(self, dtype, count: int) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        if out.nbytes > self.nbytes:
            raise ValueError("read past buffer end")
        check(lib().i8conv_copy_to_host(out.ctypes.data, self.ptr, out.nbytes), "copy to host")
        return out

    def fill(self, byte: int) -> None:
        check(lib().i8conv_device_fill(self.ptr, int(byte), self.nbytes), "device fill")

    def close(self) -> None:
        if getattr(self, "ptr", None):
            lib().i8conv_device_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _ptr(buf) -> Optional[int]:
    if buf is None:
        return None
    return buf.ptr if isinstance(buf, DeviceBuffer) else int(buf)


def launch(name: str, shape: ConvShape, input, filter, bias, output,
           workspace=None, workspace_nbytes: int = 0, stream=None) -> None:
    """Asynchronous launch of one candidate (raises on a non-OK status, e.g.
    an ineligible shape or a too-small workspace)."""
    if isinstance(workspace, DeviceBuffer) and not workspace_nbytes:
        workspace_nbytes = workspace.nbytes
    status = lib().i8conv_launch(_kernel_id(name), ctypes.byref(shape.c_struct()),
                                 _ptr(input), _ptr(filter), _ptr(bias), _ptr(output),
                                 _ptr(workspace), int(workspace_nbytes), _ptr(stream))
    check(status, f"launch {name}")


NOALLOC_SCRATCH_BYTES = 16 << 20  # the static scratch of launch_noalloc (i8conv.h)


def launch_noalloc(name: str, shape: ConvShape, input, filter, bias, output,
                   stream=None) -> None:
    """i8conv_launch_noalloc: kernel `name` with its workspace (if any) in
    the library's static per-GPU scratch of 16 MiB; allocates nothing.
    Calls that overlap in time on one GPU race on that scratch."""
    check(lib().i8conv_launch_noalloc(_kernel_id(name), ctypes.byref(shape.c_struct()),
                                      _ptr(input), _ptr(filter), _ptr(bias), _ptr(output),
                                      _ptr(stream)), f"launch_noalloc {name}")


def launch_generic(shape: ConvShape, input, filter, bias, output, stream=None) -> None:
    check(lib().i8conv_launch_generic(ctypes.byref(shape.c_struct()), _ptr(input),
                                      _ptr(filter), _ptr(bias), _ptr(output), _ptr(stream)),
          "launch_generic")


def launch_spatial_strip(shape: ConvShape, input, filter, bias, output, stream=None) -> None:
    check(lib().i8conv_launch_spatial_strip(ctypes.byref(shape.c_struct()), _ptr(input),
                                            _ptr(filter), _ptr(bias), _ptr(output),
                                            _ptr(stream)),
          "launch_spatial_strip")


def synchronize() -> None:
    check(lib().i8conv_synchronize(), "synchronize")


def device_count() -> int:
    n = ctypes.c_int()
    check(lib().i8conv_device_count(ctypes.byref(n)), "device count")
    return n.value


def set_device(index: int) -> None:
    """Makes GPU `index` current for the calling thread (buffers and launches
    that follow use it)."""
    check(lib().i8conv_set_device(int(index)), f"set device {index}")


def measure(name: str, shape: ConvShape, input, filter, bias, output, workspace=None,
            workspace_nbytes: int = 0, stream=None, warmup: int = 20,
            iterations: int = 101) -> Tuple[float, float]:
    """(median ms of per-launch event pairs, mean ms per launch of one
    back-to-back batch), conv_lab.cu:88-110 plus the batched figure."""
    if isinstance(workspace, DeviceBuffer) and not workspace_nbytes:
        workspace_nbytes = workspace.nbytes
    med = ctypes.c_float()
    bat = ctypes.c_float()
    status = lib().i8conv_measure(_kernel_id(name), ctypes.byref(shape.c_struct()),
                                  _ptr(input), _ptr(filter), _ptr(bias), _ptr(output),
                                  _ptr(workspace), int(workspace_nbytes), _ptr(stream),
                                  int(warmup), int(iterations), ctypes.byref(med),
                                  ctypes.byref(bat))
    check(status, f"measure {name}")
    return med.value, bat.value


def measure_graph(name: str, shape: ConvShape, input, filter, bias, output, workspace=None,
                  workspace_nbytes: int = 0, warmup: int = 10000, iterations: int = 5000,
                  launches_per_graph: int = 100, min_warmup_ms: float = 0.0,
                  poison_byte: int = -1) -> Dict[str, float]:
    """`iterations` back-to-back launches replayed from HIP graphs
    (i8conv_measure_graph): a main graph of min(launches_per_graph,
    iterations) launches plus a remainder graph, after a warmup of at least
    `warmup` launches and `min_warmup_ms` of wall time; with poison_byte >= 0
    the output is poisoned before the capture and again right before the
    timed replays, so that afterwards it holds only what they wrote.
    Returns the i8conv_graph_timing fields as a dict (mean_ms per launch)."""
    if isinstance(workspace, DeviceBuffer) and not workspace_nbytes:
        workspace_nbytes = workspace.nbytes
    t = _lib.CGraphTiming()
    status = lib().i8conv_measure_graph(_kernel_id(name), ctypes.byref(shape.c_struct()),
                                        _ptr(input), _ptr(filter), _ptr(bias), _ptr(output),
                                        _ptr(workspace), int(workspace_nbytes), int(warmup),
                                        float(min_warmup_ms), int(iterations),
                                        int(launches_per_graph), int(poison_byte),
                                        ctypes.byref(t))
    check(status, f"measure_graph {name}")
    return {f: getattr(t, f) for f, _ in _lib.CGraphTiming._fields_}


def measure_store_floor(output, nbytes: int, workgroups: int = 256, threads: int = 512,
                        lds_bytes: int = 0, write_through: bool = True, warmup: int = 0,
                        min_warmup_ms: float = 100.0, iterations: int = 1000,
                        launches_per_graph: int = 100) -> Dict[str, float]:
    """Times a store-only kernel writing `nbytes` of `output` in the given
    launch shape (i8conv_measure_store_floor): the floor under any kernel of
    that shape that writes that output.  nbytes = 0: an empty kernel."""
    t = _lib.CGraphTiming()
    check(lib().i8conv_measure_store_floor(_ptr(output), int(nbytes), int(workgroups),
                                           int(threads), int(lds_bytes), int(write_through),
                                           int(warmup), float(min_warmup_ms), int(iterations),
                                           int(launches_per_graph), ctypes.byref(t)),
          "measure_store_floor")
    return {f: getattr(t, f) for f, _ in _lib.CGraphTiming._fields_}


LDS_PROBE_PATTERNS = ("linear", "swz128", "stride128", "stride256", "xor_rows", "pitch80")


def measure_lds_probe(pattern: str, sink, workgroups: int = 256, threads: int = 512,
                      reads_per_lane: int = 4097, warmup: int = 0, min_warmup_ms: float = 100.0,
                      iterations: int = 200, launches_per_graph: int = 100) -> Dict[str, float]:
    """Times the LDS read probe (i8conv_measure_lds_probe) in one of
    LDS_PROBE_PATTERNS: ds_read_b128 only, the control pattern for the LDS
    bank-conflict counters.  `sink` holds workgroups * threads int32."""
    t = _lib.CGraphTiming()
    check(lib().i8conv_measure_lds_probe(LDS_PROBE_PATTERNS.index(pattern), _ptr(sink),
                                         int(workgroups), int(threads), int(reads_per_lane),
                                         int(warmup), float(min_warmup_ms), int(iterations),
                                         int(launches_per_graph), ctypes.byref(t)),
          "measure_lds_probe")
    return {f: getattr(t, f) for f, _ in _lib.CGraphTiming._fields_}


def lds_probe_expected(pattern: str, threads: int, reads_per_lane: int):
    """What thread t of any workgroup of the LDS probe stores (numpy int32
    array of `threads` values): the per-lane offsets restated on the host."""
    lane = np.arange(threads) % 64
    row, chunk = lane % 16, lane // 16
    if pattern == "linear":
        base = 16 * lane
    elif pattern == "swz128":
        f = 2 * ((row + (row >> 2)) & 3) + ((row >> 2) & 1)
        base = row * 128 + ((chunk ^ f) << 4)
    elif pattern == "xor_rows":
        base = row * 128 + ((chunk ^ (row & 7) ^ ((row >> 3) & 1)) << 4)
    elif pattern == "pitch80":
        base = 80 * row + 16 * chunk
    elif pattern == "stride128":
        base = 128 * lane
    else:
        base = 256 * lane
    acc = np.zeros(threads, dtype=np.int64)
    for shift in range(4):
        # reads i with i % 4 == shift: (reads_per_lane - shift + 3) // 4 of them
        if ((reads_per_lane - shift + 3) // 4) % 2 == 0:
            continue
        u = (base + 16384 * shift) // 16
        acc ^= u ^ (~u) ^ (3 * u) ^ (u ^ 0x55)
    return (acc & 0xFFFFFFFF).astype(np.uint32).view(np.int32)


def wait_expired() -> bool:
    """True when a bounded wait (row kernel with copy waves or deep-channel
    split-K) gave up since the last call (i8conv_wait_expired: synchronizes
    the device, reads and clears the word); the outputs of the launches
    since then are then not to be trusted."""
    flag = ctypes.c_int()
    check(lib().i8conv_wait_expired(ctypes.byref(flag)), "wait_expired")
    return bool(flag.value)


DEFAULT_WAIT_SPIN_LIMIT = 1 << 20


def set_wait_spin_limit(polls: int) -> None:
    """Test hook for the give-up path (i8conv_set_wait_spin_limit): the polls
    each bounded wait of later launches makes before it gives up; 0 makes
    every wait give up at once (the launch then runs to its end with a wrong
    output that wait_expired() reports)."""
    check(lib().i8conv_set_wait_spin_limit(int(polls)), "set_wait_spin_limit")


def wait_spin_limit() -> int:
    return int(lib().i8conv_wait_spin_limit())


def device_info() -> Dict[str, object]:
    cus = ctypes.c_int()
    clk = ctypes.c_int()
    arch = ctypes.create_string_buffer(128)
    check(lib().i8conv_device_info(ctypes.byref(cus), ctypes.byref(clk), arch, 128), "device info")
    return {"compute_units": cus.value, "clock_khz": clk.value, "arch": arch.value.decode()}


# ---- seeded data -----------------------------------------------------------

def fill_int8(count: int, lo: int, hi: int, state: ctypes.c_uint64) -> np.ndarray:
    out = np.empty(int(count), dtype=np.int8)
    lib().i8conv_fill_int8(out.ctypes.data, out.size, int(lo), int(hi), ctypes.byref(state))
    return out


def fill_int32(count: int, lo: int, hi: int, state: ctypes.c_uint64) -> np.ndarray:
    out = np.empty(int(count), dtype=np.int32)
    lib().i8conv_fill_int32(out.ctypes.data, out.size, int(lo), int(hi), ctypes.byref(state))
    return out


def make_case_data(shape: ConvShape, seed: int = BASELINE_SEED, value_range=(-128, 127),
                   bias_range=(-(1 << 20), 1 << 20)):
    """(input NHWC int8, filter KRSC int8, bias int32): one SplitMix64 stream
    seeded with `seed`, filled input, then filter, then bias."""
    state = ctypes.c_uint64(seed)
    x = fill_int8(shape.input_elements, *value_range, state).reshape(shape.n, shape.h, shape.w, shape.c)
    w = fill_int8(shape.filter_elements, *value_range, state).reshape(shape.k, shape.r, shape.s, shape.c)
    b = fill_int32(shape.k, *bias_range, state)
    return x, w, b


def conv2d(input: np.ndarray, filter: np.ndarray, bias: np.ndarray, shape: ConvShape,
           kernel: str = "dispatch") -> np.ndarray:
    """Runs one candidate (or the dispatched one) on the GPU and returns the
    NHWK int32 output.  Allocates, copies, launches, synchronizes."""
    name = dispatch(shape) if kernel == "dispatch" else kernel
    g = shape.geometry()
    xb = DeviceBuffer.from_array(np.ascontiguousarray(input, dtype=np.int8))
    wb = DeviceBuffer.from_array(np.ascontiguousarray(filter, dtype=np.int8))
    bb = DeviceBuffer.from_array(np.ascontiguousarray(bias, dtype=np.int32))
    yb = DeviceBuffer(4 * g.output_elements)
    ws_n = workspace_bytes(name, shape)
    ws = DeviceBuffer(ws_n) if ws_n else None
    try:
        launch(name, shape, xb, wb, bb, yb, ws, ws_n)
        synchronize()
        if wait_expired():
            raise I8ConvError(_lib.HIP_ERROR, f"conv2d ({name}): a bounded wait gave up "
                              "during the launch; its output is not to be trusted")
        return yb.download(np.int32, g.output_elements).reshape(shape.output_shape)
    finally:
        for b in (xb, wb, bb, yb, ws):
            if b is not None:
                b.close()


# ---- requantized int8 output (no reference counterpart; README.md:89-90) ----

def requant_fused(shape: ConvShape) -> bool:
    """Whether the dispatched kernel requantizes in its own epilogue."""
    return bool(lib().i8conv_requant_fused(ctypes.byref(shape.c_struct())))


def requant_workspace_bytes(shape: ConvShape) -> int:
    return int(lib().i8conv_requant_workspace_bytes(ctypes.byref(shape.c_struct())))


def requantize(acc, pixels: int, channels: int, mult, shift, zero_point: int, output,
               stream=None) -> None:
    """Asynchronous int32 -> int8 requantization of device tensors:
    y = clamp(zero_point + round(acc * mult[k] / 2^shift[k]), -128, 127)."""
    check(lib().i8conv_requantize(_ptr(acc), int(pixels), int(channels), _ptr(mult), _ptr(shift),
                                  int(zero_point), _ptr(output), _ptr(stream)), "requantize")


def launch_requant(shape: ConvShape, input, filter, bias, mult, shift, zero_point: int, output,
                   workspace=None, workspace_nbytes: int = 0, stream=None) -> None:
    """The dispatched convolution with requantized NHWK int8 output."""
    if isinstance(workspace, DeviceBuffer) and not workspace_nbytes:
        workspace_nbytes = workspace.nbytes
    check(lib().i8conv_launch_requant(ctypes.byref(shape.c_struct()), _ptr(input), _ptr(filter),
                                      _ptr(bias), _ptr(mult), _ptr(shift), int(zero_point),
                                      _ptr(output), _ptr(workspace), int(workspace_nbytes),
                                      _ptr(stream)), "launch_requant")


def conv2d_requant(input: np.ndarray, filter: np.ndarray, bias: np.ndarray, mult: np.ndarray,
                   shift: np.ndarray, zero_point: int, shape: ConvShape) -> np.ndarray:
    """The dispatched convolution with int8 output, on host arrays: allocates,
    copies, launches, synchronizes, returns NHWK int8."""
    g = shape.geometry()
    bufs = [DeviceBuffer.from_array(np.ascontiguousarray(a, dtype=t))
            for a, t in ((input, np.int8), (filter, np.int8), (bias, np.int32),
                         (mult, np.int32), (shift, np.int32))]
    yb = DeviceBuffer(max(1, g.output_elements))
    ws_n = requant_workspace_bytes(shape)
    ws = DeviceBuffer(ws_n) if ws_n else None
    try:
        launch_requant(shape, *bufs[:5], zero_point, yb, ws, ws_n)
        synchronize()
        if wait_expired():
            raise I8ConvError(_lib.HIP_ERROR, "conv2d_requant: a bounded wait gave up during "
                              "the launch; its output is not to be trusted")
        return yb.download(np.int8, g.output_elements).reshape(shape.output_shape)
    finally:
        for b in bufs + [yb, ws]:
            if b is not None:
                b.close()


def measure_requant(shape: ConvShape, input, filter, bias, mult, shift, zero_point: int, output,
                    workspace=None, workspace_nbytes: int = 0, warmup: int = 20,
                    iterations: int = 101, stream=None) -> Tuple[float, float]:
    """measure() (conv_lab.cu:88-110) around launch_requant, timed in C++:
    (median ms per launch, mean ms of back-to-back launches)."""
    if isinstance(workspace, DeviceBuffer) and not workspace_nbytes:
        workspace_nbytes = workspace.nbytes
    med, bat = ctypes.c_float(), ctypes.c_float()
    check(lib().i8conv_measure_requant(ctypes.byref(shape.c_struct()), _ptr(input), _ptr(filter),
                                       _ptr(bias), _ptr(mult), _ptr(shift), int(zero_point),
                                       _ptr(output), _ptr(workspace), int(workspace_nbytes),
                                       _ptr(stream), int(warmup), int(iterations),
                                       ctypes.byref(med), ctypes.byref(bat)), "measure_requant")
    return med.value, bat.value


# ---- layout transforms (the step before and after the path) ----------------

def nchw_to_nhwc(src, dst, n: int, c: int, h: int, w: int, stream=None) -> None:
    check(lib().i8conv_nchw_to_nhwc(_ptr(src), _ptr(dst), n, c, h, w, _ptr(stream)),
          "nchw_to_nhwc")


def nhwc_to_nchw(src, dst, n: int, h: int, w: int, c: int, stream=None) -> None:
    check(lib().i8conv_nhwc_to_nchw(_ptr(src), _ptr(dst), n, h, w, c, _ptr(stream)),
          "nhwc_to_nchw")


def nhwk_to_nkhw(src, dst, n: int, h: int, w: int, k: int, stream=None) -> None:
    check(lib().i8conv_nhwk_to_nkhw(_ptr(src), _ptr(dst), n, h, w, k, _ptr(stream)),
          "nhwk_to_nkhw")


def pack_vect_c(src, dst, n: int, h: int, w: int, c: int, vect: int = 32, stream=None) -> None:
    """src/cudnn_lab.cu:7-18 (pack_x / pack_w) on the GPU."""
    check(lib().i8conv_pack_vect_c(_ptr(src), _ptr(dst), n, h, w, c, vect, _ptr(stream)),
          "pack_vect_c")


def unpack_vect_c(src, dst, n: int, h: int, w: int, c: int, vect: int = 32, stream=None) -> None:
    check(lib().i8conv_unpack_vect_c(_ptr(src), _ptr(dst), n, h, w, c, vect, _ptr(stream)),
          "unpack_vect_c")
