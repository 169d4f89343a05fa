"""ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or the timed CPU baseline.
Each function cites the reference code it restates (see conv_oracle.c).
"""
from __future__ import annotations

import ctypes
import os
from ctypes import c_char_p, POINTER, c_int, c_int32, c_int64, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

FIELDS = ("n", "h", "w", "c", "k", "r", "s", "pad_h", "pad_w",
          "stride_h", "stride_w", "dilation_h", "dilation_w")


class OShape(ctypes.Structure):
    _fields_ = [(f, c_int32) for f in FIELDS]


class OGeometry(ctypes.Structure):
    _fields_ = [("out_h", c_int32), ("out_w", c_int32), ("gemm_m", c_int64),
                ("gemm_n", c_int32), ("gemm_k", c_int32), ("input_elements", c_int64),
                ("filter_elements", c_int64), ("output_elements", c_int64)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
        h = ctypes.CDLL(LIB_PATH)
        h.oracle_derive.restype = c_int
        h.oracle_derive.argtypes = [POINTER(OShape), POINTER(OGeometry)]
        h.oracle_reference_value.restype = c_int32
        h.oracle_reference_value.argtypes = [POINTER(OShape), c_void_p, c_void_p, c_void_p, c_int64]
        h.oracle_conv.restype = c_int
        h.oracle_conv.argtypes = [POINTER(OShape), c_void_p, c_void_p, c_void_p, c_void_p, c_int]
        h.oracle_validate_sampled.restype = c_int64
        h.oracle_validate_sampled.argtypes = [POINTER(OShape), c_void_p, c_void_p, c_void_p, c_void_p]
        h.oracle_strip_eligible_reference.restype = c_int
        h.oracle_strip_eligible_reference.argtypes = [POINTER(OShape)]
        h.oracle_pack_vect_c.restype = None
        h.oracle_pack_vect_c.argtypes = [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32,
                                         c_int32, c_int]
        h.oracle_transpose.restype = None
        h.oracle_transpose.argtypes = [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int]
        h.oracle_requantize.restype = None
        h.oracle_requantize.argtypes = [c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_int32,
                                        c_void_p]
        h.oracle_build_info.restype = c_char_p
        h.oracle_build_info.argtypes = []
        _lib = h
    return _lib


def build_info() -> str:
    """Compiler version and flags liboracle.so was built with."""
    return lib().oracle_build_info().decode()


def _shape(shape) -> OShape:
    return OShape(*[int(getattr(shape, f)) for f in FIELDS])


def derive(shape):
    """conv_shape.cuh:22-35 -> OGeometry, or None where a static_assert fires."""
    g = OGeometry()
    return None if lib().oracle_derive(ctypes.byref(_shape(shape)), ctypes.byref(g)) else g


def _arrays(x, w, b):
    return (np.ascontiguousarray(x, dtype=np.int8), np.ascontiguousarray(w, dtype=np.int8),
            np.ascontiguousarray(b, dtype=np.int32))


def reference_value(shape, x, w, b, index: int) -> int:
    """conv_lab.cu:39-66 for one output index."""
    x, w, b = _arrays(x, w, b)
    return int(lib().oracle_reference_value(ctypes.byref(_shape(shape)), x.ctypes.data,
                                            w.ctypes.data, b.ctypes.data, int(index)))


def conv(shape, x, w, b, threads: int = 0) -> np.ndarray:
    """reference_value for every output index -> NHWK int32 array."""
    g = derive(shape)
    if g is None:
        raise ValueError(f"bad shape {shape}")
    x, w, b = _arrays(x, w, b)
    out = np.empty(g.output_elements, dtype=np.int32)
    threads = threads or min(16, os.cpu_count() or 1)
    rc = lib().oracle_conv(ctypes.byref(_shape(shape)), x.ctypes.data, w.ctypes.data,
                           b.ctypes.data, out.ctypes.data, int(threads))
    assert rc == 0
    return out.reshape(shape.n, g.out_h, g.out_w, shape.k)


def validate_sampled(shape, x, w, b, output) -> int:
    """conv_lab.cu:68-86 sampling rule; first mismatching index or -1."""
    x, w, b = _arrays(x, w, b)
    out = np.ascontiguousarray(output, dtype=np.int32)
    return int(lib().oracle_validate_sampled(ctypes.byref(_shape(shape)), x.ctypes.data,
                                             w.ctypes.data, b.ctypes.data, out.ctypes.data))


def strip_eligible_reference(shape) -> bool:
    """spatial_strip.cuh:11-15 (the reference's predicate, not the gfx950 one)."""
    return bool(lib().oracle_strip_eligible_reference(ctypes.byref(_shape(shape))))


def requantize(acc, mult, shift, zero_point: int) -> np.ndarray:
    """The lab's int32 -> int8 requantization (no reference code; see
    conv_oracle.c): acc [..., K] int32, mult/shift [K] int32 -> int8."""
    acc = np.ascontiguousarray(acc, dtype=np.int32)
    k = acc.shape[-1]
    mult = np.ascontiguousarray(mult, dtype=np.int32).reshape(k)
    shift = np.ascontiguousarray(shift, dtype=np.int32).reshape(k)
    out = np.empty(acc.shape, dtype=np.int8)
    lib().oracle_requantize(acc.ctypes.data, int(acc.size // k), int(k), mult.ctypes.data,
                            shift.ctypes.data, int(zero_point), out.ctypes.data)
    return out


def pack_vect_c(x, vect: int = 32) -> np.ndarray:
    """cudnn_lab.cu:7-18: NHWC (or KRSC) int8 -> N, C/vect, H, W, vect."""
    x = np.ascontiguousarray(x, dtype=np.int8)
    n, h, w, c = x.shape
    out = np.empty(n * h * w * c, dtype=np.int8)
    lib().oracle_pack_vect_c(x.ctypes.data, out.ctypes.data, n, h, w, c, int(vect), 0)
    return out.reshape(n, c // vect, h, w, vect)


def unpack_vect_c(p, vect: int = 32) -> np.ndarray:
    """The inverse of pack_vect_c: N, C/vect, H, W, vect -> NHWC."""
    p = np.ascontiguousarray(p, dtype=np.int8)
    n, g, h, w, v = p.shape
    out = np.empty(p.size, dtype=np.int8)
    lib().oracle_pack_vect_c(p.ctypes.data, out.ctypes.data, n, h, w, g * v, int(v), 1)
    return out.reshape(n, h, w, g * v)


def transpose(x, batch: int, rows: int, cols: int) -> np.ndarray:
    """Batched [rows][cols] -> [cols][rows] of int8 or int32 elements."""
    x = np.ascontiguousarray(x)
    assert x.dtype in (np.int8, np.int32) and x.size == batch * rows * cols
    out = np.empty(x.size, dtype=x.dtype)
    lib().oracle_transpose(x.ctypes.data, out.ctypes.data, batch, rows, cols, x.dtype.itemsize)
    return out.reshape(batch, cols, rows)
