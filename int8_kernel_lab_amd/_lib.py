"""ctypes binding of libi8conv.so (the C ABI declared in include/i8conv.h).

The library is built in-tree by ``__graft_entry__.build()`` (or ``make -C
int8_kernel_lab_amd/csrc``).  There is no fallback: if it is missing, every
entry point raises.  The environment variable I8CONV_LIBRARY names another
build of the same ABI to load instead (the timeline tool's clock-stamped
build, int8_kernel_lab_amd/timeline); unset, the in-tree library is loaded.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import (POINTER, c_char_p, c_double, c_float, c_int, c_int32, c_int64, c_size_t,
                    c_uint32, c_uint64, c_void_p)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("I8CONV_LIBRARY") or os.path.join(HERE, "libi8conv.so")

# Status codes (enum i8conv_status).
OK = 0
INELIGIBLE = 1
BAD_SHAPE = 2
BAD_ARGUMENT = 3
WORKSPACE_TOO_SMALL = 4
HIP_ERROR = 5
UNKNOWN_KERNEL = 6


class CShape(ctypes.Structure):
    """struct i8conv_shape: the 13 ConvShape parameters (conv_shape.cuh:5-21)."""

    _fields_ = [(name, c_int32) for name in (
        "n", "h", "w", "c", "k", "r", "s", "pad_h", "pad_w",
        "stride_h", "stride_w", "dilation_h", "dilation_w")]


class CGeometry(ctypes.Structure):
    """struct i8conv_geometry (conv_shape.cuh:22-32)."""

    _fields_ = [("out_h", c_int32), ("out_w", c_int32), ("gemm_m", c_int64),
                ("gemm_n", c_int32), ("gemm_k", c_int32),
                ("input_elements", c_int64), ("filter_elements", c_int64),
                ("output_elements", c_int64)]


class CGraphTiming(ctypes.Structure):
    """struct i8conv_graph_timing (result of i8conv_measure_graph)."""

    _fields_ = [("mean_ms", c_float), ("launches_per_graph", c_int), ("full_replays", c_int),
                ("remainder_launches", c_int), ("warmup_launches", c_int),
                ("warmup_ms", c_float), ("stamped_ms", c_float),
                ("stream_ms", c_float), ("kernel_ms", c_float)]


# name -> (restype, argtypes); every symbol include/i8conv.h declares.
SIGNATURES = {
    "i8conv_derive": (c_int, [POINTER(CShape), POINTER(CGeometry)]),
    "i8conv_kernel_count": (c_int, []),
    "i8conv_kernel_name": (c_char_p, [c_int]),
    "i8conv_kernel_id": (c_int, [c_char_p]),
    "i8conv_eligible": (c_int, [c_int, POINTER(CShape)]),
    "i8conv_workspace_bytes": (c_size_t, [c_int, POINTER(CShape)]),
    "i8conv_describe": (c_int, [c_int, POINTER(CShape), c_char_p, c_size_t]),
    "i8conv_dispatch": (c_int, [POINTER(CShape)]),
    "i8conv_dispatch_workspace_bytes": (c_size_t, [POINTER(CShape)]),
    "i8conv_launch": (c_int, [c_int, POINTER(CShape), c_void_p, c_void_p, c_void_p,
                              c_void_p, c_void_p, c_size_t, c_void_p]),
    "i8conv_launch_generic": (c_int, [POINTER(CShape), c_void_p, c_void_p, c_void_p,
                                      c_void_p, c_void_p]),
    "i8conv_launch_spatial_strip": (c_int, [POINTER(CShape), c_void_p, c_void_p,
                                            c_void_p, c_void_p, c_void_p]),
    "i8conv_spatial_strip_eligible": (c_int, [POINTER(CShape)]),
    "i8conv_launch_noalloc": (c_int, [c_int, POINTER(CShape), c_void_p, c_void_p, c_void_p,
                                      c_void_p, c_void_p]),
    "i8conv_launch_dispatched": (c_int, [POINTER(CShape), c_void_p, c_void_p, c_void_p,
                                         c_void_p, c_void_p, c_size_t, c_void_p]),
    "i8conv_requantize": (c_int, [c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_int32,
                                  c_void_p, c_void_p]),
    "i8conv_requant_fused": (c_int, [POINTER(CShape)]),
    "i8conv_requant_workspace_bytes": (c_size_t, [POINTER(CShape)]),
    "i8conv_launch_requant": (c_int, [POINTER(CShape), c_void_p, c_void_p, c_void_p, c_void_p,
                                      c_void_p, c_int32, c_void_p, c_void_p, c_size_t,
                                      c_void_p]),
    "i8conv_measure_requant": (c_int, [POINTER(CShape), c_void_p, c_void_p, c_void_p, c_void_p,
                                       c_void_p, c_int32, c_void_p, c_void_p, c_size_t, c_void_p,
                                       c_int, c_int, POINTER(c_float), POINTER(c_float)]),
    "i8conv_nchw_to_nhwc": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p]),
    "i8conv_nhwc_to_nchw": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p]),
    "i8conv_nhwk_to_nkhw": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p]),
    "i8conv_pack_vect_c": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int,
                                   c_void_p]),
    "i8conv_unpack_vect_c": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int,
                                     c_void_p]),
    "i8conv_device_count": (c_int, [POINTER(c_int)]),
    "i8conv_set_device": (c_int, [c_int]),
    "i8conv_device_alloc": (c_int, [POINTER(c_void_p), c_size_t]),
    "i8conv_device_free": (c_int, [c_void_p]),
    "i8conv_copy_to_device": (c_int, [c_void_p, c_void_p, c_size_t]),
    "i8conv_copy_to_host": (c_int, [c_void_p, c_void_p, c_size_t]),
    "i8conv_device_fill": (c_int, [c_void_p, c_int, c_size_t]),
    "i8conv_synchronize": (c_int, []),
    "i8conv_stream_create": (c_int, [POINTER(c_void_p)]),
    "i8conv_stream_destroy": (c_int, [c_void_p]),
    "i8conv_wait_expired": (c_int, [POINTER(c_int)]),
    "i8conv_set_wait_spin_limit": (c_int, [c_int]),
    "i8conv_wait_spin_limit": (c_int, []),
    "i8conv_device_info": (c_int, [POINTER(c_int), POINTER(c_int), c_char_p, c_size_t]),
    "i8conv_measure_graph": (c_int, [c_int, POINTER(CShape), c_void_p, c_void_p, c_void_p,
                                     c_void_p, c_void_p, c_size_t, c_int, c_double, c_int,
                                     c_int, c_int, POINTER(CGraphTiming)]),
    "i8conv_measure_store_floor": (c_int, [c_void_p, c_size_t, c_int, c_int, c_size_t, c_int,
                                           c_int, c_double, c_int, c_int,
                                           POINTER(CGraphTiming)]),
    "i8conv_measure_lds_probe": (c_int, [c_int, c_void_p, c_int, c_int, c_int, c_int, c_double,
                                         c_int, c_int, POINTER(CGraphTiming)]),
    "i8conv_measure": (c_int, [c_int, POINTER(CShape), c_void_p, c_void_p, c_void_p,
                               c_void_p, c_void_p, c_size_t, c_void_p, c_int, c_int,
                               POINTER(c_float), POINTER(c_float)]),
    "i8conv_status_string": (c_char_p, [c_int]),
    "i8conv_last_error": (c_char_p, []),
    "i8conv_fill_int8": (None, [c_void_p, c_size_t, c_int, c_int, POINTER(c_uint64)]),
    "i8conv_fill_int32": (None, [c_void_p, c_size_t, c_int32, c_int32, POINTER(c_uint64)]),
}

_lib = None


def lib() -> ctypes.CDLL:
    """Loads libi8conv.so once; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; "
                "g.build()'` (there is no CPU fallback)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


class I8ConvError(RuntimeError):
    """A non-OK i8conv_status, with the library's last error text."""

    def __init__(self, status: int, what: str):
        self.status = status
        text = lib().i8conv_status_string(status).decode()
        detail = lib().i8conv_last_error().decode()
        super().__init__(f"{what}: {text}" + (f" ({detail})" if detail else ""))


def check(status: int, what: str) -> None:
    if status != OK:
        raise I8ConvError(status, what)
