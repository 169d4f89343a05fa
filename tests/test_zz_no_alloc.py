"""i8conv_launch_noalloc: the launch entry point that allocates nothing.

It runs a kernel with its workspace in the library's static per-GPU scratch
(16 MiB).  The GPU test compares it with i8conv_launch (the same kernel with
a caller-allocated workspace) bit for bit, on two calls in a row, the second
with a smaller input, so that a stale or misaddressed scratch would show;
the CPU test checks the size limit without touching the GPU.
"""
import ctypes
import os

import numpy as np
import pytest

import int8_kernel_lab_amd as lab
from int8_kernel_lab_amd import _lib
from oracle import oracle
from tests.conftest import say

FAKE = 0x10000  # a 64 KB-aligned address that is never dereferenced


def test_noalloc_rejects_workspaces_beyond_the_scratch(baseline_cases):
    # split-K on the stride-2 layer needs 25088 x 256 int32 per split, far
    # beyond 16 MiB: rejected before any HIP call
    cfg3 = baseline_cases["cfg3_down_3x3_s2"]
    assert lab.workspace_bytes("splitk", cfg3) > lab.NOALLOC_SCRATCH_BYTES
    rc = _lib.lib().i8conv_launch_noalloc(3, ctypes.byref(cfg3.c_struct()), FAKE, FAKE, FAKE,
                                          FAKE, None)
    assert rc == _lib.WORKSPACE_TOO_SMALL
    msg = _lib.lib().i8conv_last_error().decode()
    assert str(lab.NOALLOC_SCRATCH_BYTES) in msg and "splitk" in msg
    # errors i8conv_launch reports come through unchanged
    assert _lib.lib().i8conv_launch_noalloc(9, ctypes.byref(cfg3.c_struct()), FAKE, FAKE, FAKE,
                                            FAKE, None) == _lib.UNKNOWN_KERNEL
    bad = lab.ConvShape(1, 8, 8, 24, 8, 3, 3, 1, 1).c_struct()
    assert _lib.lib().i8conv_launch_noalloc(3, ctypes.byref(bad), FAKE, FAKE, FAKE, FAKE,
                                            None) == _lib.BAD_SHAPE


@pytest.mark.gpu
def test_noalloc_matches_launch_on_two_calls(baseline_cases):
    # first the deep-K layer (12.25 MiB of partial sums: most of the
    # scratch), then a smaller split-K layer that reuses the scratch the
    # first call left full
    cases = [("cfg5a_deep_k", baseline_cases["cfg5a_deep_k"]),
             ("smaller 2x7x7x1024->256", lab.ConvShape(2, 7, 7, 1024, 256, 3, 3, 1, 1))]
    assert lab.workspace_bytes("splitk", cases[1][1]) < lab.workspace_bytes("splitk", cases[0][1])
    for label, shape in cases:
        need = lab.workspace_bytes("splitk", shape)
        assert 0 < need <= lab.NOALLOC_SCRATCH_BYTES
        g = shape.geometry()
        x, w, b = lab.make_case_data(shape)
        bufs = [lab.DeviceBuffer.from_array(a) for a in (x, w, b)]
        ws = lab.DeviceBuffer(need)
        y_ref = lab.DeviceBuffer(4 * g.output_elements)
        y = lab.DeviceBuffer(4 * g.output_elements)
        try:
            say(f"[gpu] splitk with a caller workspace on {label}")
            y_ref.fill(0xA5)
            lab.launch("splitk", shape, *bufs, y_ref, ws, need)
            lab.synchronize()
            expected = y_ref.download(np.int32, g.output_elements)
            say(f"[gpu] launch_noalloc splitk on {label}")
            y.fill(0x5A)
            lab.launch_noalloc("splitk", shape, *bufs, y)
            lab.synchronize()
            got = y.download(np.int32, g.output_elements)
            assert np.array_equal(got, expected), \
                f"{label}: {int(np.count_nonzero(got != expected))} outputs differ"
            # and both equal the oracle
            assert np.array_equal(got.reshape(shape.output_shape), oracle.conv(shape, x, w, b))
        finally:
            for buf in bufs + [ws, y_ref, y]:
                buf.close()
