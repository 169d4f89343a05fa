"""The give-up path of the bounded chunk waits, forced from the host.

The row kernel with copy waves (config 2's kernel) and the deep-channel
split-K (config 5a's) poll LDS flags that copy waves set as their chunks
land; each wait is bounded, and a wave that gives up records it in a device
word that i8conv_wait_expired reads and clears, so that a launch over data
that had not landed never passes as correct.  Here the host sets the poll
limit to 0 (i8conv_set_wait_spin_limit), so every wait gives up at once:
every wave still runs to its end (the waits only get shorter), the output is
wrong, and the word must read 1 once, then 0.  With the default limit
restored, the same launch is bit-exact and sets nothing.
"""
import os

import numpy as np
import pytest

import int8_kernel_lab_amd as lab
from oracle import oracle
from tests.conftest import say


def _baseline(name):
    return lab.load_case(os.path.join(lab.WORKLOADS_DIR, "baseline.csv"), name)


def test_spin_limit_knob_without_gpu():
    assert lab.wait_spin_limit() == lab.DEFAULT_WAIT_SPIN_LIMIT
    with pytest.raises(lab.I8ConvError):
        lab.set_wait_spin_limit(-1)
    lab.set_wait_spin_limit(7)
    try:
        assert lab.wait_spin_limit() == 7
    finally:
        lab.set_wait_spin_limit(lab.DEFAULT_WAIT_SPIN_LIMIT)
    assert lab.wait_spin_limit() == lab.DEFAULT_WAIT_SPIN_LIMIT


@pytest.mark.gpu
@pytest.mark.parametrize("name,kernel", [("cfg2_resnet_3x3_s1", "halo"),
                                         ("cfg5a_deep_k", "splitk")])
def test_give_up_is_reported_once_then_cleared(name, kernel):
    shape = _baseline(name)
    assert lab.dispatch(shape) == kernel
    x, w, b = lab.make_case_data(shape)
    expected = oracle.conv(shape, x, w, b)
    g = shape.geometry()
    xb, wb, bb = (lab.DeviceBuffer.from_array(a) for a in (x, w, b))
    yb = lab.DeviceBuffer(4 * g.output_elements)
    ws_n = lab.workspace_bytes(kernel, shape)
    ws = lab.DeviceBuffer(ws_n) if ws_n else None
    try:
        assert not lab.wait_expired()
        lab.set_wait_spin_limit(0)
        try:
            say(f"[gpu] {name} ({kernel}) with a wait limit of 0 polls")
            lab.launch(kernel, shape, xb, wb, bb, yb, ws, ws_n)
            lab.synchronize()
        finally:
            lab.set_wait_spin_limit(lab.DEFAULT_WAIT_SPIN_LIMIT)
        assert lab.wait_expired()       # set by the launch with no polls ...
        assert not lab.wait_expired()   # ... and cleared by the read
        # the conv2d helper checks the word after its launch and raises
        lab.set_wait_spin_limit(0)
        try:
            say(f"[gpu] {name} conv2d with a wait limit of 0 polls")
            with pytest.raises(lab.I8ConvError, match="bounded wait gave up"):
                lab.conv2d(x, w, b, shape, kernel=kernel)
        finally:
            lab.set_wait_spin_limit(lab.DEFAULT_WAIT_SPIN_LIMIT)
        assert not lab.wait_expired()   # conv2d's check cleared it
        # the default limit: bit-exact, nothing set
        yb.fill(0xA5)
        say(f"[gpu] {name} with the default wait limit")
        lab.launch(kernel, shape, xb, wb, bb, yb, ws, ws_n)
        lab.synchronize()
        assert not lab.wait_expired()
        got = yb.download(np.int32, g.output_elements).reshape(shape.output_shape)
        np.testing.assert_array_equal(got, expected)
    finally:
        for buf in (xb, wb, bb, yb, ws):
            if buf is not None:
                buf.close()
