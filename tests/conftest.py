"""Shared test setup.

* registers the ``gpu`` marker (tests that need an MI355X);
* puts the repository root on sys.path;
* builds libi8conv.so, the drivers and liboracle.so only when they are missing (the GPU box
  runs the prebuilt files and never builds).
"""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

LIB = os.path.join(ROOT, "int8_kernel_lab_amd", "libi8conv.so")
DRIVER = os.path.join(ROOT, "int8_kernel_lab_amd", "conv_lab")
VENDOR = os.path.join(ROOT, "int8_kernel_lab_amd", "vendor_lab")
ORACLE = os.path.join(ROOT, "oracle", "liboracle.so")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _build_if_missing():
    if not os.path.exists(ORACLE):
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle")], check=True)
    if not (os.path.exists(LIB) and os.path.exists(DRIVER) and os.path.exists(VENDOR)):
        subprocess.run(["make", "-j8", "-C", os.path.join(ROOT, "int8_kernel_lab_amd", "csrc")],
                       check=True)


_build_if_missing()


def say(msg: str) -> None:
    """Names the case before each GPU step (flushed, so a fault still shows it)."""
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="session")
def baseline_cases():
    import int8_kernel_lab_amd as lab
    return lab.load_workloads(os.path.join(lab.WORKLOADS_DIR, "baseline.csv"))


@pytest.fixture(autouse=True)
def _no_expired_waits(request):
    """After every GPU test: no bounded wait (row kernel with copy waves or
    deep-channel split-K) gave up (i8conv_wait_expired), so no launch of the
    test returned I8CONV_OK over an output computed from data that had not
    landed."""
    yield
    if request.node.get_closest_marker("gpu") is None:
        return
    import int8_kernel_lab_amd as lab
    assert not lab.wait_expired(), \
        f"{request.node.nodeid}: a bounded wait gave up; its outputs are not to be trusted"
