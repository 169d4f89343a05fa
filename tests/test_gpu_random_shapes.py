"""Seeded random shapes beyond the hand-picked ones: every eligible kernel,
bit-exact against the oracle, and the dispatched int8 path against
oracle.requantize.  The shapes mix arbitrary filters, strides, paddings,
dilations, channel counts and batch sizes with the lab's favourite
families (3x3 over 64, 128 and 256 channels); every output stays below
64 MiB so the oracle runs in seconds."""
import numpy as np
import pytest

import int8_kernel_lab_amd as lab
from oracle import oracle
from tests.conftest import say
from tests.test_gpu_parity import assert_bit_exact, run_kernel

CHANNELS = [16, 32, 48, 64, 80, 96, 128, 192, 256, 384, 512, 1024]


def random_shapes(seed: int, count: int):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        n = int(rng.integers(1, 5))
        h, w = int(rng.integers(1, 41)), int(rng.integers(1, 41))
        c, k = int(rng.choice(CHANNELS)), int(rng.integers(1, 301))
        r, s = (int(rng.choice([1, 1, 2, 3, 3, 3, 5, 7])) for _ in range(2))
        sh, sw = (int(rng.choice([1, 1, 1, 2, 3])) for _ in range(2))
        ph, pw = int(rng.integers(0, 4)), int(rng.integers(0, 4))
        dh, dw = (int(rng.choice([1, 1, 1, 2, 3])) for _ in range(2))
        if rng.random() < 0.3:
            c = int(rng.choice([64, 128, 256]))
            r = s = 3
            sh = sw = int(rng.choice([1, 2]))
            ph = pw = 1
            dh = dw = 1
            h = w = int(rng.choice([7, 13, 14, 28, 29, 30]))
            k = int(rng.choice([36, 63, 64, 96, 128, 132, 256]))
        shape = lab.ConvShape(n, h, w, c, k, r, s, ph, pw, sh, sw, dh, dw)
        try:
            g = shape.geometry()
        except Exception:
            continue  # no output pixels (a filter wider than the padded image)
        if g is None or g.output_elements <= 0 or g.output_elements * 4 > (64 << 20):
            continue
        out.append(shape)
    return out


SHAPES = random_shapes(20261202, 80)


def test_random_shapes_are_varied():
    # the draw covers every kernel family and the edges it is meant to reach
    dispatched = {lab.dispatch(s) for s in SHAPES}
    assert {"generic", "halo", "splitk"} <= dispatched
    assert any(s.stride_h > 1 for s in SHAPES) and any(s.dilation_h > 1 for s in SHAPES)
    assert any(s.k % 4 for s in SHAPES) and any(s.r != s.s for s in SHAPES)


@pytest.mark.gpu
@pytest.mark.parametrize("i", range(len(SHAPES)))
def test_random_shape_bit_exact(i):
    shape = SHAPES[i]
    x, w, b = lab.make_case_data(shape, seed=100 + i)
    expected = oracle.conv(shape, x, w, b)
    for kernel in lab.KERNELS:
        if not lab.eligible(kernel, shape):
            continue
        say(f"[gpu] random shape {i}: {kernel} {shape}")
        assert_bit_exact(run_kernel(kernel, shape, x, w, b), expected, f"{kernel}/random{i}")
    rng = np.random.default_rng(500 + i)
    mult = (rng.integers(2 ** 29, 2 ** 31, size=shape.k)
            * rng.choice([-1, 1], size=shape.k)).astype(np.int32)
    shift = rng.integers(36, 52, size=shape.k).astype(np.int32)
    zp = int(rng.integers(-20, 20))
    say(f"[gpu] random shape {i}: requant via {lab.dispatch(shape)}")
    got = lab.conv2d_requant(x, w, b, mult, shift, zp, shape)
    np.testing.assert_array_equal(got, oracle.requantize(expected, mult, shift, zp))
