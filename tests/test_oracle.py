"""Pins the CPU oracle (oracle/conv_oracle.c) before anything trusts it.

* golden fixtures written by torch.nn.functional.conv2d in float64
  (tests/golden/make_golden.py), an implementation independent of the
  oracle: every BASELINE configuration at full size (by SHA-256) and tiny
  edge shapes (full arrays);
* a scatter-form brute force (each input pixel pushes its products to the
  outputs that read it), the transpose of the oracle's gather loop, so a
  swapped index or a wrong tap offset fails one of the two;
* invariants that fix the answer without any convolution: zero input or
  zero filter gives the bias, a one-hot filter copies one shifted input
  channel, linearity in the filter, outputs whose window lies wholly in
  the padding equal the bias, int32 wraps like two's complement;
* the sampling rule of conv_lab.cu:68-86, with planted mismatches.
The reference ships no golden vectors; these checks stand in for them.
"""
import hashlib
import json
import os

import numpy as np
import pytest

import int8_kernel_lab_amd as lab
from oracle import oracle
from tests.golden.make_golden import SMALL, out_extent, torch_conv

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
with open(os.path.join(GOLDEN, "baseline_outputs.json")) as _f:
    BASELINE_GOLDEN = json.load(_f)


def sha256(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def rand_case(shape, rng, lo=-128, hi=127):
    x = rng.integers(lo, hi + 1, size=(shape.n, shape.h, shape.w, shape.c), dtype=np.int8)
    w = rng.integers(lo, hi + 1, size=(shape.k, shape.r, shape.s, shape.c), dtype=np.int8)
    b = rng.integers(-(1 << 20), (1 << 20) + 1, size=shape.k, dtype=np.int32)
    return x, w, b


def scatter_conv(shape, x, w, b):
    """Brute force in scatter form: input pixel (iy, ix) feeds output
    (oy, ox) through tap (fy, fx) iff iy = oy*sh + fy*dh - ph and likewise
    for x; written from that relation, not from the oracle's loop."""
    oh = out_extent(shape.h, shape.pad_h, shape.dilation_h, shape.r, shape.stride_h)
    ow = out_extent(shape.w, shape.pad_w, shape.dilation_w, shape.s, shape.stride_w)
    y = np.zeros((shape.n, oh, ow, shape.k), dtype=np.int64)
    wt = w.astype(np.int64)
    for n in range(shape.n):
        for iy in range(shape.h):
            for ix in range(shape.w):
                px = x[n, iy, ix].astype(np.int64)
                for fy in range(shape.r):
                    num_y = iy + shape.pad_h - fy * shape.dilation_h
                    if num_y < 0 or num_y % shape.stride_h or num_y // shape.stride_h >= oh:
                        continue
                    for fx in range(shape.s):
                        num_x = ix + shape.pad_w - fx * shape.dilation_w
                        if num_x < 0 or num_x % shape.stride_w or num_x // shape.stride_w >= ow:
                            continue
                        y[n, num_y // shape.stride_h, num_x // shape.stride_w] += wt[:, fy, fx] @ px
    return (y + b).astype(np.int32)


# ---- golden fixtures ---------------------------------------------------------

@pytest.mark.parametrize("name", sorted(SMALL))
def test_small_cases_match_torch_float64_golden(name):
    golden = np.load(os.path.join(GOLDEN, "small_cases.npz"))
    shape = lab.ConvShape(*[int(v) for v in golden[name + "__shape"]])
    assert shape == SMALL[name]
    x, w, b = lab.make_case_data(shape, seed=7)
    np.testing.assert_array_equal(oracle.conv(shape, x, w, b), golden[name])


@pytest.mark.parametrize("name", sorted(BASELINE_GOLDEN["configs"]))
def test_baseline_configs_match_torch_float64_golden(name, baseline_cases):
    rec = BASELINE_GOLDEN["configs"][name]
    shape = lab.ConvShape(**rec["shape"])
    assert shape == baseline_cases[name.split("@")[0]]
    ranges = {}
    if rec.get("range") == "reference":
        ranges = dict(value_range=(-4, 4), bias_range=(-31, 31))
    x, w, b = lab.make_case_data(shape, **ranges)
    # the generator is part of the contract: same bytes on every host
    assert (sha256(x), sha256(w), sha256(b)) == (
        rec["input_sha256"], rec["filter_sha256"], rec["bias_sha256"])
    y = oracle.conv(shape, x, w, b)
    assert list(y.shape) == rec["output_shape"]
    flat = y.reshape(-1)
    for i, v in rec["samples"]:
        assert int(flat[i]) == v, f"output {i}"
    assert int(flat.astype(np.int64).sum()) == rec["output_sum"]
    assert sha256(y) == rec["output_sha256"]


# ---- independent implementations -------------------------------------------

RANDOM_SHAPES = [
    lab.ConvShape(1, 6, 7, 16, 5, 3, 3, 1, 1, 1, 1, 1, 1),
    lab.ConvShape(2, 9, 8, 32, 3, 3, 2, 2, 0, 2, 1, 1, 2),
    lab.ConvShape(1, 11, 10, 16, 4, 5, 3, 0, 3, 3, 2, 2, 1),
    lab.ConvShape(1, 4, 4, 48, 2, 4, 4, 3, 3, 1, 1, 1, 1),
    lab.ConvShape(2, 3, 5, 16, 6, 1, 1, 1, 0, 2, 2, 1, 1),
    lab.ConvShape(1, 2, 3, 16, 2, 3, 3, 0, 0, 2, 3, 1, 1),   # truncating out_h/out_w
]


@pytest.mark.parametrize("shape", RANDOM_SHAPES, ids=str)
def test_oracle_equals_scatter_brute_force(shape):
    x, w, b = rand_case(shape, np.random.default_rng(11))
    np.testing.assert_array_equal(oracle.conv(shape, x, w, b), scatter_conv(shape, x, w, b))


@pytest.mark.parametrize("seed", range(6))
def test_oracle_equals_torch_on_random_shapes(seed):
    rng = np.random.default_rng(100 + seed)
    r, s = int(rng.integers(1, 6)), int(rng.integers(1, 6))
    shape = lab.ConvShape(int(rng.integers(1, 3)), int(rng.integers(1, 14)),
                          int(rng.integers(1, 14)), 16 * int(rng.integers(1, 5)),
                          int(rng.integers(1, 40)), r, s, int(rng.integers(0, 4)),
                          int(rng.integers(0, 4)), int(rng.integers(1, 4)),
                          int(rng.integers(1, 4)), int(rng.integers(1, 3)),
                          int(rng.integers(1, 3)))
    if oracle.derive(shape) is None:
        pytest.skip(f"empty output for {shape}")
    x, w, b = rand_case(shape, rng)
    np.testing.assert_array_equal(oracle.conv(shape, x, w, b), torch_conv(shape, x, w, b))


def test_reference_value_equals_full_conv_at_every_index():
    shape = RANDOM_SHAPES[1]
    x, w, b = rand_case(shape, np.random.default_rng(3))
    full = oracle.conv(shape, x, w, b, threads=3).reshape(-1)
    for i in range(full.size):
        assert oracle.reference_value(shape, x, w, b, i) == full[i]


# ---- invariants ------------------------------------------------------------

def test_zero_input_or_filter_gives_bias():
    shape = lab.ConvShape(2, 7, 6, 32, 9, 3, 3, 1, 1, 1, 1, 1, 1)
    x, w, b = rand_case(shape, np.random.default_rng(5))
    for xi, wi in ((np.zeros_like(x), w), (x, np.zeros_like(w))):
        y = oracle.conv(shape, xi, wi, b)
        assert np.array_equal(y, np.broadcast_to(b, y.shape))


@pytest.mark.parametrize("fy,fx,c0", [(0, 0, 0), (1, 2, 17), (2, 1, 31), (2, 2, 5)])
def test_one_hot_filter_copies_a_shifted_channel(fy, fx, c0):
    shape = lab.ConvShape(2, 8, 9, 32, 3, 3, 3, 2, 1, 2, 1, 2, 1)
    x, _, b = rand_case(shape, np.random.default_rng(6))
    w = np.zeros((shape.k, 3, 3, 32), np.int8)
    w[1, fy, fx, c0] = 1
    y = oracle.conv(shape, x, w, b)
    g = oracle.derive(shape)
    for oy in range(g.out_h):
        for ox in range(g.out_w):
            iy = oy * shape.stride_h - shape.pad_h + fy * shape.dilation_h
            ix = ox * shape.stride_w - shape.pad_w + fx * shape.dilation_w
            inside = 0 <= iy < shape.h and 0 <= ix < shape.w
            want = (x[:, iy, ix, c0].astype(np.int32) if inside else 0) + b[1]
            assert np.array_equal(y[:, oy, ox, 1], np.broadcast_to(want, (shape.n,)))
            assert np.array_equal(y[:, oy, ox, 0], np.full(shape.n, b[0]))


def test_linear_in_the_filter():
    shape = lab.ConvShape(1, 9, 9, 48, 7, 3, 3, 1, 1, 1, 1, 1, 1)
    rng = np.random.default_rng(8)
    x, w1, b = rand_case(shape, rng, -64, 63)
    _, w2, _ = rand_case(shape, rng, -64, 63)
    zero = np.zeros_like(b)
    y12 = oracle.conv(shape, x, (w1 + w2).astype(np.int8), b).astype(np.int64)
    y1 = oracle.conv(shape, x, w1, zero).astype(np.int64)
    y2 = oracle.conv(shape, x, w2, b).astype(np.int64)
    assert np.array_equal(y12, y1 + y2)


def test_windows_entirely_in_padding_give_bias():
    # pad 3 with a 3x3 filter: the outer ring of outputs reads only padding
    shape = lab.ConvShape(1, 3, 3, 16, 4, 3, 3, 3, 3, 1, 1, 1, 1)
    x, w, b = rand_case(shape, np.random.default_rng(9))
    y = oracle.conv(shape, x, w, b)
    assert y.shape == (1, 7, 7, 4)
    for oy, ox in [(0, 0), (0, 6), (6, 0), (6, 6), (0, 3), (3, 0)]:
        assert np.array_equal(y[0, oy, ox], b)
    assert not np.array_equal(y[0, 3, 3], b)


def test_int32_accumulator_wraps_like_twos_complement():
    # 9 taps x 16384 channels x (-128 * -128) = 9 * 2^28 > 2^31: the int32
    # sum wraps (the reference's int32 accumulator and the MFMA's both do)
    shape = lab.ConvShape(1, 3, 3, 16384, 1, 3, 3, 1, 1, 1, 1, 1, 1)
    x = np.full((1, 3, 3, 16384), -128, np.int8)
    w = np.full((1, 3, 3, 16384), -128, np.int8)
    b = np.array([12345], np.int32)
    y = oracle.conv(shape, x, w, b)
    exact = 9 * 16384 * 16384 + 12345
    wrapped = (exact + 2 ** 31) % 2 ** 32 - 2 ** 31
    assert int(y[0, 1, 1, 0]) == wrapped
    assert int(y[0, 0, 0, 0]) == 4 * 16384 * 16384 + 12345  # corner: 4 taps, no wrap


# ---- the reference's sampling rule (conv_lab.cu:68-86) -----------------------

def test_sampled_validate_full_check_below_65536_outputs():
    shape = lab.ConvShape(1, 16, 16, 64, 64, 3, 3, 1, 1, 1, 1, 1, 1)  # 16384 outputs
    x, w, b = lab.make_case_data(shape)
    y = oracle.conv(shape, x, w, b)
    assert oracle.validate_sampled(shape, x, w, b, y) == -1
    for i in (0, 777, y.size - 1):
        bad = y.copy().reshape(-1)
        bad[i] ^= 1
        assert oracle.validate_sampled(shape, x, w, b, bad) == i


def test_sampled_validate_checks_2048_strided_outputs_above_65536():
    shape = lab.ConvShape(2, 32, 32, 16, 64, 1, 1, 0, 0, 1, 1, 1, 1)  # 131072 outputs
    x, w, b = lab.make_case_data(shape)
    y = oracle.conv(shape, x, w, b).reshape(-1)
    total = y.size
    sampled = 5 * total // 2048
    bad = y.copy()
    bad[sampled] += 1
    assert oracle.validate_sampled(shape, x, w, b, bad) == sampled
    bad = y.copy()
    bad[sampled + 1] += 1  # between samples: the reference's check misses it
    assert oracle.validate_sampled(shape, x, w, b, bad) == -1
