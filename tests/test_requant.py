"""The int32 -> int8 requantization: the oracle pinned by exact rational
arithmetic (CPU), and the GPU paths (standalone kernel, fused epilogue,
dispatched conv + requant) bit-exact against the oracle.

The reference has no requantizing code (its cuDNN comparison writes INT8,
README.md:89-90); the lab defines
    y = clamp(zero_point + round(acc * mult[k] / 2^shift[k]), -128, 127)
with shift clamped to [0, 62] and ties rounded away from zero.  The checks
below compute that from its definition with Python's exact Fractions, not
by repeating the oracle's shift-and-add steps.
"""
from fractions import Fraction
import math

import numpy as np
import pytest

from oracle import oracle


def exact_requant(acc: int, mult: int, shift: int, zp: int) -> int:
    s = min(max(shift, 0), 62)
    x = Fraction(acc * mult, 2 ** s)
    mag = math.floor(abs(x) + Fraction(1, 2))  # ties away from zero
    r = mag if x >= 0 else -mag
    return max(-128, min(127, r + zp))


def _check(acc, mult, shift, zp):
    got = oracle.requantize(acc, mult, shift, zp)
    k = acc.shape[-1]
    flat = acc.reshape(-1, k)
    exp = np.array([[exact_requant(int(a), int(mult[j]), int(shift[j]), zp)
                     for j, a in enumerate(row)] for row in flat], dtype=np.int8).reshape(acc.shape)
    np.testing.assert_array_equal(got, exp)


def test_requant_oracle_matches_exact_rationals_random():
    rng = np.random.default_rng(7)
    k = 13
    acc = rng.integers(-(2 ** 31), 2 ** 31, size=(40, k), dtype=np.int64).astype(np.int32)
    acc[0, :] = np.iinfo(np.int32).min
    acc[1, :] = np.iinfo(np.int32).max
    mult = rng.integers(-(2 ** 31), 2 ** 31, size=k, dtype=np.int64).astype(np.int32)
    mult[0] = np.iinfo(np.int32).min
    mult[1] = np.iinfo(np.int32).max
    shift = rng.integers(0, 63, size=k).astype(np.int32)
    shift[2], shift[3] = 0, 62
    for zp in (0, -128, 5, 127):
        _check(acc, mult, shift, zp)


def test_requant_oracle_typical_scales():
    # the usual case: a positive Q31 multiplier in [2^30, 2^31) and shifts
    # that bring accumulators of a few million into int8 range
    rng = np.random.default_rng(11)
    k = 8
    acc = rng.integers(-(2 ** 24), 2 ** 24, size=(200, k)).astype(np.int32)
    mult = rng.integers(2 ** 30, 2 ** 31, size=k).astype(np.int32)
    shift = rng.integers(40, 56, size=k).astype(np.int32)
    _check(acc, mult, shift, 3)


def test_requant_oracle_special_cases():
    acc = np.array([[-300, -129, -128, -1, 0, 1, 127, 128, 300]], dtype=np.int32)
    k = acc.shape[1]
    one = np.ones(k, dtype=np.int32)
    zero = np.zeros(k, dtype=np.int32)
    # mult 1, shift 0: saturation of acc + zp
    np.testing.assert_array_equal(oracle.requantize(acc, one, zero, 0)[0],
                                  [-128, -128, -128, -1, 0, 1, 127, 127, 127])
    np.testing.assert_array_equal(oracle.requantize(acc, one, zero, 10)[0],
                                  [-128, -119, -118, 9, 10, 11, 127, 127, 127])
    # mult 2^s with shift s is the identity before saturation
    for s in (1, 7, 30):
        np.testing.assert_array_equal(oracle.requantize(acc, one * (1 << s) if s < 31 else one,
                                                        one * s, 0),
                                      oracle.requantize(acc, one, zero, 0))
    # halves round away from zero: acc * 1 / 2
    halves = np.array([[-5, -3, -1, 1, 3, 5, -4, 4]], dtype=np.int32)
    h1 = np.ones(halves.shape[1], dtype=np.int32)
    np.testing.assert_array_equal(oracle.requantize(halves, h1, h1, 0)[0],
                                  [-3, -2, -1, 1, 2, 3, -2, 2])
    # shift outside [0, 62] is clamped
    np.testing.assert_array_equal(oracle.requantize(acc, one, zero - 5, 0),
                                  oracle.requantize(acc, one, zero, 0))
    big = np.full(k, 2 ** 31 - 1, dtype=np.int32)
    np.testing.assert_array_equal(oracle.requantize(acc, big, zero + 100, 0),
                                  oracle.requantize(acc, big, zero + 62, 0))


def test_requant_oracle_detects_planted_rounding_error():
    # a floor instead of ties-away rounding differs from the exact result
    acc = np.array([[3]], dtype=np.int32)
    assert exact_requant(3, 1, 1, 0) == 2
    assert int(oracle.requantize(acc, np.array([1], np.int32), np.array([1], np.int32), 0)[0, 0]) == 2
    assert (3 * 1) >> 1 == 1  # the floor a plausible mistake would give


# ---- ABI (no GPU) -----------------------------------------------------------

import int8_kernel_lab_amd as lab
from int8_kernel_lab_amd import _lib


def _baseline(name):
    import os
    return lab.load_case(os.path.join(lab.WORKLOADS_DIR, "baseline.csv"), name)


def test_requant_fused_where_the_dispatched_kernel_requantizes():
    assert lab.requant_fused(_baseline("cfg2_resnet_3x3_s1"))
    # the generic kernel's pointwise streaming form, slices of 64 channels
    assert lab.requant_fused(_baseline("cfg4a_pointwise_1x1"))
    assert lab.requant_workspace_bytes(_baseline("cfg4a_pointwise_1x1")) == 0
    # the pipelined GEMM's epilogue and split-K's second pass
    for name in ("cfg3_down_3x3_s2", "cfg5b_dilated", "cfg5a_deep_k"):
        assert lab.requant_fused(_baseline(name)), name
    # the row kernel without copy waves (C = 64) has no requantizing epilogue
    assert not lab.requant_fused(_baseline("cfg1_smoke"))
    # pointwise slices of 32 channels (C = 512) have no requantizing
    # instance: the pipelined GEMM (C % 128 == 0) requantizes in its
    # epilogue instead; slices of 256 (C = 64, N = 256) or 32 channels with
    # C = 64 go unfused (the register-staged GEMM has no such epilogue)
    wide = lab.ConvShape(1, 8, 8, 512, 64, 1, 1, 0, 0, 1, 1, 1, 1)
    assert lab.requant_fused(wide) and lab.requant_workspace_bytes(wide) == 0
    for shape in (lab.ConvShape(1, 8, 8, 64, 256, 1, 1, 0, 0, 1, 1, 1, 1),
                  lab.ConvShape(1, 8, 8, 64, 32, 1, 1, 0, 0, 1, 1, 1, 1)):
        assert not lab.requant_fused(shape), shape


def test_requant_workspace_sizes():
    s2 = _baseline("cfg2_resnet_3x3_s1")
    assert lab.requant_workspace_bytes(s2) == 0
    # the pipelined GEMM's epilogue writes no int32 tensor: no workspace
    s3 = _baseline("cfg3_down_3x3_s2")
    assert lab.requant_workspace_bytes(s3) == 0
    # split-K's second pass requantizes: only the partial sums
    s5 = _baseline("cfg5a_deep_k")
    assert lab.requant_workspace_bytes(s5) == lab.workspace_bytes("splitk", s5)
    # unfused (the C = 64 row kernel): the int32 output, 256-byte aligned
    s1 = _baseline("cfg1_smoke")
    acc = (s1.output_elements * 4 + 255) // 256 * 256
    assert lab.requant_workspace_bytes(s1) == acc + lab.workspace_bytes(lab.dispatch(s1), s1)


def test_requant_launch_errors_without_gpu():
    s3 = _baseline("cfg3_down_3x3_s2")
    fake = 1 << 20  # never dereferenced: the checks fail before any launch
    # unfused (the C = 64 row kernel) without a workspace
    with pytest.raises(lab.I8ConvError) as e:
        lab.launch_requant(_baseline("cfg1_smoke"), fake, fake, fake, fake, fake, 0, fake, None, 0)
    assert e.value.status == _lib.WORKSPACE_TOO_SMALL
    # the pipelined GEMM fuses only with 16-byte aligned mult and shift: a
    # multiplier array at +4 bytes takes the unfused way, which needs the
    # int32 workspace
    with pytest.raises(lab.I8ConvError, match="16-byte aligned") as e:
        lab.launch_requant(s3, fake, fake, fake, fake + 4, fake, 0, fake, None, 0)
    assert e.value.status == _lib.WORKSPACE_TOO_SMALL
    # fused split-K still needs its partial sums' workspace
    with pytest.raises(lab.I8ConvError, match="split-K") as e:
        lab.launch_requant(_baseline("cfg5a_deep_k"), fake, fake, fake, fake, fake, 0, fake,
                           None, 0)
    assert e.value.status == _lib.WORKSPACE_TOO_SMALL
    with pytest.raises(lab.I8ConvError) as e:
        lab.launch_requant(s3, fake, fake, fake, None, fake, 0, fake, fake, 1 << 30)
    assert e.value.status == _lib.BAD_ARGUMENT
    with pytest.raises(lab.I8ConvError) as e:
        lab.requantize(fake, 10, 0, fake, fake, 0, fake)
    assert e.value.status == _lib.BAD_ARGUMENT
    # the pointwise form fuses only with 16-byte aligned bias, mult, shift
    # and output; an output at +4 bytes needs the unfused workspace
    s4a = _baseline("cfg4a_pointwise_1x1")
    with pytest.raises(lab.I8ConvError, match="16-byte aligned") as e:
        lab.launch_requant(s4a, fake, fake, fake, fake, fake, 0, fake + 4, None, 0)
    assert e.value.status == _lib.WORKSPACE_TOO_SMALL


# ---- GPU: bit-exact against the oracle --------------------------------------

def _qparams(k, seed=3):
    """Per-channel parameters that map accumulators of about 2^28 onto int8,
    plus a few saturating and exactly-representable channels."""
    rng = np.random.default_rng(seed)
    mult = rng.integers(2 ** 30, 2 ** 31, size=k).astype(np.int32)
    shift = rng.integers(50, 54, size=k).astype(np.int32)
    if k > 4:
        mult[0], shift[0] = 1, 0            # saturates nearly everything
        mult[1], shift[1] = -(2 ** 31), 58  # negative multiplier
        mult[2], shift[2] = 1 << 20, 20     # identity before saturation
        mult[3], shift[3] = 3, 62           # everything rounds to 0
    return mult, shift


@pytest.mark.gpu
@pytest.mark.parametrize("channels", [64, 6])
def test_requantize_kernel_bit_exact(channels):
    from tests.conftest import say
    rng = np.random.default_rng(channels)
    pixels = 4099
    acc = rng.integers(-(2 ** 31), 2 ** 31, size=(pixels, channels), dtype=np.int64).astype(np.int32)
    mult, shift = _qparams(channels)
    say(f"[gpu] requantize {pixels}x{channels}")
    bufs = [lab.DeviceBuffer.from_array(a) for a in (acc, mult, shift)]
    out = lab.DeviceBuffer(pixels * channels)
    out.fill(0x5A)
    lab.requantize(bufs[0], pixels, channels, bufs[1], bufs[2], -7, out)
    lab.synchronize()
    got = out.download(np.int8, pixels * channels).reshape(pixels, channels)
    np.testing.assert_array_equal(got, oracle.requantize(acc, mult, shift, -7))


REQUANT_CASES = ["cfg1_smoke", "cfg2_resnet_3x3_s1", "cfg3_down_3x3_s2", "cfg4a_pointwise_1x1",
                 "cfg4b_k36_tail", "cfg5a_deep_k", "cfg5b_dilated"]


@pytest.mark.gpu
@pytest.mark.parametrize("name", REQUANT_CASES)
def test_conv_requant_bit_exact_on_baseline_configs(name):
    from tests.conftest import say
    shape = _baseline(name)
    x, w, b = lab.make_case_data(shape)
    mult, shift = _qparams(shape.k)
    say(f"[gpu] conv2d_requant {name} fused={lab.requant_fused(shape)}")
    got = lab.conv2d_requant(x, w, b, mult, shift, 3, shape)
    exp = oracle.requantize(oracle.conv(shape, x, w, b), mult, shift, 3)
    np.testing.assert_array_equal(got, exp)


FUSED_EDGES = {
    # the row kernel with copy waves in its int8 form: channel tail (byte
    # stores), one, two and four fragments per row, unequal blocks, no padding
    "k126_tail": lab.ConvShape(4, 30, 30, 128, 126, 3, 3, 1, 1, 1, 1, 1, 1),
    "nfr1": lab.ConvShape(8, 14, 14, 128, 128, 3, 3, 1, 1, 1, 1, 1, 1),
    "nfr4": lab.ConvShape(4, 20, 60, 128, 64, 3, 3, 1, 1, 1, 1, 1, 1),
    "r2_uneven": lab.ConvShape(8, 28, 28, 128, 128, 3, 3, 1, 1, 1, 1, 1, 1),
    "pad0": lab.ConvShape(4, 30, 30, 128, 64, 3, 3, 0, 0, 1, 1, 1, 1),
    # blocks of 5/4 and 6/5 rows
    "split_r5_w29": lab.ConvShape(32, 19, 29, 128, 128, 3, 3, 1, 1, 1, 1, 1, 1),
    "split_r6_k96": lab.ConvShape(32, 22, 13, 128, 96, 3, 3, 1, 1, 1, 1, 1, 1),
}


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(FUSED_EDGES))
def test_fused_requant_edges_bit_exact(name):
    from tests.conftest import say
    shape = FUSED_EDGES[name]
    assert lab.requant_fused(shape), name
    x, w, b = lab.make_case_data(shape, seed=99)
    mult, shift = _qparams(shape.k, seed=5)
    say(f"[gpu] fused requant {name} {shape}")
    got = lab.conv2d_requant(x, w, b, mult, shift, -20, shape)
    exp = oracle.requantize(oracle.conv(shape, x, w, b), mult, shift, -20)
    np.testing.assert_array_equal(got, exp)


SPLITK_RQ = {
    # split-K's reduce requantizing as it adds the splits (N % 4 == 0): the
    # deep-channel form with a 4-channel tail past 256; the GEMM form (1x1,
    # 13x13, C = 1024); N % 4 != 0 takes the int32 pass instead
    "deepc_k260": lab.ConvShape(4, 5, 9, 4096, 260, 3, 3, 0, 0, 1, 1, 1, 1),
    "gemm_1x1_13": lab.ConvShape(1, 13, 13, 1024, 256, 1, 1, 0, 0, 1, 1, 1, 1),
    "k66_pass": lab.ConvShape(1, 7, 7, 2048, 66, 3, 3, 1, 1, 1, 1, 1, 1),
}


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(SPLITK_RQ))
def test_splitk_requant_bit_exact(name):
    from tests.conftest import say
    shape = SPLITK_RQ[name]
    assert lab.dispatch(shape) == "splitk", name
    x, w, b = lab.make_case_data(shape, seed=17)
    mult, shift = _qparams(shape.k, seed=18)
    say(f"[gpu] split-K requant {name} {shape}")
    got = lab.conv2d_requant(x, w, b, mult, shift, -9, shape)
    exp = oracle.requantize(oracle.conv(shape, x, w, b), mult, shift, -9)
    np.testing.assert_array_equal(got, exp)


GEMM_RQ = {
    # the pipelined GEMM's requantizing epilogue (C % 128 == 0, N % 4 == 0):
    # a 1x1 layer whose pointwise form has no requantizing instance (C =
    # 512); a stride-2 layer with a 4-channel tail past 128; C = 64 takes the
    # register-staged GEMM and the int32 pass
    "c512_1x1_k64": lab.ConvShape(1, 9, 9, 512, 64, 1, 1, 0, 0, 1, 1, 1, 1),
    "s2_k132": lab.ConvShape(8, 28, 28, 128, 132, 3, 3, 1, 1, 2, 2, 1, 1),
    "c64_s2_pass": lab.ConvShape(2, 16, 16, 64, 64, 3, 3, 1, 1, 2, 2, 1, 1),
}


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(GEMM_RQ))
def test_gemm_requant_bit_exact(name):
    from tests.conftest import say
    shape = GEMM_RQ[name]
    assert lab.dispatch(shape) == "generic", name
    x, w, b = lab.make_case_data(shape, seed=19)
    mult, shift = _qparams(shape.k, seed=20)
    say(f"[gpu] generic requant {name} {shape}")
    got = lab.conv2d_requant(x, w, b, mult, shift, 11, shape)
    exp = oracle.requantize(oracle.conv(shape, x, w, b), mult, shift, 11)
    np.testing.assert_array_equal(got, exp)


POINTWISE_RQ = {
    # the generic kernel's pointwise form with its requantizing epilogue:
    # one 64-channel group (whole 128-byte lines of two pixels per store)
    # with a pixel tail; two groups paired per store; 128-channel slices (2);
    # 64-channel slices (2 and 4: half-line ordinary stores)
    "c64_k64_tail": lab.ConvShape(3, 7, 9, 64, 64, 1, 1, 0, 0, 1, 1, 1, 1),
    "c64_k128": lab.ConvShape(2, 11, 13, 64, 128, 1, 1, 0, 0, 1, 1, 1, 1),
    "c128_k128_tail": lab.ConvShape(1, 5, 7, 128, 128, 1, 1, 0, 0, 1, 1, 1, 1),
    "c128_k256_slices2": lab.ConvShape(5, 13, 17, 128, 256, 1, 1, 0, 0, 1, 1, 1, 1),
    "c256_k128_slices2": lab.ConvShape(1, 52, 51, 256, 128, 1, 1, 0, 0, 1, 1, 1, 1),
    "c256_k256_slices4": lab.ConvShape(2, 9, 10, 256, 256, 1, 1, 0, 0, 1, 1, 1, 1),
}


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(POINTWISE_RQ))
def test_pointwise_requant_bit_exact(name):
    from tests.conftest import say
    shape = POINTWISE_RQ[name]
    assert lab.requant_fused(shape), name
    x, w, b = lab.make_case_data(shape, seed=11)
    mult, shift = _qparams(shape.k, seed=12)
    say(f"[gpu] pointwise requant {name} {shape}")
    got = lab.conv2d_requant(x, w, b, mult, shift, 5, shape)
    exp = oracle.requantize(oracle.conv(shape, x, w, b), mult, shift, 5)
    np.testing.assert_array_equal(got, exp)


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["c64_k64_tail", "c128_k256_slices2", "c256_k256_slices4",
                                  "c64_k128"])
@pytest.mark.parametrize("mixed", [False, True])
def test_pointwise_requant_short_form_bit_exact(name, mixed):
    # every channel with shift >= 33: every wave takes the short form; mixed:
    # one channel of the last slice with shift 32 sends that slice's waves
    # to the exact form while the others stay short
    from tests.conftest import say
    shape = POINTWISE_RQ[name]
    x, w, b = lab.make_case_data(shape, seed=15)
    rng = np.random.default_rng(16)
    mult = (rng.integers(2 ** 30, 2 ** 31, size=shape.k)
            * rng.choice([-1, 1], size=shape.k)).astype(np.int32)
    mult[9] = -(2 ** 31)
    shift = rng.integers(44, 47, size=shape.k).astype(np.int32)
    if mixed:
        shift[shape.k - 3] = 32
    say(f"[gpu] pointwise requant short form {name} mixed={mixed}")
    got = lab.conv2d_requant(x, w, b, mult, shift, -3, shape)
    exp = oracle.requantize(oracle.conv(shape, x, w, b), mult, shift, -3)
    assert len(np.unique(exp)) > 200
    np.testing.assert_array_equal(got, exp)


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["c64_k64_tail", "c128_k256_slices2", "c256_k256_slices4",
                                  "c64_k128"])
@pytest.mark.parametrize("mixed", [False, True])
def test_pointwise_requant_odd_form_bit_exact(name, mixed):
    # multipliers of both signs with 0..8 trailing zeros and shifts raised to
    # match: every wave takes the odd-multiplier form, whose normalization
    # (mult = mo 2^t, s' = s - t) decides every value; mixed: one channel of
    # the last slice with s' = 32 (outside the odd form, inside the short
    # one) sends that slice's waves to the short form
    from tests.conftest import say
    shape = POINTWISE_RQ[name]
    x, w, b = lab.make_case_data(shape, seed=17)
    rng = np.random.default_rng(18)
    t = rng.integers(0, 9, size=shape.k)
    mult = ((rng.integers(2 ** 22, 2 ** 23, size=shape.k) * 2 + 1)
            * rng.choice([-1, 1], size=shape.k) << t).astype(np.int32)
    shift = (rng.integers(35, 38, size=shape.k) + t).astype(np.int32)
    if mixed:
        mult[shape.k - 3] = 3 << 4
        shift[shape.k - 3] = 36
    say(f"[gpu] pointwise requant odd form {name} mixed={mixed}")
    got = lab.conv2d_requant(x, w, b, mult, shift, 7, shape)
    exp = oracle.requantize(oracle.conv(shape, x, w, b), mult, shift, 7)
    assert len(np.unique(exp)) > 200
    np.testing.assert_array_equal(got, exp)


@pytest.mark.gpu
def test_pointwise_requant_unaligned_output_takes_the_unfused_path():
    # output at +4 bytes: the convolution into the int32 workspace and the
    # requantizing pass, bit-exact, nothing written outside the output
    from tests.conftest import say
    shape = POINTWISE_RQ["c64_k128"]
    x, w, b = lab.make_case_data(shape, seed=13)
    mult, shift = _qparams(shape.k, seed=14)
    count = shape.output_elements
    g = shape.geometry()
    ws_n = (count * 4 + 255) // 256 * 256 + lab.workspace_bytes(lab.dispatch(shape), shape)
    bufs = [lab.DeviceBuffer.from_array(a) for a in (x, w, b, mult, shift)]
    out = lab.DeviceBuffer(count + 32)
    ws = lab.DeviceBuffer(ws_n)
    try:
        out.fill(0x5A)
        say(f"[gpu] pointwise requant, output at +4 bytes, workspace {ws_n}")
        lab.launch_requant(shape, *bufs[:3], bufs[3], bufs[4], 5, out.ptr + 4, ws, ws_n)
        lab.synchronize()
        raw = out.download(np.int8, count + 32)
    finally:
        for buf in bufs + [out, ws]:
            buf.close()
    assert g.gemm_m * g.gemm_n == count
    assert np.all(raw[:4] == 0x5A) and np.all(raw[count + 4:] == 0x5A)
    exp = oracle.requantize(oracle.conv(shape, x, w, b), mult, shift, 5)
    np.testing.assert_array_equal(raw[4:count + 4].reshape(exp.shape), exp)


FUSED_FORMS = {
    # the row kernel's epilogue takes the odd-multiplier form per wave when
    # all of its channels are in that form's domain (requant_odd_params):
    # here every wave but the one holding channel 9 (mult -2^31: 31
    # trailing zeros leave s' below 33), which takes the general form;
    # multipliers of both signs, quotients spread over the int8 range
    "odd": (-3, (), False),
    # two more waves' channels leave the domain (shift 32 and 20)
    "mixed": (-3, ((77, 32), (5, 20)), False),
    # multipliers with 0..8 trailing zeros and shifts raised to match, so the
    # form's normalization (mult = mo 2^t, s' = s - t) decides every value
    "trailing_zeros": (-3, (), True),
    # zero points that put k = 2^(sh-1) + zp 2^sh outside +-2^30: every wave
    # takes the general form
    "zp_limit": (-(2 ** 30), (), False),
    "zp_outside": (2 ** 30 + 1, (), False),
}


@pytest.mark.gpu
@pytest.mark.parametrize("variant", sorted(FUSED_FORMS))
def test_fused_requant_forms_bit_exact(variant):
    from tests.conftest import say
    shape = _baseline("cfg2_resnet_3x3_s1")
    assert lab.requant_fused(shape)
    x, w, b = lab.make_case_data(shape, seed=7)
    rng = np.random.default_rng(8)
    mult = (rng.integers(2 ** 30, 2 ** 31, size=shape.k)
            * rng.choice([-1, 1], size=shape.k)).astype(np.int32)
    mult[9] = -(2 ** 31)
    shift = rng.integers(44, 47, size=shape.k).astype(np.int32)
    zp, general, trailing = FUSED_FORMS[variant]
    if trailing:
        t = rng.integers(0, 9, size=shape.k)
        mult = ((mult.astype(np.int64) >> 8) << t).astype(np.int32)   # |mult| < 2^31
        shift = (shift - 8 + t).astype(np.int32)
    for ch, sh in general:
        shift[ch] = sh
    say(f"[gpu] fused requant form {variant}")
    got = lab.conv2d_requant(x, w, b, mult, shift, zp, shape)
    exp = oracle.requantize(oracle.conv(shape, x, w, b), mult, shift, zp)
    if variant in ("odd", "mixed", "trailing_zeros"):
        assert len(np.unique(exp)) > 200       # the quotients reach most int8 values
    np.testing.assert_array_equal(got, exp)


def test_kernel_requant_function_matches_oracle_on_host(tmp_path):
    # the device function itself, built for the host with g++
    import os
    import subprocess
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    exe = tmp_path / "requant_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-I", os.path.join(root, "include"), "-I",
                    os.path.join(root, "int8_kernel_lab_amd", "csrc"),
                    os.path.join(root, "tests", "requant_check.cpp"), "-o", str(exe)], check=True)
    rng = np.random.default_rng(21)
    n = 4000
    acc = rng.integers(-(2 ** 31), 2 ** 31, size=n, dtype=np.int64)
    mult = rng.integers(-(2 ** 31), 2 ** 31, size=n, dtype=np.int64)
    shift = rng.integers(-3, 66, size=n, dtype=np.int64)
    zp = rng.integers(-200, 200, size=n, dtype=np.int64)
    # edges: extremes, exact ties of both signs, shift 0 and 62
    acc[:8] = [-(2 ** 31), 2 ** 31 - 1, 3, -3, 5, -5, 1, -1]
    mult[:8] = [-(2 ** 31), -(2 ** 31), 1, 1, 1, 1, 2 ** 31 - 1, 2 ** 31 - 1]
    shift[:8] = [62, 0, 1, 1, 1, 1, 62, 62]
    zp[:8] = 0
    # a block of typical Q31 scales
    acc[8:400] = rng.integers(-(2 ** 26), 2 ** 26, size=392)
    mult[8:400] = rng.integers(2 ** 30, 2 ** 31, size=392)
    shift[8:400] = rng.integers(48, 58, size=392)
    # the short form's domain (shift >= 33, |zp| <= 2^30): its edges, exact
    # ties of both signs, the largest quotients, zero points at the limit
    acc[400:416] = [-(2 ** 31), -(2 ** 31), 2 ** 31 - 1, 2 ** 31 - 1, 0, 0, 3, -3,
                    2 ** 20, -(2 ** 20), 1, -1, 2 ** 31 - 1, -(2 ** 31), 12345, -12345]
    mult[400:416] = [-(2 ** 31), 2 ** 31 - 1, -(2 ** 31), 2 ** 31 - 1, -(2 ** 31), 7,
                     2 ** 31 - 1, 2 ** 31 - 1, 2 ** 13, 2 ** 13, 2 ** 31 - 1, -(2 ** 31), 5, 5,
                     -1, -1]
    shift[400:416] = [33, 62, 33, 34, 40, 33, 33, 33, 34, 34, 62, 62, 66, 33, 33, 33]
    zp[400:416] = [2 ** 30, -(2 ** 30), 0, 5, -7, 0, 0, 0, 0, 0, 2 ** 30, -(2 ** 30), 1, 1, -1, 1]
    # exact ties at shift 33 of both signs: acc * mult = -+(2q + 1) * 2^32
    for i, q in zip(range(416, 424), [0, 1, 5, 100, 0, 1, 5, 100]):
        sign = 1 if i < 420 else -1
        acc[i], mult[i], shift[i], zp[i] = sign * 2 * (2 * q + 1), -(2 ** 31), 33, 0
    acc[424:1400] = rng.integers(-(2 ** 31), 2 ** 31, size=976)
    mult[424:1400] = rng.integers(-(2 ** 31), 2 ** 31, size=976)
    shift[424:1400] = rng.integers(33, 70, size=976)
    zp[424:1400] = rng.integers(-(2 ** 30), 2 ** 30 + 1, size=976)
    # the odd-multiplier form's edges: multipliers with trailing zeros, the
    # shift at both ends of 1 <= sh <= 30, k at +-2^30, negative products
    # just past a multiple of 2^32, the extreme accumulators, mult 0 and
    # -2^31 (outside the form: t = 31)
    e = 1400
    rows = [(-1, 2 ** 31 - 1, 33, 0), (1, 2 ** 31 - 1, 33, 0), (-(2 ** 31), 2 ** 31 - 1, 33, 0),
            (-(2 ** 31), 2 ** 31 - 1, 62, 0), (2 ** 31 - 1, -(2 ** 31 - 1), 33, 5),
            (-(2 ** 31), -(2 ** 31 - 1), 34, -7), (12345, 3 << 20, 53, 1), (-12345, 3 << 20, 53, 1),
            (-(2 ** 31), 3 << 20, 53, 0), (2 ** 31 - 1, 5 << 28, 62, 0), (-77, 5 << 28, 62, 0),
            (-3, 1, 33, 2 ** 29 - 1), (3, -1, 33, -(2 ** 29)), (3, 1, 33, 2 ** 29),
            (-(2 ** 31), 1, 62, 0), (2 ** 31 - 1, 1, 62, 0), (-5, 7, 62, 0), (5, -7, 62, 0),
            (99, 0, 40, -3), (-99, 0, 40, 127), (100, -(2 ** 31), 62, 0), (-100, 2 ** 30, 62, 0),
            (-100, 2 ** 30, 63, 0), (2 ** 20, 2 ** 31 - 1, 51, 0), (-(2 ** 20), 2 ** 31 - 1, 51, 0),
            (-(2 ** 20) - 1, 2 ** 31 - 3, 51, 0), (2 ** 26, 2 ** 30 + 1, 48, 3),
            (-(2 ** 26), 2 ** 30 + 1, 48, 3), (-(2 ** 26), 2 ** 30 + 1, 48, -128),
            (2 ** 30, 2 ** 31 - 1, 34, 127)]
    for i, (a, m, sv, z) in enumerate(rows):
        acc[e + i], mult[e + i], shift[e + i], zp[e + i] = a, m, sv, z
    text = "\n".join(f"{a} {m} {s} {z}" for a, m, s, z in zip(acc, mult, shift, zp))
    out = subprocess.run([str(exe)], input=text, text=True, capture_output=True, check=True)
    got = np.array([int(v) for v in out.stdout.split()], dtype=np.int64).reshape(-1, 4)
    assert got.shape[0] == n
    short = (shift >= 33) & (np.abs(zp) <= 2 ** 30)
    assert short.sum() > 1000
    # the odd-multiplier form's domain: 1 <= min(shift, 62) - t - 32 <= 30
    # (t = trailing zeros of mult) and |2^(sh-1) + zp 2^sh| <= 2^30
    sc = np.clip(shift, 0, 62)
    tz = np.array([(int(m) & -int(m)).bit_length() - 1 if m else 0 for m in mult])
    sh = np.where(mult == 0, 1, sc - tz - 32)
    kk = [(1 << (int(h) - 1)) + int(z) * (1 << int(h)) if 1 <= h <= 30 else None
          for h, z in zip(sh, zp)]
    odd = np.array([k is not None and abs(k) <= 2 ** 30 for k in kk])
    np.testing.assert_array_equal(got[:, 3], odd.astype(np.int64))
    assert odd.sum() > 1000
    for i in range(n):
        want = exact_requant(int(acc[i]), int(mult[i]), int(shift[i]), int(zp[i]))
        assert got[i, 0] == want, (i, acc[i], mult[i], shift[i], zp[i], got[i], want)
        assert got[i, 1] == want, ("short", i, acc[i], mult[i], shift[i], zp[i], got[i], want)
        assert got[i, 2] == want, ("odd", i, acc[i], mult[i], shift[i], zp[i], got[i], want)
