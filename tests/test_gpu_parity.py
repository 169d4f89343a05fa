"""GPU parity: every candidate kernel, bit-exact against the CPU oracle.

Each check poisons the output buffer first (so a kernel that skips stores
cannot pass on stale data), launches through the C ABI, and compares EVERY
output element with oracle.conv (the restatement of conv_lab.cu:39-66).
The reference checked 2048 sampled outputs (conv_lab.cu:72-77).
"""
import hashlib
import json
import os

import numpy as np
import pytest

import int8_kernel_lab_amd as lab
from oracle import oracle
from tests.conftest import say

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                      "baseline_outputs.json")
with open(GOLDEN) as _f:
    GOLDEN_CONFIGS = json.load(_f)["configs"]

BASELINE_NAMES = ["cfg1_smoke", "cfg2_resnet_3x3_s1", "cfg3_down_3x3_s2",
                  "cfg4a_pointwise_1x1", "cfg4b_k36_tail", "cfg5a_deep_k", "cfg5b_dilated"]

# Edge shapes the reference's tests never reached (its sampled check and
# compile-time predicate hid them): odd and non-multiple-of-4 K, C = 16/48,
# asymmetric filters, stride 2/4, 5x5, dilation with taps outside the image,
# a 1x1 image, the truncating out_h formula, rows wider than one tile,
# multi-tile K with a tail, M tails.
EDGE = {
    "k63": lab.ConvShape(1, 18, 18, 64, 63, 3, 3, 1, 1, 1, 1, 1, 1),
    "k69_s2": lab.ConvShape(2, 17, 19, 64, 69, 3, 3, 1, 1, 2, 2, 1, 1),
    "c16_1x1_k5": lab.ConvShape(3, 9, 7, 16, 5, 1, 1, 0, 0, 1, 1, 1, 1),
    "c48_3x3": lab.ConvShape(2, 10, 12, 48, 24, 3, 3, 1, 1, 1, 1, 1, 1),
    "asym_1x3": lab.ConvShape(2, 16, 16, 64, 32, 1, 3, 0, 1, 1, 1, 1, 1),
    "asym_3x1": lab.ConvShape(2, 16, 16, 64, 32, 3, 1, 1, 0, 1, 1, 1, 1),
    "k5x5_s2": lab.ConvShape(2, 23, 23, 64, 40, 5, 5, 2, 2, 2, 2, 1, 1),
    "patch4x4_s4": lab.ConvShape(2, 32, 32, 32, 96, 4, 4, 0, 0, 4, 4, 1, 1),
    "dil3_pad1": lab.ConvShape(1, 20, 20, 64, 64, 3, 3, 1, 1, 1, 1, 3, 3),
    "one_pixel": lab.ConvShape(2, 1, 1, 64, 64, 3, 3, 1, 1, 1, 1, 1, 1),
    "trunc_out": lab.ConvShape(1, 2, 2, 16, 8, 3, 3, 0, 0, 2, 2, 1, 1),
    "wide_row": lab.ConvShape(1, 3, 200, 64, 64, 3, 3, 1, 1, 1, 1, 1, 1),
    "deep_c": lab.ConvShape(1, 5, 5, 1024, 80, 3, 3, 1, 1, 1, 1, 1, 1),
    "k300": lab.ConvShape(1, 8, 8, 64, 300, 3, 3, 1, 1, 1, 1, 1, 1),
    "m_tail": lab.ConvShape(3, 7, 9, 128, 128, 3, 3, 1, 1, 1, 1, 1, 1),
    "s2_dil2": lab.ConvShape(2, 30, 30, 64, 64, 3, 3, 2, 2, 2, 2, 2, 2),
    # c % 128 == 0: the LDS-DMA pipelined generic / split-K kernel.  Channel
    # tails with N % 4 != 0 (scalar stores and the scalar reduce), pixel
    # tails, stride + dilation + asymmetric padding, a grid of tiles that is
    # not a multiple of the 8 XCDs, one k-stage per tap and several.
    "dma_k38_tails": lab.ConvShape(3, 11, 13, 128, 38, 3, 3, 1, 1, 1, 1, 1, 1),
    "dma_k198_s2_dil2": lab.ConvShape(2, 23, 21, 256, 198, 3, 3, 2, 1, 2, 2, 2, 1),
    "dma_1x1_m_tail": lab.ConvShape(5, 17, 19, 384, 96, 1, 1, 0, 0, 1, 1, 1, 1),
    "dma_5x3_asym": lab.ConvShape(1, 40, 36, 128, 136, 5, 3, 2, 0, 1, 2, 1, 3),
    "dma_grid_9x2": lab.ConvShape(1, 48, 48, 128, 200, 3, 3, 1, 1, 1, 1, 1, 1),
    "dma_256x128_tails": lab.ConvShape(4, 63, 99, 128, 134, 3, 3, 1, 1, 1, 1, 1, 1),
    "dma_1x1_k62_short": lab.ConvShape(16, 56, 55, 256, 62, 1, 1, 0, 0, 1, 1, 1, 1),
    "dma_256x64_tails": lab.ConvShape(16, 57, 55, 128, 62, 3, 3, 1, 1, 1, 1, 1, 1),
    # tiles that store fewer pixel rows than they hold (the tile step, 80 of
    # 128 on grids just over 256 tiles): a partial last tile, with vector
    # stores and with element stores (K % 4)
    "dma_step_k100_tail": lab.ConvShape(17, 45, 45, 128, 100, 3, 3, 1, 1, 1, 1, 1, 1),
    "dma_step_1x1_k70": lab.ConvShape(17, 45, 45, 256, 70, 1, 1, 0, 0, 1, 1, 1, 1),
    # c == 128 3x3 stride 1: the row-streaming kernel with copy waves.
    # Blocks of unequal height (8/7 and 2/1 output rows), a channel tail with
    # scalar stores, four fragments per row (the two-walk form, 5 plane
    # copies per row: copy waves with 1 and 2 per row), one fragment per row
    # (2 plane copies: copy waves with none), no padding.
    "stream_r8_uneven_k126": lab.ConvShape(32, 30, 30, 128, 126, 3, 3, 1, 1, 1, 1, 1, 1),
    "stream_r2_uneven": lab.ConvShape(8, 28, 28, 128, 128, 3, 3, 1, 1, 1, 1, 1, 1),
    "stream_nfr4": lab.ConvShape(16, 20, 60, 128, 64, 3, 3, 1, 1, 1, 1, 1, 1),
    "stream_nfr1": lab.ConvShape(8, 14, 14, 128, 128, 3, 3, 1, 1, 1, 1, 1, 1),
    "stream_pad0": lab.ConvShape(4, 30, 30, 128, 64, 3, 3, 0, 0, 1, 1, 1, 1),
    # Blocks of 4-6 rows: 4 rows with one fragment, 5/4 rows of 29
    # columns, 6/5 rows with a 96-channel tail (half a channel tile).
    "stream_split_r4_nfr1": lab.ConvShape(32, 16, 16, 128, 128, 3, 3, 1, 1, 1, 1, 1, 1),
    "stream_split_r5_w29": lab.ConvShape(32, 19, 29, 128, 128, 3, 3, 1, 1, 1, 1, 1, 1),
    "stream_split_r6_k96": lab.ConvShape(32, 22, 13, 128, 96, 3, 3, 1, 1, 1, 1, 1, 1),
    # n % 8 == 0 launches the row kernels on the grid that keeps each image
    # on one XCD (blockIdx.x = image % 8 + 8 x channel tile): four channel
    # tiles with a partial last one (copy-wave kernel and the c = 64 one),
    # and three groups of eight images with a 36-channel tile.
    "stream_xcd_k200": lab.ConvShape(8, 14, 14, 128, 200, 3, 3, 1, 1, 1, 1, 1, 1),
    "row_xcd_k200": lab.ConvShape(8, 28, 28, 64, 200, 3, 3, 1, 1, 1, 1, 1, 1),
    "row_xcd_n24_k36": lab.ConvShape(24, 14, 14, 64, 36, 3, 3, 1, 1, 1, 1, 1, 1),
    # c == 128 3x3 stride 2 (config 3's family): a 4-channel tail in the
    # second 128-channel tile; no padding with odd input sizes and 64
    # channels; 20-column output rows with a 72-channel tail.
    "s2_k132": lab.ConvShape(64, 28, 28, 128, 132, 3, 3, 1, 1, 2, 2, 1, 1),
    "s2_pad0_odd_k64": lab.ConvShape(32, 27, 27, 128, 64, 3, 3, 0, 0, 2, 2, 1, 1),
    "s2_w40_k200": lab.ConvShape(16, 40, 40, 128, 200, 3, 3, 1, 1, 2, 2, 1, 1),
    # deep channels, few pixels (the split-K regime): 32 slices of 128
    # channels with an output-channel tail of 4 and no padding; padding 2;
    # 14x14 images.
    "deepc_k260_pad0": lab.ConvShape(4, 5, 9, 4096, 260, 3, 3, 0, 0, 1, 1, 1, 1),
    "deepc_pad2": lab.ConvShape(2, 6, 6, 2048, 512, 3, 3, 2, 2, 1, 1, 1, 1),
    "deepc_14x14": lab.ConvShape(2, 14, 14, 1024, 512, 3, 3, 1, 1, 1, 1, 1, 1),
    # split-K's deep-channel form (every output pixel in one workgroup): 40
    # one-pixel images (halo only, 41 chunk flags); 3 slices with a 36-channel
    # tail; no padding with a 13-pixel last fragment; one-column images; 512
    # pixels (eight fragments per MFMA wave, the largest plan)
    "deepk_many_images_1x1": lab.ConvShape(40, 1, 1, 256, 32, 3, 3, 1, 1, 1, 1, 1, 1),
    "deepk_k36_c384": lab.ConvShape(2, 7, 7, 384, 36, 3, 3, 1, 1, 1, 1, 1, 1),
    "deepk_pad0_m_tail": lab.ConvShape(3, 9, 11, 256, 64, 3, 3, 0, 0, 1, 1, 1, 1),
    "deepk_w1_rows": lab.ConvShape(4, 12, 1, 256, 64, 3, 3, 1, 1, 1, 1, 1, 1),
    "deepk_m512": lab.ConvShape(2, 16, 16, 256, 64, 3, 3, 1, 1, 1, 1, 1, 1),
    # the generic kernel's pointwise streaming form (1x1, stride 1, no pad):
    # C = 64 -> 256 channels with a 13-pixel last fragment; C = 512 -> 32
    # (eight k-steps); 128 -> 128 with a pixel tail; one pixel (one wave of
    # the grid idle); 2110 fragments, more than one per wave over 1024 waves;
    # an output above 128 MiB (evict-first stores)
    "pw_c64_k256_m_tail": lab.ConvShape(3, 7, 9, 64, 256, 1, 1, 0, 0, 1, 1, 1, 1),
    "pw_c512_k32": lab.ConvShape(2, 10, 11, 512, 32, 1, 1, 0, 0, 1, 1, 1, 1),
    "pw_c128_k128_tail": lab.ConvShape(5, 13, 17, 128, 128, 1, 1, 0, 0, 1, 1, 1, 1),
    "pw_one_pixel": lab.ConvShape(1, 1, 1, 128, 64, 1, 1, 0, 0, 1, 1, 1, 1),
    "pw_2110_frags": lab.ConvShape(33, 31, 33, 256, 64, 1, 1, 0, 0, 1, 1, 1, 1),
    "pw_out_above_128mib": lab.ConvShape(9, 120, 128, 64, 256, 1, 1, 0, 0, 1, 1, 1, 1),
    # output channels in slices (one wave each, one fragment stream per
    # workgroup): 2 slices of 64 with a pixel tail; 8 slices of 32 channels;
    # 2 slices of 128; 2 slices of 32 over two fragments
    "pw_slices2_c256_k128": lab.ConvShape(1, 52, 51, 256, 128, 1, 1, 0, 0, 1, 1, 1, 1),
    "pw_slices8_c512_k256": lab.ConvShape(3, 10, 10, 512, 256, 1, 1, 0, 0, 1, 1, 1, 1),
    "pw_slices2_c128_k256": lab.ConvShape(5, 13, 17, 128, 256, 1, 1, 0, 0, 1, 1, 1, 1),
    "pw_slices2_c512_k64": lab.ConvShape(1, 3, 7, 512, 64, 1, 1, 0, 0, 1, 1, 1, 1),
}

_expected_cache = {}


def _case(name, shape, seed=lab.BASELINE_SEED):
    key = (name, shape, seed)
    if key not in _expected_cache:
        x, w, b = lab.make_case_data(shape, seed)
        _expected_cache.clear()  # keep one case resident (config 5b is 34 MB)
        _expected_cache[key] = (x, w, b, oracle.conv(shape, x, w, b))
    return _expected_cache[key]


def run_kernel(kernel, shape, x, w, b, poison=0xA5):
    """Poisoned output -> launch -> synchronize -> host copy."""
    g = shape.geometry()
    xb = lab.DeviceBuffer.from_array(x)
    wb = lab.DeviceBuffer.from_array(w)
    bb = lab.DeviceBuffer.from_array(b)
    yb = lab.DeviceBuffer(4 * g.output_elements)
    ws_n = lab.workspace_bytes(kernel, shape)
    ws = lab.DeviceBuffer(ws_n) if ws_n else None
    try:
        yb.fill(poison)
        if ws is not None:
            ws.fill(0x5A)
        lab.launch(kernel, shape, xb, wb, bb, yb, ws, ws_n)
        lab.synchronize()
        return yb.download(np.int32, g.output_elements).reshape(shape.output_shape)
    finally:
        for buf in (xb, wb, bb, yb, ws):
            if buf is not None:
                buf.close()


def assert_bit_exact(got, expected, label):
    if not np.array_equal(got, expected):
        bad = np.argwhere(got != expected)
        first = tuple(int(v) for v in bad[0])
        raise AssertionError(f"{label}: {len(bad)} mismatches; first at NHWK {first}: "
                             f"expected {int(expected[first])}, got {int(got[first])}")


@pytest.mark.gpu
@pytest.mark.parametrize("kernel", lab.KERNELS)
@pytest.mark.parametrize("case", BASELINE_NAMES)
def test_baseline_config_bit_exact(case, kernel, baseline_cases):
    shape = baseline_cases[case]
    if not lab.eligible(kernel, shape):
        pytest.skip(f"{kernel} ineligible for {case}")
    x, w, b, expected = _case(case, shape)
    say(f"[gpu] {kernel} on {case} {shape}")
    got = run_kernel(kernel, shape, x, w, b)
    assert_bit_exact(got, expected, f"{kernel}/{case}")
    # and the torch-float64 golden hash of the full output (tests/golden)
    assert hashlib.sha256(got.tobytes()).hexdigest() == GOLDEN_CONFIGS[case]["output_sha256"]


@pytest.mark.gpu
@pytest.mark.parametrize("kernel", lab.KERNELS)
@pytest.mark.parametrize("case", sorted(EDGE))
def test_edge_shape_bit_exact(case, kernel):
    shape = EDGE[case]
    if not lab.eligible(kernel, shape):
        pytest.skip(f"{kernel} ineligible for {case}")
    x, w, b, expected = _case(case, shape, seed=7)
    say(f"[gpu] {kernel} on edge {case} {shape}")
    got = run_kernel(kernel, shape, x, w, b)
    assert_bit_exact(got, expected, f"{kernel}/{case}")


@pytest.mark.gpu
def test_dispatched_kernel_matches_on_every_baseline_config(baseline_cases):
    for case in BASELINE_NAMES:
        shape = baseline_cases[case]
        kernel = lab.dispatch(shape)
        x, w, b, expected = _case(case, shape)
        say(f"[gpu] dispatch -> {kernel} on {case}")
        got = lab.conv2d(x, w, b, shape)
        assert_bit_exact(got, expected, f"dispatch({kernel})/{case}")


@pytest.mark.gpu
def test_extreme_values_do_not_lose_bits():
    # all -128 input and filter: every product is +16384, the largest
    # magnitude an int8 x int8 product reaches; C = 2048, 3x3 -> |acc| near
    # 3.0e8 plus bias 2^20 (configuration 5a's worst case).
    shape = lab.ConvShape(1, 7, 7, 2048, 64, 3, 3, 1, 1, 1, 1, 1, 1)
    x = np.full((1, 7, 7, 2048), -128, np.int8)
    w = np.full((64, 3, 3, 2048), -128, np.int8)
    b = np.full(64, (1 << 20), np.int32)
    expected = oracle.conv(shape, x, w, b)
    assert int(expected.max()) == 9 * 2048 * 16384 + (1 << 20)
    for kernel in lab.KERNELS:
        if not lab.eligible(kernel, shape):
            continue
        say(f"[gpu] {kernel} on extreme values")
        assert_bit_exact(run_kernel(kernel, shape, x, w, b), expected, f"{kernel}/extreme")


@pytest.mark.gpu
def test_int32_accumulator_wraps_like_the_oracle():
    # 9 taps x 16384 channels x (-128 * -128) = 9 * 2^28 > 2^31 at the
    # centre output: the int32 sum wraps in the oracle and on the MFMA alike
    shape = lab.ConvShape(1, 3, 3, 16384, 8, 3, 3, 1, 1, 1, 1, 1, 1)
    x = np.full((1, 3, 3, 16384), -128, np.int8)
    w = np.full((8, 3, 3, 16384), -128, np.int8)
    w[1] = 127  # products of -16256: a negative sum that does not wrap
    b = np.arange(8, dtype=np.int32) * 1000 - 3000
    expected = oracle.conv(shape, x, w, b)
    exact = 9 * 16384 * 16384 - 3000
    assert int(expected[0, 1, 1, 0]) == (exact + 2 ** 31) % 2 ** 32 - 2 ** 31
    for kernel in lab.KERNELS:
        if not lab.eligible(kernel, shape):
            continue
        say(f"[gpu] {kernel} on int32 wrap case")
        assert_bit_exact(run_kernel(kernel, shape, x, w, b), expected, f"{kernel}/wrap")


@pytest.mark.gpu
def test_pointwise_form_falls_back_for_an_unaligned_output():
    # The pointwise streaming form needs 16-byte aligned pointers: an output
    # 4 bytes past an allocation's start runs the tile GEMM instead, bit-exact,
    # and nothing outside the output is written.
    name = "pw_c128_k128_tail"
    shape = EDGE[name]
    assert "pointwise streaming" in lab.describe("generic", shape)
    x, w, b, expected = _case(name, shape, seed=7)
    count = shape.geometry().output_elements
    bufs = [lab.DeviceBuffer.from_array(a) for a in (x, w, b)]
    yb = lab.DeviceBuffer(4 * count + 16)
    try:
        yb.fill(0xA5)
        say(f"[gpu] generic on {name} with the output at +4 bytes")
        lab.launch("generic", shape, *bufs, yb.ptr + 4)
        lab.synchronize()
        raw = yb.download(np.int32, count + 4)
    finally:
        for buf in bufs + [yb]:
            buf.close()
    poison = np.uint32(0xA5A5A5A5).view(np.int32)
    assert raw[0] == poison and np.all(raw[count + 1:] == poison)
    assert_bit_exact(raw[1:count + 1].reshape(shape.output_shape), expected,
                     "generic/unaligned output")


@pytest.mark.gpu
def test_split_k_is_deterministic(baseline_cases):
    shape = baseline_cases["cfg5a_deep_k"]
    x, w, b, expected = _case("cfg5a_deep_k", shape)
    say("[gpu] splitk twice on cfg5a_deep_k (different poison)")
    first = run_kernel("splitk", shape, x, w, b, poison=0x00)
    second = run_kernel("splitk", shape, x, w, b, poison=0xFF)
    assert first.tobytes() == second.tobytes()
    assert_bit_exact(first, expected, "splitk/cfg5a")


@pytest.mark.gpu
def test_launch_errors_are_statuses_not_faults(baseline_cases):
    shape = baseline_cases["cfg3_down_3x3_s2"]  # stride 2: strip ineligible
    g = shape.geometry()
    xb = lab.DeviceBuffer(g.input_elements)
    wb = lab.DeviceBuffer(g.filter_elements)
    bb = lab.DeviceBuffer(4 * shape.k)
    yb = lab.DeviceBuffer(4 * g.output_elements)
    try:
        with pytest.raises(lab.I8ConvError, match="ineligible"):
            lab.launch("strip", shape, xb, wb, bb, yb)
        with pytest.raises(lab.I8ConvError, match="workspace too small"):
            lab.launch("splitk", shape, xb, wb, bb, yb, None, 0)
        with pytest.raises(lab.I8ConvError, match="bad argument"):
            lab.launch("generic", shape, xb.ptr + 1, wb, bb, yb)  # misaligned input
        lab.synchronize()
    finally:
        for buf in (xb, wb, bb, yb):
            buf.close()


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["cfg2_resnet_3x3_s1", "cfg5a_deep_k"])
def test_graph_replays_bit_exact(case, baseline_cases):
    # the bench's timing path: launches captured in HIP graphs (split-K: two
    # kernels per launch, the workspace rewritten every launch); the output
    # is poisoned outside the graphs right before the timed replays, so the
    # check sees only what the replays wrote.  Three calls: a main graph that
    # divides the launches, one with a remainder graph (7 = 2 x 3 + 1), and
    # one graph holding every timed launch (the bench's form).
    shape = baseline_cases[case]
    kernel = lab.dispatch(shape)
    x, w, b, expected = _case(case, shape)
    g = shape.geometry()
    bufs = [lab.DeviceBuffer.from_array(a) for a in (x, w, b)]
    yb = lab.DeviceBuffer(4 * g.output_elements)
    ws_n = lab.workspace_bytes(kernel, shape)
    ws = lab.DeviceBuffer(ws_n) if ws_n else None
    try:
        for call, (iterations, per_graph) in enumerate([(6, 3), (7, 3), (5, 5)]):
            say(f"[gpu] graph replays {kernel} on {case}, call {call}")
            t = lab.measure_graph(kernel, shape, *bufs, yb, ws, ws_n, warmup=2,
                                  iterations=iterations, launches_per_graph=per_graph,
                                  min_warmup_ms=1.0, poison_byte=0x5A + call)
            assert t["mean_ms"] > 0
            # the stamped pass spans the launches and one stamp dispatch, but
            # not the gap before the first timed replay: positive and no
            # longer than the event-timed mean plus a few microseconds
            assert 0 < t["stamped_ms"] < t["mean_ms"] + 0.005
            assert t["launches_per_graph"] == per_graph
            assert t["full_replays"] * per_graph + t["remainder_launches"] == iterations
            assert t["warmup_launches"] >= 2 and t["warmup_ms"] >= 1.0
            got = yb.download(np.int32, g.output_elements).reshape(shape.output_shape)
            assert_bit_exact(got, expected, f"graph {kernel}/{case} call {call}")
    finally:
        for buf in bufs + [yb, ws]:
            if buf is not None:
                buf.close()
