"""CPU tests of the C ABI (include/i8conv.h): exports, status codes, shape
derivation, eligibility predicates, dispatch policy and launch-argument
errors.  Nothing here launches a kernel: every launch call below fails its
argument checks before the library touches HIP.
"""
import ctypes
import os
import re

import numpy as np
import pytest

import int8_kernel_lab_amd as lab
from int8_kernel_lab_amd import _lib
from oracle import oracle
from tests.golden.make_golden import out_extent

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "i8conv.h")
REFERENCE_TABLE = os.path.join(lab.WORKLOADS_DIR, "reference.csv")
BASELINE_TABLE = os.path.join(lab.WORKLOADS_DIR, "baseline.csv")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return sorted(set(re.findall(r"\b(i8conv_\w+)\s*\(", text)))


def all_shapes():
    shapes = dict(lab.load_workloads(REFERENCE_TABLE))
    shapes.update(lab.load_workloads(BASELINE_TABLE))
    return shapes


# ---- exports ---------------------------------------------------------------

def test_library_exports_every_declared_function():
    names = header_functions()
    assert len(names) >= 30
    handle = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in names if not hasattr(handle, n)]
    assert not missing, f"declared in i8conv.h but not exported: {missing}"


def test_python_binding_covers_exactly_the_header():
    assert sorted(_lib.SIGNATURES) == header_functions()


def test_status_strings():
    expected = {_lib.OK: "ok", _lib.INELIGIBLE: "ineligible", _lib.BAD_SHAPE: "bad shape",
                _lib.BAD_ARGUMENT: "bad argument",
                _lib.WORKSPACE_TOO_SMALL: "workspace too small",
                _lib.HIP_ERROR: "hip error", _lib.UNKNOWN_KERNEL: "unknown kernel"}
    for code, text in expected.items():
        assert text in _lib.lib().i8conv_status_string(code).decode()
    assert _lib.lib().i8conv_status_string(99)


def test_kernel_registry():
    assert lab.kernel_names() == lab.KERNELS
    for i, name in enumerate(lab.KERNELS):
        assert _lib.lib().i8conv_kernel_id(name.encode()) == i
    assert _lib.lib().i8conv_kernel_id(b"cudnn") == -1
    assert _lib.lib().i8conv_kernel_name(4) is None
    assert _lib.lib().i8conv_kernel_name(-1) is None


# ---- shape derivation (conv_shape.cuh:22-35) --------------------------------

def test_reference_workload_table_is_complete():
    shapes = lab.load_workloads(REFERENCE_TABLE)
    assert len(shapes) == 41
    assert "big_3x3_s1" in shapes and "smoke" in shapes


@pytest.mark.parametrize("name,shape", sorted(all_shapes().items()), ids=lambda v: str(v))
def test_derive_matches_closed_form_and_oracle(name, shape):
    g = shape.geometry()
    oh = out_extent(shape.h, shape.pad_h, shape.dilation_h, shape.r, shape.stride_h)
    ow = out_extent(shape.w, shape.pad_w, shape.dilation_w, shape.s, shape.stride_w)
    assert (g.out_h, g.out_w) == (oh, ow)
    assert g.gemm_m == shape.n * oh * ow
    assert g.gemm_n == shape.k
    assert g.gemm_k == shape.r * shape.s * shape.c
    assert g.input_elements == shape.n * shape.h * shape.w * shape.c
    assert g.filter_elements == shape.k * shape.r * shape.s * shape.c
    assert g.output_elements == g.gemm_m * shape.k
    og = oracle.derive(shape)
    assert (og.out_h, og.out_w, og.gemm_m, og.gemm_k) == (g.out_h, g.out_w, g.gemm_m, g.gemm_k)


@pytest.mark.parametrize("shape,reason", [
    (lab.ConvShape(1, 8, 8, 24, 8, 3, 3, 1, 1), "divisible by 16"),      # conv_shape.cuh:34
    (lab.ConvShape(1, 2, 2, 16, 8, 5, 5, 0, 0), "nonempty"),             # conv_shape.cuh:35
    (lab.ConvShape(1, 8, 8, 16, 8, 3, 3, 1, 1, 0, 1), "out of range"),   # stride 0
    (lab.ConvShape(0, 8, 8, 16, 8, 3, 3), "out of range"),
    (lab.ConvShape(1, 8, 8, 16, 8, 3, 3, -1, 0), "out of range"),
    (lab.ConvShape(1, 8, 8, 16, 8, 3, 3, 1, 1, 1, 1, 0, 1), "out of range"),
    (lab.ConvShape(1, 65536, 65536, 16, 8, 1, 1), "too large"),          # 2^36 input bytes
])
def test_bad_shapes_are_rejected(shape, reason):
    g = _lib.CGeometry()
    assert _lib.lib().i8conv_derive(ctypes.byref(shape.c_struct()), ctypes.byref(g)) == _lib.BAD_SHAPE
    assert reason in _lib.lib().i8conv_last_error().decode()
    with pytest.raises(ValueError):
        shape.geometry()
    for name in lab.KERNELS:
        assert not lab.eligible(name, shape)
    assert _lib.lib().i8conv_dispatch(ctypes.byref(shape.c_struct())) == -1


def test_truncating_output_formula_is_kept():
    # (2 + 0 - 2 - 1) / 2 + 1 = 1 in C (truncation toward zero), 0 with floor
    shape = lab.ConvShape(1, 2, 2, 16, 8, 3, 3, 0, 0, 2, 2, 1, 1)
    assert (shape.out_h, shape.out_w) == (1, 1)


# ---- eligibility predicates --------------------------------------------------

def test_reference_strip_predicate_selects_only_big_3x3_s1():
    # spatial_strip.cuh:11-15 over the reference's own table
    chosen = [n for n, s in lab.load_workloads(REFERENCE_TABLE).items()
              if oracle.strip_eligible_reference(s)]
    assert chosen == ["big_3x3_s1"]


@pytest.mark.parametrize("name,shape", sorted(all_shapes().items()), ids=lambda v: str(v))
def test_gfx950_strip_predicate_closed_form(name, shape):
    # the gfx950 strip tile keeps the reference's 3x3 / unit horizontal
    # stride and dilation / C % 64 conditions and drops K % 64 and
    # out_w % 128 (it tiles whole output rows and masks channel tails)
    want = (shape.r == 3 and shape.s == 3 and shape.stride_w == 1 and
            shape.dilation_w == 1 and shape.c % 64 == 0)
    assert lab.spatial_strip_eligible(shape) == want
    assert lab.eligible("strip", shape) == want
    # every shape the reference's predicate admits stays eligible
    if oracle.strip_eligible_reference(shape):
        assert want


@pytest.mark.parametrize("name,shape", sorted(all_shapes().items()), ids=lambda v: str(v))
def test_generic_and_halo_predicates(name, shape):
    assert lab.eligible("generic", shape)
    assert lab.eligible("halo", shape) == (shape.c % 64 == 0)
    assert lab.eligible("splitk", shape) == (shape.geometry().gemm_k > 128)


BASELINE_TABLE_EXPECTED = {
    # name: (strip, halo, dispatch)
    "cfg1_smoke": (True, True, "halo"),
    "cfg2_resnet_3x3_s1": (True, True, "halo"),
    "cfg3_down_3x3_s2": (False, True, "generic"),
    "cfg4a_pointwise_1x1": (False, True, "generic"),
    "cfg4b_k36_tail": (True, True, "halo"),
    "cfg5a_deep_k": (True, True, "splitk"),
    "cfg5b_dilated": (False, True, "generic"),
}


@pytest.mark.parametrize("name", sorted(BASELINE_TABLE_EXPECTED))
def test_baseline_eligibility_and_dispatch(name, baseline_cases):
    shape = baseline_cases[name]
    strip, halo, chosen = BASELINE_TABLE_EXPECTED[name]
    assert lab.eligible("strip", shape) == strip
    assert lab.eligible("halo", shape) == halo
    assert lab.dispatch(shape) == chosen


@pytest.mark.parametrize("name,shape", sorted(all_shapes().items()), ids=lambda v: str(v))
def test_dispatch_returns_an_eligible_kernel_with_its_workspace(name, shape):
    chosen = lab.dispatch(shape)
    assert lab.eligible(chosen, shape)
    s = shape.c_struct()
    assert _lib.lib().i8conv_dispatch_workspace_bytes(ctypes.byref(s)) == \
        lab.workspace_bytes(chosen, shape)
    for name_ in ("generic", "strip", "halo"):
        assert lab.workspace_bytes(name_, shape) == 0
    if lab.eligible("splitk", shape):
        g = shape.geometry()
        ws = lab.workspace_bytes("splitk", shape)
        # one int32 partial sum per output per split, at least two splits
        assert ws % (4 * g.output_elements) == 0 and ws >= 8 * g.output_elements
    assert lab.describe(chosen, shape).startswith(chosen)


def test_splitk_deep_channel_form_and_its_workspace(baseline_cases):
    # 3x3 stride-1 layers with c % 128 == 0, c >= 256 and at most 512 output
    # pixels take split-K's deep-channel form: one split per 128 input
    # channels, 32-channel tiles over all pixels
    cfg5a = baseline_cases["cfg5a_deep_k"]
    d = lab.describe("splitk", cfg5a)
    assert "deep-channel" in d and "grid 16x16 splits" in d, d
    g = cfg5a.geometry()
    assert lab.workspace_bytes("splitk", cfg5a) == (2048 // 128) * 4 * g.output_elements
    deep = lab.ConvShape(2, 16, 16, 256, 64, 3, 3, 1, 1, 1, 1, 1, 1)     # M = 512
    assert "deep-channel" in lab.describe("splitk", deep)
    assert lab.workspace_bytes("splitk", deep) == 2 * 4 * deep.geometry().output_elements
    for other in [lab.ConvShape(3, 16, 11, 256, 64, 3, 3, 1, 1, 1, 1, 1, 1),   # M = 528
                  lab.ConvShape(8, 7, 7, 128, 64, 3, 3, 1, 1, 1, 1, 1, 1),    # c = 128
                  lab.ConvShape(8, 7, 7, 320, 64, 3, 3, 1, 1, 1, 1, 1, 1),    # c % 128
                  lab.ConvShape(8, 14, 14, 256, 64, 3, 3, 1, 1, 2, 2, 1, 1),  # stride 2
                  lab.ConvShape(8, 7, 7, 256, 66, 3, 3, 1, 1, 1, 1, 1, 1)]:   # N % 4
        assert "deep-channel" not in lab.describe("splitk", other), other


def test_describe_errors_and_truncation(baseline_cases):
    shape = baseline_cases["cfg3_down_3x3_s2"]
    buf = ctypes.create_string_buffer(8)
    s = shape.c_struct()
    L = _lib.lib()
    assert L.i8conv_describe(1, ctypes.byref(s), buf, 8) == _lib.INELIGIBLE
    assert L.i8conv_describe(7, ctypes.byref(s), buf, 8) == _lib.UNKNOWN_KERNEL
    assert L.i8conv_describe(0, ctypes.byref(s), buf, 0) == _lib.BAD_ARGUMENT
    assert L.i8conv_describe(0, ctypes.byref(s), buf, 8) == _lib.OK
    assert buf.value == b"generic"  # 7 characters and the terminator


# ---- launch argument errors (returned before any HIP call) ------------------

FAKE = 0x10000  # a 64 KB-aligned address that is never dereferenced


def _launch(kid, shape, x=FAKE, w=FAKE, b=FAKE, y=FAKE, ws=None, ws_n=0):
    s = shape.c_struct() if shape is not None else None
    return _lib.lib().i8conv_launch(kid, ctypes.byref(s) if s is not None else None,
                                    x, w, b, y, ws, ws_n, None)


def test_launch_errors_without_touching_the_gpu(baseline_cases):
    cfg3 = baseline_cases["cfg3_down_3x3_s2"]
    assert _launch(9, cfg3) == _lib.UNKNOWN_KERNEL
    assert _launch(0, None) == _lib.BAD_ARGUMENT
    assert _launch(0, lab.ConvShape(1, 8, 8, 24, 8, 3, 3, 1, 1)) == _lib.BAD_SHAPE
    assert _launch(0, cfg3, x=None) == _lib.BAD_ARGUMENT
    assert _launch(0, cfg3, y=None) == _lib.BAD_ARGUMENT
    assert _launch(0, cfg3, x=FAKE + 8) == _lib.BAD_ARGUMENT   # input not 16-byte aligned
    assert _launch(0, cfg3, w=FAKE + 4) == _lib.BAD_ARGUMENT   # filter not 16-byte aligned
    assert _launch(0, cfg3, y=FAKE + 2) == _lib.BAD_ARGUMENT   # output not 4-byte aligned
    assert _launch(1, cfg3) == _lib.INELIGIBLE                 # stride_w 2: no strip
    assert "not eligible" in _lib.lib().i8conv_last_error().decode()
    assert _launch(3, cfg3) == _lib.WORKSPACE_TOO_SMALL
    need = lab.workspace_bytes("splitk", cfg3)
    assert _launch(3, cfg3, ws=FAKE, ws_n=need - 1) == _lib.WORKSPACE_TOO_SMALL
    assert _launch(3, cfg3, ws=FAKE + 4, ws_n=need) == _lib.WORKSPACE_TOO_SMALL
    assert str(need) in _lib.lib().i8conv_last_error().decode()
    shape = cfg3.c_struct()
    assert _lib.lib().i8conv_launch_spatial_strip(ctypes.byref(shape), FAKE, FAKE, FAKE,
                                                  FAKE, None) == _lib.INELIGIBLE
    bad = lab.ConvShape(1, 8, 8, 24, 8, 3, 3, 1, 1).c_struct()
    assert _lib.lib().i8conv_launch_dispatched(ctypes.byref(bad), FAKE, FAKE, FAKE, FAKE,
                                               None, 0, None) == _lib.BAD_SHAPE


def test_measure_graph_argument_errors_without_touching_the_gpu(baseline_cases):
    # i8conv_measure_graph checks its counts, poison byte, timing record and
    # shape before any HIP call
    cfg2 = baseline_cases["cfg2_resnet_3x3_s1"].c_struct()
    t = _lib.CGraphTiming()

    def call(shape=cfg2, warmup=0, min_ms=0.0, iterations=20, per_graph=20, poison=-1,
             timing=True):
        return _lib.lib().i8conv_measure_graph(
            2, ctypes.byref(shape), FAKE, FAKE, FAKE, FAKE, None, 0, warmup, min_ms,
            iterations, per_graph, poison, ctypes.byref(t) if timing else None)

    assert call(warmup=-1) == _lib.BAD_ARGUMENT
    assert call(min_ms=-1.0) == _lib.BAD_ARGUMENT
    assert call(min_ms=float("nan")) == _lib.BAD_ARGUMENT
    assert call(iterations=0) == _lib.BAD_ARGUMENT
    assert call(per_graph=0) == _lib.BAD_ARGUMENT
    assert call(poison=256) == _lib.BAD_ARGUMENT
    assert call(timing=False) == _lib.BAD_ARGUMENT
    assert "poison_byte" in _lib.lib().i8conv_last_error().decode()
    bad = lab.ConvShape(1, 8, 8, 24, 8, 3, 3, 1, 1).c_struct()
    assert call(shape=bad) == _lib.BAD_SHAPE


def test_lds_probe_argument_errors_without_touching_the_gpu():
    # i8conv_measure_lds_probe checks pattern, shape, counts and the timing
    # record before any HIP call
    t = _lib.CGraphTiming()

    def call(pattern=0, sink=FAKE, wg=256, threads=512, reads=17, iterations=5, timing=True):
        return _lib.lib().i8conv_measure_lds_probe(
            pattern, sink, wg, threads, reads, 0, 0.0, iterations, 5,
            ctypes.byref(t) if timing else None)

    assert call(pattern=6) == _lib.BAD_ARGUMENT
    assert call(pattern=-1) == _lib.BAD_ARGUMENT
    assert call(sink=None) == _lib.BAD_ARGUMENT
    assert call(threads=100) == _lib.BAD_ARGUMENT
    assert call(threads=2048) == _lib.BAD_ARGUMENT
    assert call(wg=0) == _lib.BAD_ARGUMENT
    assert call(reads=0) == _lib.BAD_ARGUMENT
    assert call(iterations=0) == _lib.BAD_ARGUMENT
    assert call(timing=False) == _lib.BAD_ARGUMENT
    assert "pattern 0..5" in _lib.lib().i8conv_last_error().decode()


def test_lds_probe_expected_values_follow_the_pattern():
    # the host restatement of the probe's per-thread XOR: with one read per
    # lane it is the fold of the one unit read, at the pattern's offset
    def unit_fold(u):
        return (u ^ (~u) ^ (3 * u) ^ (u ^ 0x55)) & 0xFFFFFFFF

    lanes = np.arange(64)
    offsets = {"linear": 16 * lanes, "stride128": 128 * lanes, "stride256": 256 * lanes,
               "pitch80": 80 * (lanes % 16) + 16 * (lanes // 16)}
    for pattern, off in offsets.items():
        got = lab.lds_probe_expected(pattern, 64, 1).view(np.uint32).astype(np.int64)
        assert (got == unit_fold(off // 16)).all(), pattern
    # (swz128's offsets are the device layout function's; the GPU run checks
    # the probe's stores against this restatement)
    # two reads per lane at shifts 0 and 1: the folds of both units XORed
    two = lab.lds_probe_expected("linear", 64, 2).view(np.uint32).astype(np.int64)
    assert (two == (unit_fold(lanes) ^ unit_fold(lanes + 1024))).all()
    # four reads per lane (each shift once), then eight (each shift twice: zero)
    eight = lab.lds_probe_expected("stride256", 64, 8)
    assert (eight == 0).all()


def test_python_layer_raises_on_bad_calls(baseline_cases):
    with pytest.raises(ValueError, match="unknown kernel"):
        lab.eligible("cudnn", baseline_cases["cfg1_smoke"])
    with pytest.raises(lab.I8ConvError, match="ineligible"):
        lab.launch("strip", baseline_cases["cfg3_down_3x3_s2"], FAKE, FAKE, FAKE, FAKE)


def test_generic_pointwise_form_eligibility(baseline_cases):
    # 1x1, stride 1, no padding, C in {64, 128, 256, 512}, N in {32, 64, 128,
    # 256}: the streaming form, at most 1024 waves; where N * C > 16384 the
    # output channels split into slices of 16384 / C, one wave each
    d = lab.describe("generic", baseline_cases["cfg4a_pointwise_1x1"])
    assert "pointwise streaming" in d and "64oc, 1024 waves" in d, d
    small = lab.ConvShape(1, 1, 1, 128, 64, 1, 1, 0, 0, 1, 1, 1, 1)
    assert "64oc, 2 waves" in lab.describe("generic", small)
    sliced = lab.ConvShape(1, 52, 52, 256, 128, 1, 1, 0, 0, 1, 1, 1, 1)  # 169 fragments
    assert "128oc in 2 slices, 338 waves" in lab.describe("generic", sliced)
    big = lab.ConvShape(16, 256, 256, 256, 256, 1, 1, 0, 0, 1, 1, 1, 1)
    assert "256oc in 4 slices, 1024 waves" in lab.describe("generic", big)
    c512 = lab.ConvShape(1, 5, 5, 512, 256, 1, 1, 0, 0, 1, 1, 1, 1)
    assert "256oc in 8 slices, 16 waves" in lab.describe("generic", c512)
    for other in (lab.ConvShape(1, 8, 8, 256, 64, 1, 1, 0, 0, 2, 2, 1, 1),   # stride 2
                  lab.ConvShape(1, 8, 8, 256, 64, 1, 1, 1, 1, 1, 1, 1, 1),   # padded
                  lab.ConvShape(1, 8, 8, 96, 64, 1, 1, 0, 0, 1, 1, 1, 1),    # C = 96
                  lab.ConvShape(1, 8, 8, 256, 48, 1, 1, 0, 0, 1, 1, 1, 1),   # N = 48
                  lab.ConvShape(1, 8, 8, 256, 512, 1, 1, 0, 0, 1, 1, 1, 1),  # N = 512
                  lab.ConvShape(1, 8, 8, 1024, 32, 1, 1, 0, 0, 1, 1, 1, 1),  # C = 1024
                  baseline_cases["cfg2_resnet_3x3_s1"]):
        assert "pointwise" not in lab.describe("generic", other), other
    # split-K never takes it
    assert "pointwise" not in lab.describe("splitk", baseline_cases["cfg4a_pointwise_1x1"])


def test_pipelined_tile_step_evens_out_the_last_round(baseline_cases):
    # 1568 tiles of 128 pixels leave 32 workgroups for a last round on 256
    # compute units; tiles storing 112 rows give 1792 = 7 * 256.  Grids of
    # one round (196 and 256 tiles) keep whole tiles.
    d = lab.describe("generic", baseline_cases["cfg4a_pointwise_1x1"])
    assert "(112px stored), grid 1792x1" in d, d
    d = lab.describe("generic", baseline_cases["cfg3_down_3x3_s2"])
    assert "stored" not in d and "grid 98x2" in d, d
    d = lab.describe("generic", baseline_cases["cfg5b_dilated"])
    assert "stored" not in d and "grid 128x2" in d, d
    # split-K keeps whole tiles
    assert "stored" not in lab.describe("splitk", baseline_cases["cfg5a_deep_k"])


def test_dispatch_cache_returns_each_shapes_own_choice():
    # the policy's results are cached per shape (64 direct-mapped slots):
    # 300 shapes, many sharing a slot, queried in two different orders give
    # the same answers as a first pass over them
    import random
    rng = random.Random(5)
    shapes = []
    for _ in range(300):
        r = rng.choice([1, 3, 5])
        shapes.append(lab.ConvShape(rng.randint(1, 8), rng.randint(4, 40), rng.randint(4, 40),
                                    rng.choice([32, 64, 128, 256, 512, 1024, 2048]),
                                    rng.choice([16, 36, 64, 128, 256, 512]), r, r,
                                    r // 2, r // 2, rng.choice([1, 2]), rng.choice([1, 2]),
                                    rng.choice([1, 2]), 1))
    first = [lab.dispatch(s) for s in shapes]
    assert set(first) > {"generic"}
    order = list(range(len(shapes)))
    rng.shuffle(order)
    for i in order:
        assert lab.dispatch(shapes[i]) == first[i], shapes[i]
    for i in reversed(range(len(shapes))):
        assert lab.dispatch(shapes[i]) == first[i], shapes[i]
