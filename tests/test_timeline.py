"""The per-wave timeline tool (int8_kernel_lab_amd/timeline): its stamped
copies of the two kernel sources still match the sources they are made from,
the link list is the library's own, and the stamp analysis reads a synthetic
stamp buffer back as written.  No GPU."""
import numpy as np
import pytest

from int8_kernel_lab_amd.timeline import instrument
from int8_kernel_lab_amd.timeline.__main__ import _analyse


def test_every_edit_applies_once():
    src = instrument.instrumented_sources()
    assert set(src) == {"kernel_rowpass.hip", "kernel_deepk.hip"}
    assert 'extern "C" void i8conv_timeline_set(void *buffer, int workgroups)' in \
        src["kernel_rowpass.hip"]
    for text in src.values():
        # launches beyond the buffer stamp nothing
        assert "<= int64_t(g_i8_timeline_wgs) ? g_i8_timeline : nullptr" in text or \
            "<= size_t(g_i8_timeline_wgs)\n             ? g_i8_timeline : nullptr" in text
        assert "tl_put(p.tl, 0, t_start);" in text


def test_an_edit_that_no_longer_matches_fails_loudly():
    with pytest.raises(RuntimeError, match="matches 0 times"):
        instrument._apply("int x;", [("int y;", "int z;")], "probe.hip")


def test_link_list_is_the_library_source_list():
    objs = instrument.library_objects()
    assert "kernel_rowpass.o" in objs and "kernel_deepk.o" in objs and "capi.o" in objs
    assert len(objs) == len(set(objs))


def test_analysis_reads_synthetic_stamps():
    a = np.zeros((4, instrument.WAVES, instrument.SLOTS), np.uint64)
    base = 10_000
    for wg in range(2):
        for wave in range(8):
            a[wg, wave, 0] = base + wave          # start: 0.00 .. 0.07 us
            a[wg, wave, 1] = base + 30
            a[wg, wave, 31] = base + 40
        for wave in range(4):                     # copy waves
            a[wg, wave, 2] = base + 100
            a[wg, wave, 3] = base + 150
        for wave in range(4, 8):                  # MFMA waves
            a[wg, wave, 27] = base + 120
            for r in range(10):
                a[wg, wave, 4 + r] = base + 120 + 30 * r
            a[wg, wave, 26] = 1_000_000
            a[wg, wave, 28] = 1_000_000 + 6_000        # 6000 cycles in 3 us: 2 GHz
            a[wg, wave, 29] = base + 420
            a[wg, wave, 30] = base + 450
    out = _analyse(a, "kernel_rowpass.hip")
    assert out["workgroups"] == 2
    assert out["copy_waves"] == [0, 1, 2, 3] and out["mfma_waves"] == [4, 5, 6, 7]
    assert out["stamps_us"][" 0 wave start"] == [0.0, 0.035, 0.07]
    assert out["stamps_us"][" 3 copy wave: copies landed"] == [1.5, 1.5, 1.5]
    assert out["walk_us_median"] == 3.0
    assert out["walk_clock_ghz_median"] == 2.0
    assert out["row_step_us_median"] == 0.3
