"""Layout transforms (the step before the path): NCHW <-> NHWC int8, NHWK ->
NKHW int32, and the channel-vector packing of the reference's cuDNN path
(src/cudnn_lab.cu:7-18).  The oracle is pinned by numpy reshapes and
transposes (an independent statement of the same permutations); the GPU
kernels are compared with the oracle byte for byte."""
import numpy as np
import pytest

from oracle import oracle


def test_pack_vect_c_oracle_matches_numpy():
    rng = np.random.default_rng(1)
    for (n, h, w, c, v) in [(2, 3, 5, 64, 32), (1, 7, 7, 96, 32), (3, 2, 2, 32, 32), (2, 4, 3, 48, 16)]:
        x = rng.integers(-128, 128, size=(n, h, w, c), dtype=np.int64).astype(np.int8)
        want = x.reshape(n, h, w, c // v, v).transpose(0, 3, 1, 2, 4)
        got = oracle.pack_vect_c(x, v)
        np.testing.assert_array_equal(got, want)
        np.testing.assert_array_equal(oracle.unpack_vect_c(got, v), x)


def test_pack_vect_c_reference_index_formula_on_a_known_element():
    # p[(c%32) + 32*(w + W*(h + H*(c/32 + C/32*n)))] = x[((n*H+h)*W+w)*C+c]
    n_, h_, w_, c_ = 2, 3, 4, 64
    x = np.zeros((n_, h_, w_, c_), dtype=np.int8)
    n, h, w, c = 1, 2, 3, 37
    x[n, h, w, c] = 99
    flat = oracle.pack_vect_c(x).reshape(-1)
    idx = (c % 32) + 32 * (w + w_ * (h + h_ * (c // 32 + c_ // 32 * n)))
    assert flat[idx] == 99 and np.count_nonzero(flat) == 1


def test_transpose_oracle_matches_numpy():
    rng = np.random.default_rng(2)
    for dtype in (np.int8, np.int32):
        for (b, r, c) in [(1, 1, 1), (2, 7, 5), (3, 64, 129), (1, 300, 17)]:
            x = rng.integers(-100, 100, size=(b, r, c)).astype(dtype)
            np.testing.assert_array_equal(oracle.transpose(x, b, r, c), x.transpose(0, 2, 1))


# ---- ABI (no GPU) -------------------------------------------------------------

import int8_kernel_lab_amd as lab
from int8_kernel_lab_amd import _lib


def test_layout_argument_errors_without_gpu():
    fake = 1 << 20  # never dereferenced: the checks fail before any launch
    for bad in [dict(vect=24), dict(vect=32, c=48), dict(vect=0)]:
        c = bad.get("c", 64)
        with pytest.raises(lab.I8ConvError) as e:
            lab.pack_vect_c(fake, fake + 4096, 1, 2, 2, c, bad["vect"])
        assert e.value.status == _lib.BAD_ARGUMENT
    with pytest.raises(lab.I8ConvError) as e:
        lab.nchw_to_nhwc(None, fake, 1, 16, 2, 2)
    assert e.value.status == _lib.BAD_ARGUMENT
    with pytest.raises(lab.I8ConvError) as e:
        lab.nhwc_to_nchw(fake, fake, 1, 2, 2, 16)  # in place is not supported
    assert e.value.status == _lib.BAD_ARGUMENT
    with pytest.raises(lab.I8ConvError) as e:
        lab.nhwk_to_nkhw(fake, fake + 16, 1 << 16, 64, 64, 64)  # 2^36 bytes
    assert e.value.status == _lib.BAD_ARGUMENT


# ---- GPU: byte for byte against the oracle ------------------------------------

def _run_gpu(fn, src: np.ndarray, out_elems: int, out_dtype, *args):
    sb = lab.DeviceBuffer.from_array(np.ascontiguousarray(src))
    db = lab.DeviceBuffer(max(1, out_elems * np.dtype(out_dtype).itemsize))
    db.fill(0x5A)
    fn(sb, db, *args)
    lab.synchronize()
    out = db.download(out_dtype, out_elems)
    sb.close()
    db.close()
    return out


TRANSPOSE_CASES = [  # (n, c, h, w)
    # tiled (16-byte rows both ways): one or two 128-column tiles per
    # workgroup, partial tiles
    (2, 128, 28, 28), (1, 64, 16, 16), (1, 512, 16, 16),
    # one side short (H x W or C not a multiple of 16): the short-row /
    # short-column forms, with 128, 112 and 16 rows (or columns) per
    # workgroup and a partial last one
    (3, 48, 5, 5), (2, 16, 33, 17), (1, 256, 7, 7), (2, 1024, 7, 7), (1, 400, 14, 14),
    (2, 64, 17, 17), (1, 32, 45, 45),
    # element form: neither side fits
    (2, 130, 9, 7), (1, 16, 47, 47),
]


@pytest.mark.gpu
@pytest.mark.parametrize("n,c,h,w", TRANSPOSE_CASES)
def test_nchw_nhwc_round_trip_bit_exact(n, c, h, w):
    from tests.conftest import say
    rng = np.random.default_rng(c * h + w)
    x_nchw = rng.integers(-128, 128, size=(n, c, h, w), dtype=np.int64).astype(np.int8)
    say(f"[gpu] nchw->nhwc {n}x{c}x{h}x{w}")
    nhwc = _run_gpu(lab.nchw_to_nhwc, x_nchw, x_nchw.size, np.int8, n, c, h, w)
    np.testing.assert_array_equal(nhwc.reshape(n, h, w, c),
                                  oracle.transpose(x_nchw, n, c, h * w).reshape(n, h, w, c))
    say(f"[gpu] nhwc->nchw {n}x{h}x{w}x{c}")
    back = _run_gpu(lab.nhwc_to_nchw, nhwc.reshape(n, h, w, c), x_nchw.size, np.int8, n, h, w, c)
    np.testing.assert_array_equal(back.reshape(x_nchw.shape), x_nchw)


@pytest.mark.gpu
@pytest.mark.parametrize("n,h,w,k", [  # tiled, short columns (H x W rows), short rows, elements
    (2, 28, 28, 128), (2, 4, 4, 52), (3, 7, 7, 36), (2, 33, 3, 256), (2, 7, 7, 520),
    (1, 14, 14, 2048), (1, 2, 2, 37), (2, 6, 6, 99), (1, 9, 11, 63)])
def test_nhwk_to_nkhw_int32_bit_exact(n, h, w, k):
    from tests.conftest import say
    rng = np.random.default_rng(k)
    y = rng.integers(-(2 ** 31), 2 ** 31, size=(n, h, w, k), dtype=np.int64).astype(np.int32)
    say(f"[gpu] nhwk->nkhw {n}x{h}x{w}x{k}")
    got = _run_gpu(lab.nhwk_to_nkhw, y, y.size, np.int32, n, h, w, k)
    np.testing.assert_array_equal(got.reshape(n, k, h, w), y.transpose(0, 3, 1, 2))


@pytest.mark.gpu
@pytest.mark.parametrize("n,h,w,c,v", [(3, 7, 9, 96, 32), (2, 28, 28, 128, 32), (1, 5, 5, 64, 16),
                                       (2, 3, 3, 128, 64), (256, 3, 3, 128, 32)])
def test_pack_vect_c_bit_exact(n, h, w, c, v):
    from tests.conftest import say
    rng = np.random.default_rng(n + c)
    x = rng.integers(-128, 128, size=(n, h, w, c), dtype=np.int64).astype(np.int8)
    say(f"[gpu] pack_vect_c {n}x{h}x{w}x{c} v{v}")
    packed = _run_gpu(lab.pack_vect_c, x, x.size, np.int8, n, h, w, c, v)
    np.testing.assert_array_equal(packed.reshape(n, c // v, h, w, v), oracle.pack_vect_c(x, v))
    back = _run_gpu(lab.unpack_vect_c, packed, x.size, np.int8, n, h, w, c, v)
    np.testing.assert_array_equal(back.reshape(x.shape), x)
