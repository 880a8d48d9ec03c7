"""Reference preparation on the CPU: the numpy oracle (oracle/fourier.py)
pinned against the library routines the reference's helpers call, closed
forms, the C ABI's argument checks and the Python wrapper's errors.

* pad_and_fftshift == np.fft.fftshift(np.pad(...)) with the reference's
  padding split (tests/test_utils.py:217-245), for 2D, batched 2D and 3D
  inputs, odd and even edges and non-integer factors;
* ifftshift_and_crop == np.fft.ifftshift(...)[crop] with the reference's
  crop rule (tests/test_utils.py:271-293), including non-square 2D inputs
  whose slice is clipped;
* 2x centred padding leaves the spectrum's even frequencies equal to the
  unpadded spectrum / 2^dim (a wrong pad offset would add a phase ramp);
* the crop is the adjoint of the pad (dot-product test);
* normalisation at its special values.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import fourier as OF
from torch_projectors import capi, fourier

_P = ctypes.c_void_p
RNG = np.random.default_rng(20261201)
FACTORS = [1.0, 1.25, 1.5, 2.0, 2.5, 3.0]
PAD_SHAPES = [(8, 8), (7, 7), (3, 8, 8), (8, 8, 8), (9, 9, 9), (2, 6, 6, 6), (2, 3, 5, 5)]


def _lib_pad(x, os_):
    """The reference's recipe with numpy's pad and fftshift."""
    dim = 3 if x.ndim >= 3 and x.shape[-3] == x.shape[-2] else 2
    n = x.shape[-1]
    new = int(n * os_)
    if new % 2:
        new += 1
    pb = (new - n) // 2
    pa = new - n - pb
    p = np.pad(x, [(0, 0)] * (x.ndim - dim) + [(pb, pa)] * dim)
    return np.fft.fftshift(p, axes=tuple(range(x.ndim - dim, x.ndim)))


def _lib_crop(x, os_):
    dim = 3 if x.ndim >= 3 and x.shape[-3] == x.shape[-2] else 2
    cur = x.shape[-3] if dim == 3 else x.shape[-2]
    s = np.fft.ifftshift(x, axes=tuple(range(x.ndim - dim, x.ndim)))
    orig = int(cur / os_)
    a = (cur - orig) // 2
    sl = (Ellipsis,) + (slice(a, a + orig),) * dim
    return s[sl]


@pytest.mark.parametrize("shape", PAD_SHAPES, ids=[str(s) for s in PAD_SHAPES])
@pytest.mark.parametrize("os_", FACTORS)
def test_pad_matches_numpy_pad_and_fftshift(shape, os_):
    x = RNG.standard_normal(shape).astype(np.float32)
    got = OF.pad_and_fftshift(x, os_)
    exp = _lib_pad(x, os_)
    assert got.shape == exp.shape and got.dtype == exp.dtype
    assert np.array_equal(got, exp)
    xc = (RNG.standard_normal(shape) + 1j * RNG.standard_normal(shape)).astype(np.complex64)
    assert np.array_equal(OF.pad_and_fftshift(xc, os_), _lib_pad(xc, os_))


CROP_SHAPES = [(16, 16), (15, 15), (3, 16, 16), (10, 10, 10), (2, 9, 9, 9), (12, 14), (4, 12, 9)]


@pytest.mark.parametrize("shape", CROP_SHAPES, ids=[str(s) for s in CROP_SHAPES])
@pytest.mark.parametrize("os_", [1.0, 1.5, 2.0, 3.0])
def test_crop_matches_numpy_ifftshift_and_slice(shape, os_):
    x = RNG.standard_normal(shape)
    got = OF.ifftshift_and_crop(x, os_)
    exp = _lib_crop(x, os_)
    assert got.shape == exp.shape
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("shape", [(12, 12), (10, 10, 10), (3, 8, 8)])
def test_twice_padded_spectrum_at_even_frequencies(shape):
    x = RNG.standard_normal(shape)
    dim = 3 if len(shape) == 3 and shape[0] == shape[1] else 2
    axes = tuple(range(len(shape) - dim, len(shape)))
    n = shape[-1]
    X1 = np.fft.rfftn(OF.pad_and_fftshift(x, 1.0), axes=axes, norm="forward")
    X2 = np.fft.rfftn(OF.pad_and_fftshift(x, 2.0), axes=axes, norm="forward")
    full = [(2 * np.arange(n)) % (2 * n)] * (dim - 1) + [2 * np.arange(n // 2 + 1)]
    idx = np.ix_(*([np.arange(s) for s in shape[:len(shape) - dim]] + full))
    np.testing.assert_allclose(X2[idx], X1 / 2 ** dim, rtol=0, atol=1e-12 * np.abs(X1).max())
    # a pad one voxel off would not match
    bad = np.fft.rfftn(np.roll(OF.pad_and_fftshift(x, 2.0), 1, axis=-1), axes=axes, norm="forward")
    assert np.abs(bad[idx] - X1 / 2 ** dim).max() > 1e-3 * np.abs(X1).max()


@pytest.mark.parametrize("shape", [(8, 8), (6, 6, 6), (2, 10, 10)])
def test_crop_is_the_adjoint_of_the_pad(shape):
    x = RNG.standard_normal(shape)
    y = RNG.standard_normal(OF.pad_and_fftshift(x, 2.0).shape)
    lhs = np.vdot(OF.pad_and_fftshift(x, 2.0), y)
    rhs = np.vdot(x, OF.ifftshift_and_crop(y, 2.0))
    assert abs(lhs - rhs) <= 1e-12 * abs(lhs)


def test_normalize_special_values():
    d = np.array([1 + 2j, -3 + 0.5j, 4 - 4j, 7 + 7j, 1 + 1j], dtype=np.complex64)
    w = np.array([1.0, 2.0, 0.0, -1.0, 4.0], dtype=np.float32)
    out = OF.normalize_reconstruction(d, w, 0.0)
    assert out.dtype == np.complex64
    assert out[0] == d[0] and out[1] == np.complex64(-1.5 + 0.25j)
    assert out[2] == 0 and out[3] == 0  # weight + reg <= 0
    assert out[4] == np.complex64(0.25 + 0.25j)
    out = OF.normalize_reconstruction(d, w, 1.0)
    assert out[2] == d[2] and out[3] == 0 and out[0] == np.complex64(0.5 + 1j)


def test_size_helpers_match_the_reference_rules():
    for n in (1, 7, 8, 31, 64, 128, 255):
        for os_ in (1.0, 1.1, 1.25, 1.5, 2.0, 2.5, 3.0):
            assert capi.padded_boxsize(n, os_) == OF.padded_boxsize(n, os_)
            assert capi.cropped_boxsize(n, os_) == OF.cropped_boxsize(n, os_)
    assert capi.padded_boxsize(31, 1.5) == 46 and capi.rec_boxsize(31, 1.5) == 48  # different rules


@pytest.mark.parametrize("args,msg", [
    (dict(elem=3), "elem_bytes"),
    (dict(dim=4), "dim"),
    (dict(N=7), "padded_boxsize"),
    (dict(pb=9), "pad_before"),
    (dict(pb=-1), "pad_before"),
    (dict(batch=-1), "batch"),
])
def test_capi_pad_rejects(args, msg):
    a = dict(elem=4, src=_P(8), batch=1, dim=2, n=8, N=16, pb=4, dst=_P(8), stream=_P(None))
    a.update(args)
    rc = capi.lib().tp_fftshift_pad(*a.values())
    assert rc == capi.TP_ERR_INVALID
    assert msg in capi.lib().tp_last_error().decode()


@pytest.mark.parametrize("args,msg", [
    (dict(elem=5), "elem_bytes"),
    (dict(start=-1), "crop_start"),
    (dict(L1=0), "axis lengths"),
])
def test_capi_crop_rejects(args, msg):
    a = dict(elem=8, src=_P(8), batch=1, dim=2, L0=16, L1=16, L2=1, start=4, length=8, dst=_P(8),
             stream=_P(None))
    a.update(args)
    assert capi.lib().tp_ifftshift_crop(*a.values()) == capi.TP_ERR_INVALID
    assert msg in capi.lib().tp_last_error().decode()


def test_capi_normalize_rejects():
    L = capi.lib()
    assert L.tp_normalize_reconstruction(3, _P(8), _P(8), 4, 0.0, _P(8), _P(None)) == capi.TP_ERR_INVALID
    assert L.tp_normalize_reconstruction(0, _P(8), _P(8), 4, float("inf"), _P(8), _P(None)) == capi.TP_ERR_INVALID
    assert "reg" in L.tp_last_error().decode()
    assert L.tp_normalize_reconstruction(0, _P(None), _P(8), 4, 0.0, _P(8), _P(None)) == capi.TP_ERR_INVALID
    # nothing to do: no pointers needed
    assert L.tp_normalize_reconstruction(0, _P(None), _P(None), 0, 0.0, _P(None), _P(None)) == capi.TP_OK


def test_wrapper_errors_follow_the_reference():
    with pytest.raises(ValueError, match="Oversampling factor must be >= 1.0"):
        fourier.pad_and_fftshift(torch.zeros(8, 8), 0.5)
    with pytest.raises(ValueError, match="at least 2 dimensions"):
        fourier.pad_and_fftshift(torch.zeros(8), 2.0)
    with pytest.raises(ValueError, match="cubic"):
        fourier.pad_and_fftshift(torch.zeros(8, 8, 6), 2.0)
    with pytest.raises(ValueError, match="square"):
        fourier.pad_and_fftshift(torch.zeros(3, 8, 6), 2.0)
    with pytest.raises(ValueError, match="Oversampling factor must be >= 1.0"):
        fourier.ifftshift_and_crop(torch.zeros(8, 8), 0.9)
    # valid arguments on the CPU: there is no CPU path
    with pytest.raises(RuntimeError, match="on the GPU"):
        fourier.pad_and_fftshift(torch.zeros(8, 8), 2.0)
    with pytest.raises(RuntimeError, match="on the GPU"):
        fourier.ifftshift_and_crop(torch.zeros(8, 8), 2.0)


@pytest.mark.parametrize("fn,args,msg", [
    ("tp_rfftn", (5, 3, 1, 8), "dtype"),
    ("tp_rfftn", (0, 4, 1, 8), "dim"),
    ("tp_rfftn", (0, 3, -1, 8), "batch"),
    ("tp_rfftn", (0, 3, 1, 0), "boxsize"),
    ("tp_irfftn", (1, 2, 1, 1 << 31), "boxsize"),
])
def test_capi_fft_rejects(fn, args, msg):
    rc = getattr(capi.lib(), fn)(*args, _P(8), _P(8), _P(None))
    assert rc == capi.TP_ERR_INVALID
    assert msg in capi.lib().tp_last_error().decode()


def test_capi_fft_nothing_to_do():
    # no boxes: nothing enqueued, no pointers needed (no GPU touched)
    assert capi.lib().tp_rfftn(0, 3, 0, 8, _P(None), _P(None), _P(None)) == capi.TP_OK
    assert capi.lib().tp_irfftn(0, 2, 0, 8, _P(None), _P(None), _P(None)) == capi.TP_OK
