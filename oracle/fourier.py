"""TEST INFRASTRUCTURE — NOT PART OF THE PRODUCT.

numpy restatement of the reference's real-space preparation helpers, as the
checker of the GPU kernels behind torch_projectors.fourier.  Every function
works by explicit index arithmetic (no np.pad / np.fft.fftshift), so the tests
can pin it against those library routines, which are what the reference's
helpers call (through torch):

  padded_boxsize, pad_and_fftshift   tests/test_utils.py:174-247
  cropped_boxsize, ifftshift_and_crop tests/test_utils.py:250-293
  normalize_reconstruction           out = data / (weights + reg) where
                                     positive, else 0 (no reference code: the
                                     step its dual volumes exist for,
                                     paper/main.tex:72)

Only tests/ import this module.
"""
import numpy as np


def padded_boxsize(n, oversampling):
    new = int(n * oversampling)  # tests/test_utils.py:217
    return new + 1 if new % 2 else new  # :218-220


def cropped_boxsize(n, oversampling):
    return int(n / oversampling)  # tests/test_utils.py:282


def spatial_rank(shape):
    """3 when the last three sizes start with two equal ones (tests/test_utils.py:197, 271)."""
    return 3 if len(shape) >= 3 and shape[-3] == shape[-2] else 2


def pad_and_fftshift(x, oversampling):
    """fftshift(centred zero-pad(x)) over the spatial axes, one axis at a time:
    output i of an axis holds padded index (i + N - N//2) mod N, i.e. input
    index that minus pad_before, or zero outside the input."""
    x = np.asarray(x)
    dim = spatial_rank(x.shape)
    n = x.shape[-1]
    N = padded_boxsize(n, oversampling)
    pb = (N - n) // 2  # tests/test_utils.py:223-225
    out = x
    for ax in range(x.ndim - dim, x.ndim):
        src = (np.arange(N) + (N - N // 2)) % N - pb
        ok = (src >= 0) & (src < n)
        taken = np.take(out, np.where(ok, src, 0), axis=ax)
        shape = [1] * out.ndim
        shape[ax] = N
        out = np.where(ok.reshape(shape), taken, np.zeros((), dtype=x.dtype))
    return out.astype(x.dtype, copy=False)


def ifftshift_and_crop(x, oversampling):
    """ifftshift each spatial axis (output j holds input (j + L//2) mod L),
    then keep [start, start + int(cur/os)) of it, clipped like a slice."""
    x = np.asarray(x)
    dim = spatial_rank(x.shape)
    cur = x.shape[-3] if dim == 3 else x.shape[-2]  # tests/test_utils.py:273, 278
    orig = cropped_boxsize(cur, oversampling)
    start = (cur - orig) // 2  # :285-286
    out = x
    for ax in range(x.ndim - dim, x.ndim):
        L = x.shape[ax]
        keep = np.arange(start, min(start + orig, L))
        out = np.take(out, (keep + L // 2) % L, axis=ax)
    return out


def normalize_reconstruction(data, weights, reg=0.0):
    """Component-wise data / (weights + reg) in the data's real type where the
    denominator is positive, else 0."""
    data = np.asarray(data)
    real = np.float32 if data.dtype == np.complex64 else np.float64
    den = (np.asarray(weights, dtype=real) + real(reg)).astype(real)
    safe = np.where(den > 0, den, real(1))
    re = np.where(den > 0, data.real / safe, real(0)).astype(real)
    im = np.where(den > 0, data.imag / safe, real(0)).astype(real)
    out = np.empty(data.shape, dtype=data.dtype)
    out.real, out.imag = re, im
    return out
