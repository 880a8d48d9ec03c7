"""Reference preparation on the GPU: the real-space steps around the FFTs
that turn a real image or volume into the projectors' rfft reconstruction
and back, and the normalisation of a backprojected (data, weight) pair.

The reference keeps the first two as tensor-op helpers next to its tests
and in its README (tests/test_utils.py:174-247 `pad_and_fftshift`,
:250-293 `ifftshift_and_crop`; README.md:106-143), which every user repeats
around the operators.  Here they keep the same names, arguments, shape rules
and errors, and run as one HIP pass each (tp_fftshift_pad /
tp_ifftshift_crop of include/torch_projectors_hip.h) instead of
F.pad + fftshift (and ifftshift + a slice).  Both are differentiable: each
one's backward is the other kernel (they are adjoints of each other).

    to_fourier(x, os)        pad_and_fftshift, then rfftn(norm="forward")
    from_fourier(X, os)      irfftn(norm="forward"), then ifftshift_and_crop
    normalize_reconstruction(data, weights, reg)
                             data / (weights + reg) where positive, else 0
    reconstruct(data, weights, os, reg)
                             normalize, then from_fourier

The FFTs are hipFFT (rocFFT) calls from the library (tp_rfftn / tp_irfftn)
with plans cached per shape, writing the row-major layout the projectors
read; inputs that require grad take torch.fft so autograd sees the chain.
Tensors must be on the GPU (no CPU path); any dtype of 2, 4, 8 or 16 bytes
moves through the pad/crop kernels.
"""
import ctypes

import torch

from . import capi

_P = ctypes.c_void_p


def _stream():
    return _P(torch.cuda.current_stream().cuda_stream)


def _on_gpu(t, what):
    if not t.is_cuda:
        raise RuntimeError(f"torch_projectors.fourier: {what} must be on the GPU (got {t.device})")


def _elem_bytes(t):
    b = t.element_size()
    if b not in (2, 4, 8, 16):
        raise RuntimeError(f"torch_projectors.fourier: unsupported dtype {t.dtype}")
    return b


def _pad_dims(shape):
    """Spatial rank and edge of pad_and_fftshift's input (tests/test_utils.py:197-214)."""
    if len(shape) < 2:
        raise ValueError("Tensor must have at least 2 dimensions")
    if len(shape) >= 3 and shape[-3] == shape[-2]:
        D, H, W = shape[-3:]
        if D != H or H != W:
            raise ValueError("3D tensors must be cubic (D == H == W)")
        return 3, D
    H, W = shape[-2:]
    if H != W:
        raise ValueError("2D tensors must be square (H == W)")
    return 2, H


def _crop_dims(shape):
    """Spatial rank and reference edge of ifftshift_and_crop's input (tests/test_utils.py:271-279)."""
    if len(shape) >= 3 and shape[-3] == shape[-2]:
        return 3, shape[-3]
    return 2, shape[-2]


def _fftshift_pad(x, dim, n, N, pb):
    x = x.contiguous()
    batch = x.numel() // (n ** dim) if n > 0 else 0
    out = torch.empty(*x.shape[:-dim], *([N] * dim), dtype=x.dtype, device=x.device)
    capi.call("tp_fftshift_pad", _elem_bytes(x), _P(x.data_ptr()), batch, dim, n, N, pb, _P(out.data_ptr()),
              _stream())
    return out


def _ifftshift_crop(x, dim, start, length):
    x = x.contiguous()
    L = list(x.shape[-dim:])
    m = [max(0, min(start + length, La) - start) for La in L]
    out = torch.empty(*x.shape[:-dim], *m, dtype=x.dtype, device=x.device)
    sp = 1
    for La in L:
        sp *= La
    batch = x.numel() // sp if sp > 0 else 0
    L3 = L + [1] * (3 - dim)
    capi.call("tp_ifftshift_crop", _elem_bytes(x), _P(x.data_ptr()), batch, dim, L3[0], L3[1], L3[2], start, length,
              _P(out.data_ptr()), _stream())
    return out


class _FftshiftPad(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, dim, n, N, pb):
        ctx.geom = (dim, n, N, pb)
        return _fftshift_pad(x, dim, n, N, pb)

    @staticmethod
    def backward(ctx, g):
        dim, n, N, pb = ctx.geom
        # adjoint: ifftshift (shift N//2), then keep [pb, pb + n) of each axis
        return _ifftshift_crop(g, dim, pb, n), None, None, None, None


class _IfftshiftCrop(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, dim, start, length):
        ctx.geom = (dim, list(x.shape[-dim:]), start, length)
        return _ifftshift_crop(x, dim, start, length)

    @staticmethod
    def backward(ctx, g):
        dim, L, start, length = ctx.geom
        m = g.shape[-1]
        if any(La != L[0] for La in L) or any(s != m for s in g.shape[-dim:]):
            raise RuntimeError("torch_projectors.fourier: the gradient of ifftshift_and_crop needs equal axes")
        # adjoint: zero-embed at `start`, then fftshift (shift L - L//2)
        return _fftshift_pad(g, dim, m, L[0], start), None, None, None


def pad_and_fftshift(tensor, oversampling_factor):
    """Zero-pad a real-space square/cube to int(n*os) (made even), centred, then
    fftshift its spatial axes (tests/test_utils.py:174-247): one HIP pass."""
    if oversampling_factor < 1.0:
        raise ValueError("Oversampling factor must be >= 1.0")
    dim, n = _pad_dims(tensor.shape)
    _on_gpu(tensor, "tensor")
    N = capi.padded_boxsize(n, oversampling_factor)
    return _FftshiftPad.apply(tensor, dim, n, N, (N - n) // 2)


def ifftshift_and_crop(real_tensor, oversampling_factor):
    """ifftshift the spatial axes, then keep the centred int(N/os) of each
    (tests/test_utils.py:250-293): one HIP pass."""
    if oversampling_factor < 1.0:
        raise ValueError("Oversampling factor must be >= 1.0")
    dim, cur = _crop_dims(real_tensor.shape)
    _on_gpu(real_tensor, "real_tensor")
    orig = capi.cropped_boxsize(cur, oversampling_factor)
    start = (cur - orig) // 2
    return _IfftshiftCrop.apply(real_tensor, dim, start, orig)


_REAL_DT = {torch.float32: capi.TP_F32, torch.float64: capi.TP_F64}
_CX_DT = {torch.complex64: capi.TP_F32, torch.complex128: capi.TP_F64}


def _rfftn(x, dim):
    """tp_rfftn of a contiguous real [..., N^dim] (norm="forward")."""
    N = x.shape[-1]
    batch = x.numel() // N ** dim
    out = torch.empty(*x.shape[:-1], N // 2 + 1, dtype=torch.complex64 if x.dtype == torch.float32
                      else torch.complex128, device=x.device)
    capi.call("tp_rfftn", _REAL_DT[x.dtype], dim, batch, N, _P(x.data_ptr()), _P(out.data_ptr()), _stream())
    return out


def _irfftn_consuming(spec, dim):
    """tp_irfftn of a contiguous [..., N^(dim-1), N/2+1] spectrum, which it overwrites."""
    N = spec.shape[-2]
    batch = spec.numel() // (N ** (dim - 1) * (N // 2 + 1))
    if spec.shape[-1] != N // 2 + 1 or any(s != N for s in spec.shape[-dim:-1]):
        raise RuntimeError(f"torch_projectors.fourier: spectrum must be [..., {'N, ' * (dim - 1)}N/2+1]")
    out = torch.empty(*spec.shape[:-1], N, dtype=torch.float32 if spec.dtype == torch.complex64
                      else torch.float64, device=spec.device)
    capi.call("tp_irfftn", _CX_DT[spec.dtype], dim, batch, N, _P(spec.data_ptr()), _P(out.data_ptr()), _stream())
    return out


def _spectrum_rank(spectrum, dim):
    if dim is None:
        s = spectrum.shape
        dim = 3 if len(s) >= 3 and s[-3] == s[-2] and s[-1] == s[-2] // 2 + 1 else 2
    return dim


def to_fourier(tensor, oversampling_factor):
    """Real square/cube -> the projectors' reconstruction, row-major:
    pad_and_fftshift, then rfftn(norm="forward") over the spatial axes
    (README.md:106-118).  The FFT is hipFFT with a cached plan; inputs that
    require grad go through torch.fft instead, so the result stays
    differentiable."""
    dim, _ = _pad_dims(tensor.shape)
    x = pad_and_fftshift(tensor, oversampling_factor)
    if x.requires_grad or x.dtype not in _REAL_DT:
        # torch.fft hands back the last axis outermost; the projectors read row-major
        return torch.fft.rfftn(x, dim=tuple(range(-dim, 0)), norm="forward").contiguous()
    return _rfftn(x, dim)


def from_fourier(spectrum, oversampling_factor, dim=None):
    """The projectors' rfft layout [..., (N,) N, N/2+1] -> real space cropped
    to int(N/os): irfftn(norm="forward") then ifftshift_and_crop.  `dim`
    (2 or 3) defaults to 3 when the last three sizes are (N, N, N/2+1)."""
    dim = _spectrum_rank(spectrum, dim)
    if oversampling_factor < 1.0:
        raise ValueError("Oversampling factor must be >= 1.0")
    _on_gpu(spectrum, "spectrum")
    N = spectrum.shape[-2]
    if spectrum.requires_grad or spectrum.dtype not in _CX_DT:
        x = torch.fft.irfftn(spectrum, s=[N] * dim, dim=tuple(range(-dim, 0)), norm="forward")
    else:
        x = _irfftn_consuming(spectrum.detach().clone(memory_format=torch.contiguous_format), dim)
    orig = capi.cropped_boxsize(N, oversampling_factor)
    return _IfftshiftCrop.apply(x, dim, (N - orig) // 2, orig)


def normalize_reconstruction(data, weights, reg=0.0):
    """data / (weights + reg) where weights + reg > 0, else 0 (a Wiener-style
    filter of a backprojected pair when reg ~ 1/SNR; reg = 0 divides by the
    accumulated weights).  data complex64/128, weights the matching real type
    and shape.  Not differentiable."""
    _on_gpu(data, "data")
    _on_gpu(weights, "weights")
    if data.dtype not in (torch.complex64, torch.complex128):
        raise RuntimeError("normalize_reconstruction: data must be complex64 or complex128")
    real = torch.float32 if data.dtype == torch.complex64 else torch.float64
    if weights.dtype != real or weights.shape != data.shape:
        raise RuntimeError(f"normalize_reconstruction: weights must be {real} with the data's shape")
    data, weights = data.detach().contiguous(), weights.detach().contiguous()
    out = torch.empty_like(data)
    capi.call("tp_normalize_reconstruction", capi.TP_F32 if real == torch.float32 else capi.TP_F64,
              _P(data.data_ptr()), _P(weights.data_ptr()), data.numel(), float(reg), _P(out.data_ptr()), _stream())
    return out


def reconstruct(data, weights, oversampling_factor, reg=0.0, dim=None):
    """normalize_reconstruction, then irfftn and ifftshift_and_crop: a
    backprojected pair to a real-space map of the original box (the
    normalised spectrum is a temporary the inverse FFT consumes)."""
    dim = _spectrum_rank(data, dim)
    if oversampling_factor < 1.0:
        raise ValueError("Oversampling factor must be >= 1.0")
    spec = normalize_reconstruction(data, weights, reg)
    N = spec.shape[-2]
    x = _irfftn_consuming(spec, dim)
    orig = capi.cropped_boxsize(N, oversampling_factor)
    return _IfftshiftCrop.apply(x, dim, (N - orig) // 2, orig)
