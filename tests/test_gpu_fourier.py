"""Reference preparation on the GPU against the numpy oracle (oracle/fourier.py).

The pad / crop kernels move elements without arithmetic and the
normalisation is one correctly rounded division per component, so all three
must equal the oracle bit for bit.  Their autograd backward is checked
against the oracle's adjoint, and the FFT-wrapped steps end to end:
to_fourier against numpy's rfftn of the oracle's padding, the projector's
identity-pose projection of a 2x-padded spectrum against the closed form
(unpadded spectrum / 2^dim, masked), and from_fourier(to_fourier(x)) == x.
"""
import numpy as np
import pytest
import torch

from oracle import fourier as OF
from tests.parity import rel_l2

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(7)
DTYPES = [torch.float32, torch.float64, torch.complex64, torch.complex128, torch.float16]


@pytest.fixture(scope="module")
def F(gpu):
    from torch_projectors import fourier
    return fourier


def _rand(shape, dtype):
    t = torch.from_numpy(RNG.standard_normal(shape))
    if dtype.is_complex:
        t = torch.complex(t, torch.from_numpy(RNG.standard_normal(shape)))
    return t.to(dtype)


PAD_CASES = [((8, 8), 2.0), ((7, 7), 1.5), ((3, 8, 8), 2.0), ((16, 16, 16), 2.0), ((9, 9, 9), 1.25),
             ((2, 6, 6, 6), 3.0), ((4, 64, 64), 2.0), ((64, 64, 64), 2.0), ((5, 5), 1.0)]


@pytest.mark.parametrize("shape,os_", PAD_CASES, ids=[f"{s}-{o}" for s, o in PAD_CASES])
@pytest.mark.parametrize("dtype", DTYPES, ids=[str(d) for d in DTYPES])
def test_pad_and_fftshift_bit_exact(F, gpu, shape, os_, dtype):
    print(f"[fourier] pad {shape} os={os_} {dtype}", flush=True)
    x = _rand(shape, dtype)
    got = F.pad_and_fftshift(x.to(gpu), os_).cpu()
    exp = torch.from_numpy(OF.pad_and_fftshift(x.numpy(), os_))
    assert got.shape == exp.shape and got.dtype == exp.dtype
    assert torch.equal(got, exp)


CROP_CASES = [((16, 16), 2.0), ((15, 15), 1.5), ((3, 16, 16), 2.0), ((20, 20, 20), 2.0), ((2, 9, 9, 9), 1.5),
              ((12, 14), 2.0), ((4, 12, 9), 1.0), ((128, 128, 128), 2.0)]


@pytest.mark.parametrize("shape,os_", CROP_CASES, ids=[f"{s}-{o}" for s, o in CROP_CASES])
@pytest.mark.parametrize("dtype", DTYPES, ids=[str(d) for d in DTYPES])
def test_ifftshift_and_crop_bit_exact(F, gpu, shape, os_, dtype):
    print(f"[fourier] crop {shape} os={os_} {dtype}", flush=True)
    x = _rand(shape, dtype)
    got = F.ifftshift_and_crop(x.to(gpu), os_).cpu()
    exp = torch.from_numpy(np.ascontiguousarray(OF.ifftshift_and_crop(x.numpy(), os_)))
    assert got.shape == exp.shape
    assert torch.equal(got, exp)


@pytest.mark.parametrize("shape", [(8, 8), (3, 10, 10), (12, 12, 12)])
def test_backward_is_the_adjoint(F, gpu, shape):
    x = _rand(shape, torch.float64).to(gpu).requires_grad_(True)
    y = F.pad_and_fftshift(x, 2.0)
    g = _rand(tuple(y.shape), torch.float64)
    (gx,) = torch.autograd.grad(y, x, g.to(gpu))
    assert torch.equal(gx.cpu(), torch.from_numpy(np.ascontiguousarray(OF.ifftshift_and_crop(g.numpy(), 2.0))))
    z = _rand(tuple(y.shape), torch.float64).to(gpu).requires_grad_(True)
    c = F.ifftshift_and_crop(z, 2.0)
    h = _rand(tuple(c.shape), torch.float64)
    (gz,) = torch.autograd.grad(c, z, h.to(gpu))
    assert torch.equal(gz.cpu(), torch.from_numpy(OF.pad_and_fftshift(h.numpy(), 2.0)))


@pytest.mark.parametrize("dtype", [torch.complex64, torch.complex128])
@pytest.mark.parametrize("reg", [0.0, 0.5, 1e-3])
def test_normalize_bit_exact(F, gpu, dtype, reg):
    real = torch.float32 if dtype == torch.complex64 else torch.float64
    d = _rand((3, 33, 17), dtype)
    w = torch.from_numpy(RNG.standard_normal((3, 33, 17))).to(real)
    w[0, :4] = 0.0
    w[1, :4] = -reg
    got = F.normalize_reconstruction(d.to(gpu), w.to(gpu), reg).cpu()
    exp = torch.from_numpy(OF.normalize_reconstruction(d.numpy(), w.numpy(), reg))
    assert torch.equal(got, exp)


@pytest.mark.parametrize("shape", [(64, 64), (4, 32, 32), (32, 32, 32)])
def test_to_fourier_matches_numpy(F, gpu, shape):
    x = _rand(shape, torch.float32)
    got = F.to_fourier(x.to(gpu), 2.0).cpu()
    dim = 3 if len(shape) == 3 and shape[0] == shape[1] else 2
    exp = np.fft.rfftn(OF.pad_and_fftshift(x.double().numpy(), 2.0), axes=tuple(range(-dim, 0)), norm="forward")
    assert rel_l2(got, torch.from_numpy(exp)) < 2e-6  # fp32 FFT


def _mask(n, cutoff=None):
    r = torch.fft.fftfreq(n, 1.0 / n)[:, None]
    c = torch.arange(n // 2 + 1)[None, :].double()
    rad = n / 2.0 if cutoff is None else cutoff
    return (r * r + c * c) <= rad * rad


def test_identity_projection_of_padded_spectrum(F, gpu):
    """2D and 3D: the os=2 identity-pose projection samples the padded
    spectrum at even frequencies, which equal the unpadded spectrum / 2^dim."""
    import torch_projectors as tp
    n = 48
    img = _rand((n, n), torch.float32)
    rec = F.to_fourier(img.to(gpu), 2.0)[None]
    proj = tp.project_2d_forw(rec, torch.eye(2, device=gpu)[None, None], output_shape=(n, n),
                              interpolation="linear", oversampling=2.0).cpu()[0, 0]
    X1 = torch.from_numpy(np.fft.rfft2(OF.pad_and_fftshift(img.double().numpy(), 1.0), norm="forward"))
    exp = torch.where(_mask(n), X1 / 4, torch.zeros((), dtype=X1.dtype))
    assert rel_l2(proj, exp) < 1e-5
    vol = _rand((n, n, n), torch.float32)
    rec3 = F.to_fourier(vol.to(gpu), 2.0)[None]
    proj3 = tp.project_3d_to_2d_forw(rec3, torch.eye(3, device=gpu)[None, None], output_shape=(n, n),
                                     interpolation="linear", oversampling=2.0).cpu()[0, 0]
    V1 = torch.from_numpy(np.fft.rfftn(OF.pad_and_fftshift(vol.double().numpy(), 1.0), norm="forward"))
    exp3 = torch.where(_mask(n), V1[0] / 8, torch.zeros((), dtype=V1.dtype))
    assert rel_l2(proj3, exp3) < 1e-5


@pytest.mark.parametrize("shape", [(64, 64), (3, 40, 40), (48, 48, 48)])
def test_round_trip(F, gpu, shape):
    x = _rand(shape, torch.float32).to(gpu)
    back = F.from_fourier(F.to_fourier(x, 2.0), 2.0, dim=3 if len(shape) == 3 and shape[0] == shape[1] else 2)
    assert back.shape == x.shape
    assert rel_l2(back.cpu(), x.cpu()) < 2e-6  # two fp32 FFTs
    spec = F.to_fourier(x, 2.0)
    ones = torch.ones(spec.shape, dtype=torch.float32, device=gpu)
    rec = F.reconstruct(spec * 2.0, ones * 2.0, 2.0, 0.0, dim=3 if len(shape) == 3 and shape[0] == shape[1] else 2)
    assert rel_l2(rec.cpu(), x.cpu()) < 2e-6


@pytest.mark.parametrize("shape", [(64, 64), (2, 48, 48), (40, 40, 40)])
def test_hipfft_and_autograd_paths(F, gpu, shape):
    """to_fourier runs hipFFT for plain inputs and torch.fft (differentiable) for
    inputs that require grad: both give the same spectrum, and the gradient
    matches the reference's recipe (F.pad, fftshift, rfftn) under autograd."""
    dim = 3 if len(shape) == 3 and shape[0] == shape[1] else 2
    x = _rand(shape, torch.float32).to(gpu)
    plain = F.to_fourier(x, 2.0)
    xg = x.clone().requires_grad_(True)
    diff = F.to_fourier(xg, 2.0)
    assert plain.is_contiguous() and diff.is_contiguous()
    assert rel_l2(plain.cpu(), diff.detach().cpu()) < 2e-6
    w = _rand(tuple(diff.shape), torch.complex64).to(gpu)
    (torch.view_as_real(diff * w).sum()).backward()
    xr = x.clone().requires_grad_(True)
    n = shape[-1]
    pb = (2 * n - n) // 2
    pad = torch.nn.functional.pad(xr, (pb, n - pb) * dim)
    ref = torch.fft.rfftn(torch.fft.fftshift(pad, dim=tuple(range(-dim, 0))), dim=tuple(range(-dim, 0)),
                          norm="forward")
    (torch.view_as_real(ref * w).sum()).backward()
    assert rel_l2(xg.grad.cpu(), xr.grad.cpu()) < 1e-6


def test_from_fourier_leaves_its_input(F, gpu):
    x = _rand((32, 32, 32), torch.float32).to(gpu)
    spec = F.to_fourier(x, 2.0)
    keep = spec.clone()
    F.from_fourier(spec, 2.0)
    torch.cuda.synchronize()
    assert torch.equal(spec, keep)


def test_plan_cache_eviction_keeps_results(F, gpu):
    """More distinct transform shapes than the library caches plans for (32): the least recently
    used plans are destroyed and made again when needed, and every transform stays correct."""
    from torch_projectors import fourier as FM
    xs = {b: _rand((b, 16, 16), torch.float32).to(gpu) for b in range(1, 41)}
    for b in list(range(1, 41)) + [1, 2, 3]:
        got = FM._rfftn(xs[b], 2).cpu()
        exp = np.fft.rfftn(xs[b].cpu().double().numpy(), axes=(-2, -1), norm="forward")
        assert rel_l2(got, torch.from_numpy(exp)) < 2e-6, b


def test_same_shape_on_two_streams(F, gpu):
    """Transforms of one shape queued on two streams at once have their own plans (and work
    areas), so neither corrupts the other."""
    from torch_projectors import fourier as FM
    a = _rand((4, 64, 64, 64), torch.float32).to(gpu)
    b = _rand((4, 64, 64, 64), torch.float32).to(gpu)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    outs = {}
    for _ in range(3):
        with torch.cuda.stream(s1):
            outs["a"] = FM._rfftn(a, 3)
        with torch.cuda.stream(s2):
            outs["b"] = FM._rfftn(b, 3)
    torch.cuda.synchronize()
    for k, x in (("a", a), ("b", b)):
        exp = np.fft.rfftn(x.cpu().double().numpy(), axes=(-3, -2, -1), norm="forward")
        assert rel_l2(outs[k].cpu(), torch.from_numpy(exp)) < 2e-6, k
