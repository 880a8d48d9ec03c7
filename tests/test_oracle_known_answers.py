"""Known answers that pin the projectors independently of the reference build.

Each check follows from the mathematics of the ops, not from their code:
central slices at the identity pose, the reference's 90-degree peak test
(tests/2d/forw/test_basic_projection.py:55-97), the Fourier shift theorem
(ibid. :100-141), impulse responses against the textbook tent and Keys
(a = -0.5) kernels including the Friedel partner (fftw_sampling.h:96-137),
backprojection impulses with the x = 0 Hermitian mirror
(projection_utils.h:482-492), the adjoint identity between the forward and its
volume gradient, and central finite differences of the pose gradients.

Every test runs against the CPU oracle; the same checks run on the HIP library
(through its C ABI) under the `gpu` marker.
"""
import math

import numpy as np
import pytest
import torch

IMPLS = ["oracle", pytest.param("hip", marks=pytest.mark.gpu)]


@pytest.fixture(params=IMPLS)
def ops(request):
    if request.param == "oracle":
        from oracle import oracle as O
        return O
    return request.getfixturevalue("hip")


def freq(i, n):
    return i if i <= n // 2 else i - n


def rand_rotations(P, seed, dim=3):
    g = np.random.default_rng(seed)
    if dim == 2:
        th = g.uniform(0, 2 * math.pi, P)
        return np.stack([np.stack([np.cos(th), -np.sin(th)], -1), np.stack([np.sin(th), np.cos(th)], -1)], -2)
    q = g.normal(size=(P, 4))
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    w, x, y, z = q.T
    return np.stack([
        np.stack([1 - 2 * (y * y + z * z), 2 * (x * y - z * w), 2 * (x * z + y * w)], -1),
        np.stack([2 * (x * y + z * w), 1 - 2 * (x * x + z * z), 2 * (y * z - x * w)], -1),
        np.stack([2 * (x * z - y * w), 2 * (y * z + x * w), 1 - 2 * (x * x + y * y)], -1)], -2)


def tent(u):
    return np.maximum(0.0, 1.0 - np.abs(u))


def keys(u, a=-0.5):
    t = np.abs(u)
    near = (a + 2) * t ** 3 - (a + 3) * t ** 2 + 1
    far = a * t ** 3 - 5 * a * t ** 2 + 8 * a * t - 4 * a
    return np.where(t <= 1, near, np.where(t < 2, far, 0.0))


def kernel(interp):
    return tent if interp == "linear" else keys


def sample_coords(R, n, os_, dim):
    """Continuous sample position of every projection pixel, float64: (..., n, n/2+1, dim) in (c, r[, d])."""
    r = np.array([freq(i, n) for i in range(n)], dtype=np.float64)[:, None] * os_
    c = np.arange(n // 2 + 1, dtype=np.float64)[None, :] * os_
    s = [np.broadcast_to(c, (n, n // 2 + 1)), np.broadcast_to(r, (n, n // 2 + 1))]
    if dim == 3:  # rows of R give (c, r, d)
        return np.stack([R[:, k, 0, None, None] * s[0] + R[:, k, 1, None, None] * s[1] for k in range(3)], -1)
    # 2D: xc = R00 sc + R01 sr, xr = R10 sc + R11 sr
    return np.stack([R[:, k, 0, None, None] * s[0] + R[:, k, 1, None, None] * s[1] for k in range(2)], -1)


def plane_through(vec):
    """A rotation whose first column (the image c axis, in (c, r, d) rows) points along vec."""
    e1 = np.asarray(vec, dtype=np.float64) / np.linalg.norm(vec)
    u = np.array([0.0, 0.0, 1.0]) if abs(e1[2]) < 0.9 else np.array([1.0, 0.0, 0.0])
    e2 = u - (u @ e1) * e1
    e2 /= np.linalg.norm(e2)
    return np.stack([e1, e2, np.cross(e1, e2)], 1)


def active_mask(n, cutoff):
    r = np.array([freq(i, n) for i in range(n)], dtype=np.float64)[:, None]
    c = np.arange(n // 2 + 1, dtype=np.float64)[None, :]
    return r * r + c * c <= cutoff * cutoff


CDT = {"f32": torch.complex64, "f64": torch.complex128}
RDT = {"f32": torch.float32, "f64": torch.float64}
TOL = {"f32": 2e-5, "f64": 1e-10}


# ----------------------------------------------------------------------------- central slices and peaks
@pytest.mark.parametrize("interp", ["linear", "cubic"])
@pytest.mark.parametrize("dim", [2, 3])
def test_identity_pose_gives_masked_central_slice(ops, interp, dim):
    n = 32
    g = torch.Generator().manual_seed(5)
    shape = (1, n, n // 2 + 1) if dim == 2 else (1, n, n, n // 2 + 1)
    rec = torch.randn(shape, generator=g, dtype=torch.complex64)
    rot = torch.eye(dim)[None, None].clone()
    fn = ops.project_2d_forw if dim == 2 else ops.project_3d_to_2d_forw
    out = fn(rec, rot, None, [n, n], interp, 1.0, None)[0, 0]
    expect = rec[0] if dim == 2 else rec[0, 0]
    m = torch.from_numpy(active_mask(n, n / 2))
    assert torch.equal(out[m], expect[m])
    assert torch.count_nonzero(out[~m]) == 0


@pytest.mark.parametrize("interp", ["linear", "cubic"])
def test_quarter_turns_move_a_peak(ops, interp):
    """A peak at (r=0, c=5) lands at (5, 0) / (n-5, 0) under the two quarter turns, with its Friedel twin."""
    n = 32
    a = 1.0 + 1.0j
    rec = torch.zeros(1, n, n // 2 + 1, dtype=torch.complex64)
    rec[0, 0, 5] = a
    rot = torch.tensor([[[1., 0.], [0., 1.]], [[0., 1.], [-1., 0.]], [[0., -1.], [1., 0.]]])[None]
    out = ops.project_2d_forw(rec, rot, None, [n, n], interp, 1.0, None)[0]
    assert out[0, 0, 5] == a
    assert out[1, 5, 0] == a and out[1, n - 5, 0] == np.conj(a)
    assert out[2, n - 5, 0] == a and out[2, 5, 0] == np.conj(a)
    for p in range(3):
        assert torch.count_nonzero(out[p]) == (1 if p == 0 else 2)


@pytest.mark.parametrize("prec", ["f32", "f64"])
def test_shift_theorem(ops, prec):
    """A phase shift by integer (s0, s1) equals the spectrum of the image rolled by (s0 rows, s1 columns)."""
    n = 32
    g = torch.Generator().manual_seed(7)
    img = torch.randn(n, n, generator=g, dtype=torch.float64)
    rec = torch.fft.rfft2(img)[None].to(CDT[prec])
    rot = torch.eye(2, dtype=RDT[prec])[None, None].clone()
    sh = torch.tensor([[[3.0, -5.0]]], dtype=RDT[prec])
    out = ops.project_2d_forw(rec, rot, sh, [n, n], "linear", 1.0, None)[0, 0]
    expect = torch.fft.rfft2(torch.roll(img, shifts=(3, -5), dims=(0, 1)))
    m = torch.from_numpy(active_mask(n, n / 2))
    err = (out[m].to(torch.complex128) - expect[m]).abs().max() / expect[m].abs().max()
    assert err < (5e-6 if prec == "f32" else 1e-12), err
    assert torch.count_nonzero(out[~m]) == 0


# ----------------------------------------------------------------------------- impulse responses
@pytest.mark.parametrize("prec", ["f32", "f64"])
@pytest.mark.parametrize("interp", ["linear", "cubic"])
@pytest.mark.parametrize("os_", [1.0, 2.0])
def test_forward_impulse_response_3d(ops, prec, interp, os_):
    """One voxel a at v: every sample x reads a*K(x - v) + conj(a)*K(x + v) (its Friedel twin)."""
    n, P = 24, 6
    N = int(math.ceil(n * os_)) + int(math.ceil(n * os_)) % 2
    v = (4, -4, 2)  # (d, r, c): c >= 1, far from the box edge, |v| = 6
    a = 0.75 - 0.5j
    rec = torch.zeros(1, N, N, N // 2 + 1, dtype=CDT[prec])
    rec[0, v[0] % N, v[1] % N, v[2]] = a
    R = rand_rotations(P, 3)
    R[0] = plane_through((v[2], v[1], v[0]))  # pose 0 samples v itself at (r=0, c=6/os)
    rot = torch.from_numpy(R)[None].to(RDT[prec])
    out = ops.project_3d_to_2d_forw(rec, rot, None, [n, n], interp, os_, None)[0].to(torch.complex128).numpy()
    x = sample_coords(R, n, os_, 3)  # (P, n, h, 3) in (c, r, d)
    vv = np.array([v[2], v[1], v[0]], dtype=np.float64)
    K = kernel(interp)
    kp = np.prod(K(x - vv), -1)
    km = np.prod(K(x + vv), -1)
    expect = a * kp + np.conj(a) * km
    expect[:, ~active_mask(n, n / 2)] = 0
    assert np.abs(out - expect).max() < TOL[prec] * (30 if interp == "cubic" else 10)
    assert np.abs(expect).max() > 0.3  # the impulse is actually sampled


@pytest.mark.parametrize("prec", ["f32", "f64"])
@pytest.mark.parametrize("interp", ["linear", "cubic"])
def test_forward_impulse_response_2d(ops, prec, interp):
    n, P, os_ = 32, 8, 2.0
    N = 64
    v = (-6, 5)  # (r, c)
    a = -0.25 + 1.0j
    rec = torch.zeros(1, N, N // 2 + 1, dtype=CDT[prec])
    rec[0, v[0] % N, v[1]] = a
    R = rand_rotations(P, 4, dim=2)
    rot = torch.from_numpy(R)[None].to(RDT[prec])
    out = ops.project_2d_forw(rec, rot, None, [n, n], interp, os_, None)[0].to(torch.complex128).numpy()
    x = sample_coords(R, n, os_, 2)  # (c, r)
    vv = np.array([v[1], v[0]], dtype=np.float64)
    K = kernel(interp)
    expect = a * np.prod(K(x - vv), -1) + np.conj(a) * np.prod(K(x + vv), -1)
    expect[:, ~active_mask(n, n / 2)] = 0
    assert np.abs(out - expect).max() < TOL[prec] * 30
    assert np.abs(expect).max() > 0.3


@pytest.mark.parametrize("prec", ["f32", "f64"])
@pytest.mark.parametrize("interp", ["linear", "cubic"])
def test_backprojection_impulse_3d(ops, prec, interp):
    """One projection pixel p (weight w) at sample x: cell u gets K(x-u) p + K(x+u) conj(p), weights w|K|."""
    n, os_ = 16, 2.0
    N = 32
    R = rand_rotations(1, 9)
    rot = torch.from_numpy(R)[None].to(RDT[prec])
    i0, j0 = n - 3, 4  # r = -3, c = 4: |x| = 10 voxels, far from the edge and the origin
    p, w = 0.5 + 2.0j, 0.625
    proj = torch.zeros(1, 1, n, n // 2 + 1, dtype=CDT[prec])
    proj[0, 0, i0, j0] = p
    wts = torch.zeros(1, 1, n, n // 2 + 1, dtype=RDT[prec])
    wts[0, 0, i0, j0] = w
    data, wrec = ops.backproject_2d_to_3d_forw(proj, wts, rot, None, interp, os_, None)
    data, wrec = data[0].to(torch.complex128).numpy(), wrec[0].to(torch.float64).numpy()
    x = sample_coords(R, n, os_, 3)[0, i0, j0]  # (c, r, d)
    f = np.array([freq(i, N) for i in range(N)], dtype=np.float64)
    U = np.stack(np.meshgrid(np.arange(N // 2 + 1, dtype=np.float64), f, f, indexing="ij"), -1)  # (c, r, d)
    U = np.transpose(U, (2, 1, 0, 3))  # -> [d, r, c, (c, r, d)]
    K = kernel(interp)
    kp, km = np.prod(K(x - U), -1), np.prod(K(x + U), -1)
    expect = kp * p + km * np.conj(p)
    expect_w = w * (np.abs(kp) + np.abs(km))
    assert np.abs(data - expect).max() < TOL[prec] * 30
    assert np.abs(wrec - expect_w).max() < TOL[prec] * 30
    assert np.abs(expect).max() > 0.3


@pytest.mark.parametrize("prec", ["f32", "f64"])
def test_backprojection_impulse_on_x0_plane_mirrors(ops, prec):
    """A sample whose stencil touches c = 0 also deposits conj at (-r, -d) on that plane."""
    n, os_ = 16, 1.0
    N = 16
    th = 1.2
    # rotation about the row axis keeps xr = sr and tilts c into d, so small c lands near the c = 0 plane
    R = np.array([[[math.cos(th), 0, -math.sin(th)], [0, 1, 0], [math.sin(th), 0, math.cos(th)]]])
    rot = torch.from_numpy(R)[None].to(RDT[prec])
    i0, j0 = 3, 1
    p = 1.0 - 0.5j
    proj = torch.zeros(1, 1, n, n // 2 + 1, dtype=CDT[prec])
    proj[0, 0, i0, j0] = p
    data, _ = ops.backproject_2d_to_3d_forw(proj, None, rot, None, "linear", os_, None)
    data = data[0].to(torch.complex128).numpy()
    x = sample_coords(R, n, os_, 3)[0, i0, j0]
    f = np.array([freq(i, N) for i in range(N)], dtype=np.float64)
    U = np.transpose(np.stack(np.meshgrid(np.arange(N // 2 + 1, dtype=np.float64), f, f, indexing="ij"), -1),
                     (2, 1, 0, 3))
    expect = np.prod(tent(x - U), -1) * p + np.prod(tent(x + U), -1) * np.conj(p)
    assert np.abs(expect[:, :, 0]).max() > 0.1  # the c = 0 plane is hit
    assert np.abs(data - expect).max() < TOL[prec] * 10


# ----------------------------------------------------------------------------- adjoint and gradients
def _x0_half(n):
    """Pixels the backward ops skip: column 0 with row index >= n/2."""
    m = np.zeros((n, n // 2 + 1), dtype=bool)
    m[n // 2:, 0] = True
    return torch.from_numpy(m)


@pytest.mark.parametrize("prec", ["f32", "f64"])
@pytest.mark.parametrize("interp", ["linear", "cubic"])
def test_volume_gradient_is_the_adjoint_of_the_forward(ops, prec, interp):
    """Re<P x, y> = Re<x, P^T y> for y zero on the skipped x = 0 half-line, cutoff inside the box."""
    n, P, os_ = 16, 5, 2.0
    N = 32
    g = torch.Generator().manual_seed(21)
    x = torch.randn(1, N, N, N // 2 + 1, generator=g, dtype=torch.complex128).to(CDT[prec])
    y = torch.randn(1, P, n, n // 2 + 1, generator=g, dtype=torch.complex128)
    y[:, :, _x0_half(n)] = 0
    y = y.to(CDT[prec])
    rot = torch.from_numpy(rand_rotations(P, 22))[None].to(RDT[prec])
    sh = (torch.rand(1, P, 2, generator=g, dtype=torch.float64) * 6 - 3).to(RDT[prec])
    cut = 6.0  # taps stay inside [-N/2+1, N/2], where the forward's clamp and the scatter's drop agree
    px = ops.project_3d_to_2d_forw(x, rot, sh, [n, n], interp, os_, cut)
    pty, _, _ = ops.project_3d_to_2d_back(y, x, rot, sh, interp, os_, cut)
    lhs = (px.conj().to(torch.complex128) * y.to(torch.complex128)).real.sum().item()
    rhs = (x.conj().to(torch.complex128) * pty.to(torch.complex128)).real.sum().item()
    assert abs(lhs - rhs) <= (1e-5 if prec == "f32" else 1e-12) * (abs(lhs) + abs(rhs)), (lhs, rhs)


@pytest.mark.parametrize("dim", [2, 3])
def test_pose_gradients_match_finite_differences(ops, dim):
    """d/dR and d/ds of L = Re sum conj(g) * forward(x; R, s), complex128, cubic (C1 in R and s)."""
    n, P, os_ = 16, 3, 2.0
    N = 32
    g = torch.Generator().manual_seed(31)
    shape = (1, N, N // 2 + 1) if dim == 2 else (1, N, N, N // 2 + 1)
    x = torch.randn(shape, generator=g, dtype=torch.complex128)
    up = torch.randn(1, P, n, n // 2 + 1, generator=g, dtype=torch.complex128)
    up[:, :, _x0_half(n)] = 0
    R0 = torch.from_numpy(rand_rotations(P, 32, dim=dim))[None].to(torch.float64)
    s0 = torch.rand(1, P, 2, generator=g, dtype=torch.float64) * 4 - 2
    cut = 6.0
    fwd = ops.project_2d_forw if dim == 2 else ops.project_3d_to_2d_forw
    back = ops.project_2d_back if dim == 2 else ops.project_3d_to_2d_back

    def loss(R, s):
        return (up.conj() * fwd(x, R, s, [n, n], "cubic", os_, cut)).real.sum().item()

    _, grot, gsh = back(up, x, R0.clone().requires_grad_(True), s0.clone().requires_grad_(True), "cubic", os_, cut)
    eps = 1e-6
    fd_rot = torch.zeros_like(R0)
    for idx in np.ndindex(*R0.shape):
        e = torch.zeros_like(R0)
        e[idx] = eps
        fd_rot[idx] = (loss(R0 + e, s0) - loss(R0 - e, s0)) / (2 * eps)
    fd_sh = torch.zeros_like(s0)
    for idx in np.ndindex(*s0.shape):
        e = torch.zeros_like(s0)
        e[idx] = eps
        fd_sh[idx] = (loss(R0, s0 + e) - loss(R0, s0 - e)) / (2 * eps)
    if dim == 3:  # the third column multiplies s_d = 0: no gradient there
        assert torch.count_nonzero(grot.cpu()[..., 2]) == 0
    scale = fd_rot.abs().max().item()
    assert (grot.cpu() - fd_rot).abs().max().item() < 1e-6 * scale
    assert (gsh.cpu() - fd_sh).abs().max().item() < 1e-6 * fd_sh.abs().max().item()
