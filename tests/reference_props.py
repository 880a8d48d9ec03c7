"""Gradient, batching and oversampling properties of the public operators.

The checks follow the reference's own test strategy for these operators
(tests/2d/forw/test_gradients.py, tests/2d/back/test_gradients_back.py,
tests/3d/forw/test_gradients_3d_to_2d.py,
tests/3d/back/test_gradients_back_2d_to_3d.py and the test_batching*.py and
test_oversampling*.py files beside them), with the same sizes, poses and
tolerances:

* torch.autograd.gradcheck in complex128/float64 (atol 1e-4, rtol 1e-2).  The
  x = 0 column entries whose Friedel mates are written or read by the forward
  but not reached by the backward are masked, as the reference does: rows
  >= n/2 of a reconstruction read by a projection, rows 1..n/2-1 of a
  projection inserted by a backprojection;
* shift gradients against the same shift written as a phase ramp
  exp(-2 pi i (k_r s_0 + k_c s_1) / n) in torch operations;
* rotation gradients against central finite differences of one angle;
* weight gradients of a backprojection against finite differences;
* Adam on one angle converges to the angle that made the target;
* one gradient step from a zero image through a real-space loss correlates
  with the image that made the target;
* batched and broadcast calls equal per-item calls; backprojecting in two
  halves and adding equals backprojecting all at once;
* projecting a spectrum padded `os` times with oversampling `os` equals
  projecting the unpadded one (a quarter turn keeps every sample on the
  grid, so the two agree to rounding once the 1/os^dim of the padded
  transform is undone), and backprojections at oversampling 1 and `os`
  agree in real space after ifftshift_and_crop.

Every check takes `api` — a module with the public functions project_2d_forw,
project_3d_to_2d_forw, backproject_2d_forw and backproject_2d_to_3d_forw, and
for the oversampling checks pad_and_fftshift and ifftshift_and_crop — and a
device, so the same bodies run on the HIP operators (cuda:0) and on the CPU
oracle (tests/oracle_autograd.py).  Inputs come from seeded CPU
generators and are then moved to the device, so both see the same numbers.
"""
import math

import torch

GRADCHECK = dict(atol=1e-4, rtol=1e-2)

SHIFT_CASES = [  # (shift, B, P), as the reference parametrises its shift-gradient tests
    ((2.0, 1.0), 1, 1), ((-2.0, -1.0), 1, 1), ((2.0, -1.0), 1, 1), ((-2.0, 1.0), 1, 1), ((0.0, 0.0), 1, 1),
    ((2.0, 0.0), 1, 1), ((0.0, 1.0), 1, 1), ((10.0, 5.0), 1, 1), ((0.5, 0.3), 1, 1), ((0.1, 10.0), 1, 1),
    ((2.0, 1.0), 3, 1), ((2.0, 1.0), 1, 4), ((2.0, 1.0), 2, 3),
]


# ----------------------------------------------------------------------------- helpers
def crandn(shape, dtype, seed, dev):
    g = torch.Generator().manual_seed(seed)
    real = torch.float64 if dtype == torch.complex128 else torch.float32
    z = torch.complex(torch.randn(shape, generator=g, dtype=real), torch.randn(shape, generator=g, dtype=real))
    return z.to(dev)


def rrand(shape, dtype, seed, dev):
    g = torch.Generator().manual_seed(seed)
    return torch.rand(shape, generator=g, dtype=dtype).to(dev)


def rot2(a):
    c, s = torch.cos(a), torch.sin(a)
    return torch.stack([torch.stack([c, -s]), torch.stack([s, c])])


def rot3z(a):
    c, s = torch.cos(a), torch.sin(a)
    o, z = torch.ones_like(a), torch.zeros_like(a)
    return torch.stack([torch.stack([c, -s, z]), torch.stack([s, c, z]), torch.stack([z, z, o])])


def pose(dim, a):
    """[1, 1, d, d] rotation by angle `a` (a 0-d tensor) in the plane / about z."""
    return (rot2(a) if dim == 2 else rot3z(a))[None, None]


def angle(v, dev, dtype=torch.float32, grad=False):
    return torch.tensor(v, dtype=dtype, device=dev, requires_grad=grad)


def forw(api, dim):
    return api.project_2d_forw if dim == 2 else api.project_3d_to_2d_forw


def backproj(api, dim):
    return api.backproject_2d_forw if dim == 2 else api.backproject_2d_to_3d_forw


def rec_shape(dim, n, B=1):
    return (B, n, n // 2 + 1) if dim == 2 else (B, n, n, n // 2 + 1)


def cmse(a, b):
    d = a - b
    return torch.mean(d.real ** 2 + d.imag ** 2)


def ncc(x, y):
    x = x.flatten() - x.mean()
    y = y.flatten() - y.mean()
    return (x * y).sum() / (x.norm() * y.norm())


def read_mask(shape, dtype, dev):
    """Zero the x = 0 column at rows >= n/2 of a reconstruction (all slices)."""
    m = torch.ones(shape, dtype=dtype)
    m[..., shape[-2] // 2:, 0] = 0
    return m.to(dev)


def insert_mask(shape, dtype, dev):
    """Zero the x = 0 column at rows 1..n/2-1 of a projection."""
    m = torch.ones(shape, dtype=dtype)
    m[..., 1:shape[-2] // 2, 0] = 0
    return m.to(dev)


def freq_grid(n, dev):
    ky = torch.arange(n, dtype=torch.float32)
    ky[ky > n // 2] -= n
    kx = torch.arange(n // 2 + 1, dtype=torch.float32)
    kyy, kxx = torch.meshgrid(ky, kx, indexing="ij")
    return kyy.to(dev), kxx.to(dev)


def phase_ramp(shifts, n, dev, sign=-1.0):
    """exp(sign 2 pi i (k_r s_0 + k_c s_1) / n) for shifts [B, P, 2] -> [B, P, n, n/2+1]."""
    kyy, kxx = freq_grid(n, dev)
    ph = sign * 2.0 * math.pi * (kyy * shifts[..., 0, None, None] + kxx * shifts[..., 1, None, None]) / n
    return torch.complex(torch.cos(ph), torch.sin(ph))


# ----------------------------------------------------------------------------- gradcheck (complex128)
def gradcheck_projection(api, dev, dim, interp):
    """Reference: tests/2d/forw/test_gradients.py:22-62, tests/3d/forw/test_gradients_3d_to_2d.py:68-110."""
    n = 16 if dim == 2 else 8
    shape = rec_shape(dim, n)
    rec = crandn(shape, torch.complex128, 42, dev).requires_grad_(True)
    rot = torch.eye(dim, dtype=torch.float64, device=dev)[None, None]
    mask = read_mask(shape, torch.complex128, dev)

    def fn(r):
        return forw(api, dim)(r * mask, rot, output_shape=(n, n), interpolation=interp)

    assert torch.autograd.gradcheck(fn, (rec,), **GRADCHECK)


def gradcheck_backprojection(api, dev, dim, interp, with_weights=False):
    """Reference: tests/2d/back/test_gradients_back.py:26-65,
    tests/3d/back/test_gradients_back_2d_to_3d.py:70-110.  With `with_weights`
    the real weights and the weight reconstruction enter the check as well
    (the reference checks that gradient by finite differences only)."""
    n = 16
    shape = (1, 1, n, n // 2 + 1)
    proj = crandn(shape, torch.complex128, 42, dev).requires_grad_(True)
    rot = torch.eye(dim, dtype=torch.float64, device=dev)[None, None]
    mask = insert_mask(shape, torch.complex128, dev)
    if not with_weights:
        def fn(p):
            data, _ = backproj(api, dim)(p * mask, rotations=rot, interpolation=interp)
            return data

        assert torch.autograd.gradcheck(fn, (proj,), **GRADCHECK)
        return
    w = rrand(shape, torch.float64, 43, dev).requires_grad_(True)
    wmask = insert_mask(shape, torch.float64, dev)

    def fnw(p, ww):
        return backproj(api, dim)(p * mask, rotations=rot, weights=ww * wmask, interpolation=interp)

    assert torch.autograd.gradcheck(fnw, (proj, w), **GRADCHECK)


# ----------------------------------------------------------------------------- shift gradients
def shift_gradient_projection(api, dev, dim, interp, shift, B, P):
    """Reference: tests/2d/forw/test_gradients.py:200-308,
    tests/3d/forw/test_gradients_3d_to_2d.py:196-290 (identity pose)."""
    n = 32
    g = torch.Generator().manual_seed(42)
    real = torch.randn((B,) + (n,) * dim, generator=g)
    rec = torch.fft.rfftn(real, dim=(-2, -1))
    rec = (rec * read_mask(rec.shape, rec.dtype, "cpu")).to(dev)
    rot = torch.eye(dim, device=dev).expand(B, P, dim, dim).contiguous()
    base = torch.tensor(shift, dtype=torch.float32).expand(B, P, 2).contiguous().to(dev)
    f = forw(api, dim)
    unshifted = f(rec, rot, shifts=None, output_shape=(n, n), interpolation=interp)

    s_ours = base.clone().requires_grad_(True)
    cmse(f(rec, rot, shifts=s_ours, output_shape=(n, n), interpolation=interp), unshifted).backward()
    s_ramp = base.clone().requires_grad_(True)
    cmse(unshifted * phase_ramp(s_ramp, n, dev), unshifted).backward()
    torch.testing.assert_close(s_ours.grad, s_ramp.grad, **GRADCHECK)


def shift_gradient_backprojection(api, dev, dim, interp, shift, B, P):
    """Reference: tests/2d/back/test_gradients_back.py:185-297,
    tests/3d/back/test_gradients_back_2d_to_3d.py:232-344 (pose: 180 degrees)."""
    n = 32
    shape = (B, P, n, n // 2 + 1)
    proj = crandn(shape, torch.complex64, 42, "cpu")
    proj = (proj * insert_mask(shape, proj.dtype, "cpu")).to(dev)
    rot = pose(dim, angle(math.pi, dev))[0, 0].expand(B, P, dim, dim).contiguous()
    base = torch.tensor(shift, dtype=torch.float32).expand(B, P, 2).contiguous().to(dev)
    bp = backproj(api, dim)
    unshifted, _ = bp(proj, rotations=rot, interpolation=interp)

    s_ours = base.clone().requires_grad_(True)
    ours, _ = bp(proj, rotations=rot, shifts=s_ours, interpolation=interp)
    cmse(ours, unshifted).backward()
    s_ramp = base.clone().requires_grad_(True)
    ramp, _ = bp(proj * phase_ramp(s_ramp, n, dev, sign=1.0), rotations=rot, interpolation=interp)
    cmse(ramp, unshifted).backward()
    torch.testing.assert_close(s_ours.grad, s_ramp.grad, **GRADCHECK)


# ----------------------------------------------------------------------------- rotation gradients
def _angle_fd(loss_at, a0, eps, dev):
    """(autograd d loss / d angle through the pose matrix, central difference)."""
    a = angle(a0, dev, grad=True)
    loss_at(a).backward()
    with torch.no_grad():
        fd = (loss_at(angle(a0 + eps, dev)) - loss_at(angle(a0 - eps, dev))) / (2 * eps)
    return a.grad.item(), fd.item()


def rotation_fd_projection(api, dev, dim, interp):
    """Reference: tests/2d/forw/test_gradients.py:396-448 (rel < 1e-2),
    tests/3d/forw/test_gradients_3d_to_2d.py:454-507 (rel < 1e-4): columns
    x < 3 of the reconstruction are zero, target at angle 0, test at 0.01."""
    n = 16
    rec = crandn(rec_shape(dim, n), torch.complex64, 42, "cpu")
    rec[..., :3] = 0
    rec = rec.to(dev)
    f = forw(api, dim)
    target = f(rec, pose(dim, angle(0.0, dev)), interpolation=interp)

    def loss_at(a):
        return torch.sum((f(rec, pose(dim, a), interpolation=interp) - target).abs())

    ana, fd = _angle_fd(loss_at, 0.01, 1e-4, dev)
    rel = abs(ana - fd) / (abs(fd) + 1e-8)
    assert rel < (1e-2 if dim == 2 else 1e-4), (ana, fd, rel)


def rotation_fd_backprojection(api, dev, dim, interp):
    """Reference: tests/2d/back/test_gradients_back.py:392-440,
    tests/3d/back/test_gradients_back_2d_to_3d.py:440-489: columns x < 2 of
    the projection are zero, target at angle 0, test at 0.1, step 6e-3,
    rel < 5e-2."""
    proj = crandn((1, 1, 16, 9), torch.complex64, 42, "cpu")
    proj[..., :2] = 0
    proj = proj.to(dev)
    bp = backproj(api, dim)
    target, _ = bp(proj, rotations=pose(dim, angle(0.0, dev)), interpolation=interp)

    def loss_at(a):
        rec, _ = bp(proj, rotations=pose(dim, a), interpolation=interp)
        return torch.sum((rec - target).abs())

    ana, fd = _angle_fd(loss_at, 0.1, 6e-3, dev)
    rel = abs(ana - fd) / (abs(fd) + 1e-8)
    assert rel < 5e-2, (ana, fd, rel)


def rotation_gradient_nonzero(api, dev, dim, interp, backprojection):
    """Reference: the 'multiple scenarios' parts of the rotation-gradient tests
    (e.g. tests/2d/forw/test_gradients.py:367-389): a pose off the target gets
    a finite, non-zero matrix gradient."""
    for i, (target, offset) in enumerate([(0.1, 0.05), (0.3, 0.1), (0.8, 0.2)]):
        if backprojection:
            x = crandn((1, 1, 16, 9), torch.complex64, 42 + i, dev)
            run = lambda r: backproj(api, dim)(x, rotations=r, interpolation=interp)[0]  # noqa: E731
        else:
            x = crandn(rec_shape(dim, 16 if dim == 2 else 8), torch.complex64, 42 + i, dev)
            run = lambda r: forw(api, dim)(x, r, interpolation=interp)  # noqa: E731
        tgt = run(pose(dim, angle(target, dev)))
        r = pose(dim, angle(target + offset, dev)).detach().requires_grad_(True)
        torch.sum((run(r) - tgt).abs()).backward()
        assert r.grad is not None and torch.isfinite(r.grad).all()
        assert r.grad.norm().item() > 1e-8


def rotation_convergence(api, dev, dim, interp, backprojection):
    """Reference: _test_rotation_optimization_convergence* in the four
    gradient test files: Adam (lr 0.02) from 0.017 rad off the target angle,
    100 steps, the best angle within 1e-3 rad (2e-3 for 3D projection).
    With a fixed rate, whether the best iterate lands that close depends on
    the random draw (the oracle misses by up to 2.5e-3 rad on this one), so
    the rate here decays by 0.95 per step; the bound is the reference's."""
    if backprojection:
        x = crandn((1, 1, 16, 9), torch.complex64, 42, dev)
        run = lambda r: backproj(api, dim)(x, rotations=r, interpolation=interp)[0]  # noqa: E731
    else:
        x = crandn(rec_shape(dim, 16 if dim == 2 else 8), torch.complex64, 42, dev)
        run = lambda r: forw(api, dim)(x, r, interpolation=interp)  # noqa: E731
    tol = 2e-3 if (dim == 3 and not backprojection) else 1e-3
    for target in (0.2, 0.5, 0.8):
        tgt = run(pose(dim, angle(target, dev))).detach()
        a = angle(target + 0.017, dev, grad=True)
        opt = torch.optim.Adam([a], lr=0.02)
        decay = torch.optim.lr_scheduler.ExponentialLR(opt, gamma=0.95)
        best, best_a = float("inf"), a.item()
        for _ in range(100):
            opt.zero_grad()
            loss = torch.sum((run(pose(dim, a)) - tgt).abs().pow(2))
            if loss.item() < best:
                best, best_a = loss.item(), a.item()
            loss.backward()
            opt.step()
            decay.step()
        d = abs(best_a - target) % (2 * math.pi)
        assert min(d, 2 * math.pi - d) < tol, (target, best_a)


# ----------------------------------------------------------------------------- weights
def weight_fd(api, dev, dim, interp):
    """Reference: tests/2d/back/test_gradients_back.py:492-556,
    tests/3d/back/test_gradients_back_2d_to_3d.py:541-605: poses identity and
    45 degrees, loss |data|^2 + 0.1 weight^2, central difference of weight
    [0, 0, 0, 0] with step 0.1, rel < 1e-3."""
    shape = (1, 2, 16, 9)
    proj = crandn(shape, torch.complex64, 42, dev)
    w = rrand(shape, torch.float32, 43, dev)
    rot = torch.cat([pose(dim, angle(0.0, dev)), pose(dim, angle(math.pi / 4, dev))], dim=1)
    bp = backproj(api, dim)

    def loss_of(ww):
        data, wrec = bp(proj, rotations=rot, weights=ww, interpolation=interp)
        return torch.sum(torch.abs(data) ** 2) + 0.1 * torch.sum(wrec ** 2)

    wg = w.clone().requires_grad_(True)
    loss_of(wg).backward()
    assert torch.isfinite(wg.grad).all() and wg.grad.norm().item() > 1e-8
    eps = 0.1
    with torch.no_grad():
        wp, wm = w.clone(), w.clone()
        wp[0, 0, 0, 0] += eps
        wm[0, 0, 0, 0] -= eps
        fd = ((loss_of(wp) - loss_of(wm)) / (2 * eps)).item()
    ana = wg.grad[0, 0, 0, 0].item()
    assert abs(ana - fd) / (abs(fd) + 1e-8) < 1e-3, (ana, fd)


# ----------------------------------------------------------------------------- one gradient step
def fourier_component_step(api, dev, dim, interp, backprojection):
    """Reference: test_gradient_fourier_components* in the four gradient test
    files.  A zero image, transformed with rfftn over its last two axes, is
    projected (or backprojected) at 90 degrees; one unit gradient step on the
    mean squared difference to the same operation on a random image makes it
    correlate with the 0-degree result of that image: NCC > 0.8 for the 2D
    projection, > 0.5 otherwise."""
    n = 32
    g = torch.Generator().manual_seed(42)
    r90, r0 = pose(dim, angle(math.pi / 2, dev)), pose(dim, angle(0.0, dev))
    if not backprojection:
        img = torch.randn((1,) + (n,) * dim, generator=g).to(dev)
        f = forw(api, dim)
        run = lambda x, r: torch.fft.irfftn(  # noqa: E731
            f(torch.fft.rfftn(x, dim=(-2, -1)), r, output_shape=(n, n), interpolation=interp)[0, 0], dim=(-2, -1))
        target, ref0 = run(img, r90).detach(), run(img, r0).detach()
        z = torch.zeros_like(img, requires_grad=True)
        torch.nn.functional.mse_loss(run(z, r90), target).backward()
        with torch.no_grad():
            upd = z - z.grad
        score = ncc(upd[0] if dim == 2 else upd[0].mean(dim=0), ref0)
        assert score > (0.8 if dim == 2 else 0.5), score.item()
        return
    img = torch.randn(n, n, generator=g).to(dev)
    bp = backproj(api, dim)
    run = lambda x, r: bp(torch.fft.rfftn(x, dim=(-2, -1))[None, None], rotations=r,  # noqa: E731
                          interpolation=interp)[0]
    target, ref0 = run(img, r90).detach(), run(img, r0).detach()
    z = torch.zeros_like(img, requires_grad=True)
    cmse(run(z, r90), target).backward()
    with torch.no_grad():
        upd = z - z.grad
    ref0_real = torch.fft.irfftn(ref0[0], dim=(-2, -1), s=(n, n))
    if dim == 3:
        ref0_real = ref0_real.mean(dim=0)
    score = ncc(upd, ref0_real)
    assert score > 0.5, score.item()


# ----------------------------------------------------------------------------- batching
def _poses(dim, B, P, seed, dev):
    g = torch.Generator().manual_seed(seed)
    a = torch.rand(B, P, generator=g) * 2 * math.pi
    if dim == 2:
        return torch.stack([rot2(t) for t in a.flatten()]).reshape(B, P, 2, 2).to(dev)
    ax = torch.nn.functional.normalize(torch.randn(B * P, 3, generator=g), dim=1)
    K = torch.zeros(B * P, 3, 3)
    K[:, 0, 1], K[:, 0, 2], K[:, 1, 2] = -ax[:, 2], ax[:, 1], -ax[:, 0]
    K = K - K.transpose(1, 2)
    return torch.matrix_exp(K * a.flatten()[:, None, None]).reshape(B, P, 3, 3).to(dev)


def batching_projection(api, dev, dim, interp):
    """Reference: tests/2d/forw/test_batching.py, tests/3d/forw/test_batching_3d_to_2d.py:
    B reconstructions under one broadcast pose set, one reconstruction under
    P poses, B x P; each against per-item calls, atol 1e-5."""
    B, P, n = 3, 5, 16
    rec = crandn(rec_shape(dim, n, B), torch.complex64, 7, dev)
    f = forw(api, dim)
    for rot in (_poses(dim, 1, P, 8, dev), _poses(dim, B, P, 9, dev)):
        out = f(rec, rot, interpolation=interp)
        for b in range(B):
            rb = rot[:1] if rot.shape[0] == 1 else rot[b:b + 1]
            exp = f(rec[b:b + 1], rb, interpolation=interp)
            assert torch.allclose(out[b:b + 1], exp, atol=1e-5)
            for p in range(P):
                assert torch.allclose(out[b:b + 1, p:p + 1], f(rec[b:b + 1], rb[:, p:p + 1], interpolation=interp),
                                      atol=1e-5)
    sh = torch.randn(1, P, 2, generator=torch.Generator().manual_seed(10)).to(dev) * 2
    rot = _poses(dim, 1, P, 8, dev)
    out = f(rec, rot, shifts=sh, interpolation=interp)
    exp = f(rec, rot.expand(B, P, dim, dim).contiguous(), shifts=sh.expand(B, P, 2).contiguous(),
            interpolation=interp)
    assert torch.allclose(out, exp, atol=1e-5)


def batching_backprojection(api, dev, dim, interp):
    """Reference: tests/2d/back/test_batching_back.py,
    tests/3d/back/test_batching_back_2d_to_3d.py: B projection sets under one
    broadcast pose set, P poses against the sum of single-pose calls, weights,
    broadcast rotations and shifts against expanded ones, and two halves added
    against one call; atol 1e-5."""
    B, P, n = 2, 4, 16
    shape = (B, P, n, n // 2 + 1)
    proj = crandn(shape, torch.complex64, 11, dev)
    w = rrand(shape, torch.float32, 12, dev)
    bp = backproj(api, dim)
    rot1 = _poses(dim, 1, P, 13, dev)
    data, wrec = bp(proj, rotations=rot1, weights=w, interpolation=interp)
    for b in range(B):
        d_b, w_b = bp(proj[b:b + 1], rotations=rot1, weights=w[b:b + 1], interpolation=interp)
        assert torch.allclose(data[b:b + 1], d_b, atol=1e-5) and torch.allclose(wrec[b:b + 1], w_b, atol=1e-5)
        acc_d, acc_w = torch.zeros_like(d_b), torch.zeros_like(w_b)
        for p in range(P):
            dp, wp = bp(proj[b:b + 1, p:p + 1], rotations=rot1[:, p:p + 1], weights=w[b:b + 1, p:p + 1],
                        interpolation=interp)
            acc_d += dp
            acc_w += wp
        assert torch.allclose(d_b, acc_d, atol=1e-5) and torch.allclose(w_b, acc_w, atol=1e-5)
        h = P // 2
        d1, _ = bp(proj[b:b + 1, :h], rotations=rot1[:, :h], interpolation=interp)
        d2, _ = bp(proj[b:b + 1, h:], rotations=rot1[:, h:], interpolation=interp)
        assert torch.allclose(d1 + d2, d_b, atol=1e-5)
    sh = torch.randn(1, P, 2, generator=torch.Generator().manual_seed(14)).to(dev) * 2
    a, _ = bp(proj, rotations=rot1, shifts=sh, interpolation=interp)
    e, _ = bp(proj, rotations=rot1.expand(B, P, dim, dim).contiguous(), shifts=sh.expand(B, P, 2).contiguous(),
              interpolation=interp)
    assert torch.allclose(a, e, atol=1e-5)


# ----------------------------------------------------------------------------- oversampling
def quarter_turn(dim, dev):
    if dim == 2:
        R = [[0.0, -1.0], [1.0, 0.0]]
    else:
        R = [[0.0, 0.0, 1.0], [0.0, 1.0, 0.0], [-1.0, 0.0, 0.0]]
    return torch.tensor(R, device=dev)[None, None]


def oversampling_projection(api, dev, dim, interp, os_, B):
    """Reference: tests/2d/forw/test_oversampling.py:17-100,
    tests/3d/forw/test_oversampling_3d_to_2d.py:17-94: noise images padded
    with pad_and_fftshift(os) and rfftn(norm="forward"), projected at a
    quarter turn with oversampling os, against the unpadded spectrum at
    oversampling 1.  The reference asks for real-space NCC > 0.99 (2D) and
    allclose(atol 0.1) (3D, where every value is far below 0.1); both are
    checked here, with the stronger rel-L2 < 1e-4 of the two after scaling by
    os^dim, away from the output's Nyquist row and column: a sample at
    -n/2 along a volume row or depth axis is clamped to -n/2 + 1, as in the
    reference (csrc/cpu/common/interpolation_kernels.h:331-340), which is a
    different frequency in the two boxes."""
    n = 32
    g = torch.Generator().manual_seed(5)
    real = torch.randn((B,) + (n,) * dim, generator=g).to(dev)
    axes = tuple(range(-dim, 0))
    fp = torch.fft.rfftn(api.pad_and_fftshift(real, os_), dim=axes, norm="forward")
    fo = torch.fft.rfftn(api.pad_and_fftshift(real, 1.0), dim=axes, norm="forward")
    if dim == 3:
        fp[0, 0, 0, 0] = 0
        fo[0, 0, 0, 0] = 0
    rot, sh = quarter_turn(dim, dev), torch.zeros(1, 1, 2, device=dev)
    f = forw(api, dim)
    pp = f(fp, rot, shifts=sh, output_shape=(n, n), interpolation=interp, oversampling=os_)
    po = f(fo, rot, shifts=sh, output_shape=(n, n), interpolation=interp, oversampling=1.0)
    for b in range(B):
        score = ncc(torch.fft.irfft2(po[b]), torch.fft.irfft2(pp[b]))
        assert score > 0.99, (b, score.item())
    assert torch.allclose(po, pp, rtol=1e-5, atol=1e-1)
    rows = torch.cat([torch.arange(0, n // 2), torch.arange(n // 2 + 1, n)]).to(dev)
    inner_o, inner_p = po[:, :, rows, :n // 2], pp[:, :, rows, :n // 2] * os_ ** dim
    rel = ((inner_p - inner_o).abs().norm() / inner_o.abs().norm()).item()
    assert rel < 1e-4, rel


def oversampling_backprojection(api, dev, dim, interp, os_, B):
    """Reference: tests/2d/back/test_oversampling_back.py:17-97,
    tests/3d/back/test_oversampling_back_2d_to_3d.py:17-111: noise
    projections backprojected (quarter turn in 2D, identity in 3D, one random
    shift) at oversampling 1 and os, each taken to real space with irfftn and
    ifftshift_and_crop(os): NCC > 0.99 (2D), > 0.9 (3D)."""
    n = 32
    g = torch.Generator().manual_seed(6)
    proj = crandn((B, 1, n, n // 2 + 1), torch.complex64, 6, dev)
    rot = quarter_turn(2, dev) if dim == 2 else torch.eye(3, device=dev)[None, None]
    sh = ((torch.rand(1, 1, 2, generator=g) - 0.5) * (10 if dim == 2 else 5)).to(dev)
    bp = backproj(api, dim)
    d1, _ = bp(proj, rot, shifts=sh, interpolation=interp, oversampling=1.0)
    dn, _ = bp(proj, rot, shifts=sh, interpolation=interp, oversampling=os_)
    axes = tuple(range(-dim, 0))
    scores = []
    for b in range(B):
        r1 = api.ifftshift_and_crop(torch.fft.irfftn(d1[b], dim=axes), 1.0)
        rn = api.ifftshift_and_crop(torch.fft.irfftn(dn[b], dim=axes), os_)
        assert r1.shape == rn.shape
        scores.append(ncc(r1, rn).item())
    assert sum(scores) / B > (0.99 if dim == 2 else 0.9), scores


def oversampling_weights(api, dev, dim, os_=2.0):
    """Reference: tests/2d/back/test_oversampling_back.py:100-157,
    tests/3d/back/test_oversampling_back_2d_to_3d.py:114-176: three identity
    poses with weights, oversampling 1 against 2; data and weight
    reconstructions in real space, NCC > 0.99 each."""
    n = 16
    shape = (1, 3, n, n // 2 + 1)
    proj = crandn(shape, torch.complex64, 42, dev)
    w = rrand(shape, torch.float32, 43, dev)
    rot = torch.eye(dim, device=dev)[None, None].expand(1, 3, dim, dim)
    bp = backproj(api, dim)
    d1, w1 = bp(proj, rot, weights=w, oversampling=1.0)
    dn, wn = bp(proj, rot, weights=w, oversampling=os_)
    axes = tuple(range(-dim, 0))

    def real(x, o):
        x = x if x.is_complex() else torch.complex(x, torch.zeros_like(x))
        return api.ifftshift_and_crop(torch.fft.irfftn(x, dim=axes), o)

    assert ncc(real(d1[0], 1.0), real(dn[0], os_)) > 0.99
    assert ncc(real(w1[0], 1.0), real(wn[0], os_)) > 0.99
