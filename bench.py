"""Benchmark of the MI355X projector operators on one GPU.

Default workload (the headline of the metric): one step = a 3D linear
central-slice projection `project_3d_to_2d_forw` of a 2x-oversampled
512x512x257 complex64 volume onto 2048 poses (256x129 rfft projections),
followed by the weighted backprojection `backproject_2d_to_3d_forw` of those
2048 projections into a 512x512x257 data volume and its float32 weight volume.

Prints ONE JSON line: whole-step Fourier samples/s (samples = B*P*n*(n/2+1)
per op) over the K timed steps, the median step beside the mean, per-op
rates, the HBM roofline of the dominant op (algorithmic bytes per call / its
mean duration, measured with HIP events on the stream the kernels run on),
and the reference CPU path timed on a bounded sample of the same inputs on
the host cores.

Three fractions of the 8 TB/s peak are reported per op, and they mean
different things:
  alg_frac         algorithmic (per-tap, "effective") bytes / time: the
                   reference's memory traffic if every tap went to memory;
                   above 1 is possible for kernels that stage taps in LDS
  compulsory_frac  each input read once and each output written once / time
  traffic_frac     HBM bytes the rocprofv3 counters measured per call (the
                   committed profiles/hbm_traffic_<config>.md, stamped with
                   the commit it was measured at) / time

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config NAME] [--no-cpu]
Configs: headline (default, the bench line), c1..c5 (the other BASELINE.json configurations),
scaled / scaled06 / scaled14 (the headline with every pose matrix scaled by 1.02, 0.6, 1.4),
published (the reference's published H100 rows: box 256, oversampling 1), prep, half.
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "torch-projectors_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
METRIC = "Fourier samples/s + % HBM peak, 3D proj+backproj, 256 box 2x oversampled"


# ----------------------------------------------------------------------------- synthetic inputs
def quat_rotations(P, gen):
    """Uniform random rotations (normalised Gaussian quaternions) as 3x3, float32."""
    import torch
    q = torch.randn(P, 4, generator=gen, dtype=torch.float64)
    q = q / q.norm(dim=1, keepdim=True)
    w, x, y, z = q.unbind(1)
    R = torch.stack([1 - 2 * (y * y + z * z), 2 * (x * y - z * w), 2 * (x * z + y * w),
                     2 * (x * y + z * w), 1 - 2 * (x * x + z * z), 2 * (y * z - x * w),
                     2 * (x * z - y * w), 2 * (y * z + x * w), 1 - 2 * (x * x + y * y)], 1)
    return R.reshape(P, 3, 3).float()


def angle_rotations(shape, gen):
    import torch
    a = torch.rand(*shape, generator=gen, dtype=torch.float64) * 2 * math.pi
    c, s = torch.cos(a), torch.sin(a)
    return torch.stack([c, -s, s, c], -1).reshape(*shape, 2, 2).float()


def blob_volume_rfft(size, pad, n_blobs, radius, gen, dev):
    """Sum of Gaussian blobs on a size^3 grid, zero-padded to pad^3, fftshifted
    and rfft'd with norm='forward' (the reference's pad_and_fftshift recipe,
    tests/test_utils.py:174-247) -> [1, pad, pad, pad//2+1] complex64."""
    import torch
    u = torch.rand(n_blobs, generator=gen, dtype=torch.float64)
    d = torch.randn(n_blobs, 3, generator=gen, dtype=torch.float64)
    d = d / d.norm(dim=1, keepdim=True)
    mu = size / 2 + radius * u.pow(1 / 3)[:, None] * d
    sigma = 2 + 4 * torch.rand(n_blobs, generator=gen, dtype=torch.float64)
    amp = 0.5 + 0.5 * torch.rand(n_blobs, generator=gen, dtype=torch.float64)
    ax = torch.arange(size, device=dev, dtype=torch.float32)
    vol = torch.zeros(size, size, size, device=dev, dtype=torch.float32)
    for k in range(n_blobs):
        g = [torch.exp(-(ax - float(mu[k, a])) ** 2 / (2 * float(sigma[k]) ** 2)) for a in range(3)]
        vol += float(amp[k]) * g[0][:, None, None] * g[1][None, :, None] * g[2][None, None, :]
    lo = (pad - size) // 2
    padded = torch.nn.functional.pad(vol, (lo, pad - size - lo) * 3)
    spec = torch.fft.rfftn(torch.fft.fftshift(padded), norm="forward")
    del vol, padded
    return spec.to(torch.complex64).unsqueeze(0).contiguous()


def noise_image_rfft(B, size, pad, gen, dev):
    import torch
    img = torch.randn(B, size, size, generator=gen).to(dev)
    lo = (pad - size) // 2
    padded = torch.nn.functional.pad(img, (lo, pad - size - lo) * 2)
    return torch.fft.rfftn(torch.fft.fftshift(padded, dim=(-2, -1)), dim=(-2, -1), norm="forward").contiguous()


def ctf2_weights(B, P, n, gen):
    """sin^2(k*rho^2), rho = |frequency| / n in cycles/pixel, k ~ U(50, 200) per projection."""
    import torch
    i = torch.arange(n, dtype=torch.float64)
    r = torch.where(i <= n // 2, i, i - n)
    c = torch.arange(n // 2 + 1, dtype=torch.float64)
    rho2 = (r[:, None] ** 2 + c[None, :] ** 2) / float(n * n)
    k = 50 + 150 * torch.rand(B, P, 1, 1, generator=gen, dtype=torch.float64)
    return torch.sin(k * rho2) ** 2


# ----------------------------------------------------------------------------- Euler poses
def euler_rotations(B, P, gen):
    """Rz @ Ry @ Rx of three angles ~ U(0, 2 pi) per pose, float32 [B, P, 3, 3]: the poses of the
    reference's benchmarks (paper/results/benchmarks/benchmark_base.py:190-227)."""
    import torch
    ax, ay, az = (torch.rand(B, P, generator=gen, dtype=torch.float64) * 2 * math.pi for _ in range(3))
    z, o = torch.zeros_like(ax), torch.ones_like(ax)

    def m(rows):
        return torch.stack([torch.stack(r, -1) for r in rows], -2)

    Rx = m([[o, z, z], [z, ax.cos(), -ax.sin()], [z, ax.sin(), ax.cos()]])
    Ry = m([[ay.cos(), z, ay.sin()], [z, o, z], [-ay.sin(), z, ay.cos()]])
    Rz = m([[az.cos(), -az.sin(), z], [az.sin(), az.cos(), z], [z, z, o]])
    return (Rz @ Ry @ Rx).float()


# ----------------------------------------------------------------------------- byte model
def active_counts(n, cutoff=None):
    """(total, active forward, active scatter) pixels of one n x (n/2+1) projection
    (projection_utils.h:61-76; scatters also skip j == 0, i >= n/2)."""
    radius = cutoff if cutoff is not None else n / 2.0
    r2 = float(radius) ** 2
    total = fwd = bwd = 0
    for i in range(n):
        r = i if i <= n // 2 else i - n
        for j in range(n // 2 + 1):
            total += 1
            if r * r + j * j > r2:
                continue
            fwd += 1
            if not (j == 0 and i >= n // 2):
                bwd += 1
    return total, fwd, bwd


def taps(dim, interp):
    return (4 if interp == "linear" else 16) if dim == 2 else (8 if interp == "linear" else 64)


def bytes_forward(npose, n, dim, interp, cutoff=None):
    total, fwd, _ = active_counts(n, cutoff)
    return npose * (fwd * (taps(dim, interp) * 8 + 8) + (total - fwd) * 8)


def bytes_backproject(npose, n, dim, interp, vol_elems, weights, cutoff=None):
    _, _, bwd = active_counts(n, cutoff)
    per = 8 + (4 if weights else 0)
    return npose * bwd * per * (1 + taps(dim, interp)) + vol_elems * per


def bytes_project_back(npose, n, dim, interp, vol_elems, cutoff=None):
    _, _, bwd = active_counts(n, cutoff)
    t = taps(dim, interp)
    return npose * bwd * (8 + t * 8 + t * 8) + vol_elems * 8


def bytes_backproject_back(npose, n, dim, interp, weights, cutoff=None):
    _, _, bwd = active_counts(n, cutoff)
    lin = taps(dim, "linear")
    return npose * bwd * (taps(dim, interp) * 8 + 16 + ((4 * lin + 4) if weights else 0))


# Compulsory traffic: every input read once, every output written once (complex 8 B, real 4 B
# per element; poses are negligible).  `proj` = B*P*n*(n/2+1) projection elements, `vol` = the
# reconstruction's elements.
def compulsory_forward(proj, vol):
    return vol * 8 + proj * 8


def compulsory_backproject(proj, vol, weights):
    per = 8 + (4 if weights else 0)
    return proj * per + vol * per


def compulsory_project_back(proj, vol):
    # grad_projections and the volume read, the volume gradient written
    return proj * 8 + vol * 8 + vol * 8


def compulsory_backproject_back(proj, vol, weights):
    # grad_data_rec (+ grad_weight_rec) and the projections read; grad_projections (+ grad_weights) written
    return vol * (8 + (4 if weights else 0)) + proj * 8 + proj * (8 + (4 if weights else 0))


# ----------------------------------------------------------------------------- workloads
def timed_ops(calls, samples_per_op):
    """Run CPU calls in order, one run each; returns (seconds, samples, per-op seconds)."""
    import torch
    torch.cuda.synchronize()
    parts = {}
    total = 0.0
    for name, fn in calls:
        t0 = time.perf_counter()
        fn()
        parts[name] = time.perf_counter() - t0
        total += parts[name]
    return total, samples_per_op * len(calls), parts


class Workload:
    """Inputs on the GPU, a step as a list of ops: (name, callable, algorithmic bytes, samples, poses,
    compulsory bytes); `published` maps an op name to the reference's published rate for the same
    configuration on other hardware (proj/s, hardware, source)."""

    def __init__(self, name, desc, ops, cpu_sample=None, config=None, cpu_pmax=None, cpu_kind=None, cpu_cores=None,
                 published=None):
        self.name, self.desc, self.ops, self.cpu_sample, self.config = name, desc, ops, cpu_sample, config or {}
        self.cpu_pmax = cpu_pmax or ops[0][4]  # poses the CPU sample may take (one batch item's)
        # the CPU leg runs the reference build (or the oracle when absent) on `threads` cores,
        # unless the workload times its own port (numpy: one core)
        self.cpu_kind, self.cpu_cores = cpu_kind, cpu_cores
        self.published = published or {}


def make_headline(dev, scale=None):
    """The headline step; `scale` multiplies every pose matrix (the `scaled` workload: matrices that
    are not rotations, such as magnification-corrected poses, through the same step)."""
    import torch
    import torch_projectors as tp
    gen = torch.Generator().manual_seed(20261201 + 6)
    P, n, os_ = 2048, 256, 2.0
    vol = blob_volume_rfft(256, 512, 32, 80.0, gen, dev)
    rot = quat_rotations(P, gen)[None]
    if scale is not None:
        rot = (rot.double() * scale).float()
    rot = rot.to(dev)
    sh = ((torch.rand(1, P, 2, generator=gen) * 16) - 8).to(dev)
    w = ctf2_weights(1, P, n, gen).float().to(dev)
    state = {}

    def fwd():
        state["proj"] = tp.project_3d_to_2d_forw(vol, rot, sh, output_shape=(n, n), interpolation="linear",
                                                 oversampling=os_)

    def bp():
        state["bp"] = tp.backproject_2d_to_3d_forw(state["proj"], rot, weights=w, shifts=sh,
                                                   interpolation="linear", oversampling=os_)

    fwd()  # the backprojection's input, so that each op can also run alone (--ops)
    V = 512 * 512 * 257
    samples = P * n * (n // 2 + 1)
    ops = [("project_3d_to_2d_forw", fwd, bytes_forward(P, n, 3, "linear"), samples, P,
            compulsory_forward(samples, V)),
           ("backproject_2d_to_3d_forw", bp, bytes_backproject(P, n, 3, "linear", V, True), samples, P,
            compulsory_backproject(samples, V, True))]

    def cpu_sample(p_cpu, threads, cpu_ops):
        """Run the same two ops on the first p_cpu poses on the CPU; returns seconds and samples."""
        torch.cuda.synchronize()
        vc, rc, sc, wc = vol.cpu(), rot[:, :p_cpu].cpu(), sh[:, :p_cpu].cpu(), w[:, :p_cpu].cpu()
        pc = state["proj"][:, :p_cpu].cpu()
        t0 = time.perf_counter()
        cpu_ops.project_3d_to_2d_forw(vc, rc, sc, [n, n], "linear", os_, None)
        t1 = time.perf_counter()
        cpu_ops.backproject_2d_to_3d_forw(pc, wc, rc, sc, "linear", os_, None)
        t2 = time.perf_counter()
        return t2 - t0, 2 * p_cpu * n * (n // 2 + 1), {"project_3d_to_2d_forw": t1 - t0,
                                                       "backproject_2d_to_3d_forw": t2 - t1}

    cfg = {"workload": "headline: project_3d_to_2d_forw + backproject_2d_to_3d_forw (weights), linear",
           "volume": [1, 512, 512, 257], "poses": P, "proj": [n, n // 2 + 1], "oversampling": os_,
           "interpolation": "linear", "shifts": "U(-8,8)", "weights": "sin^2(k rho^2)"}
    name = "headline"
    if scale is not None:
        name = SCALED_NAMES[scale]
        cfg["workload"] = f"{name}: the headline step with every pose matrix scaled by {scale}"
        cfg["pose_scale"] = scale
    return Workload(name, cfg["workload"], ops, cpu_sample, cfg)


# the headline step with every pose matrix scaled: a magnification correction (x1.02) and strong
# shrinking / enlarging (x0.6, x1.4)
SCALED_NAMES = {1.02: "scaled", 0.6: "scaled06", 1.4: "scaled14"}


def make_scaled(dev):
    return make_headline(dev, scale=1.02)


def make_scaled06(dev):
    return make_headline(dev, scale=0.6)


def make_scaled14(dev):
    return make_headline(dev, scale=1.4)


def make_c1(dev):
    """c1: 2D linear forward of a 64^2 noise image padded to 128, 256 poses of 64 x 33 (BASELINE.json
    configs[0], the reference's CPU-runnable case; launch-bound on the GPU)."""
    import torch
    T = torch.ops.torch_projectors
    gen = torch.Generator().manual_seed(20261201 + 1)
    P, n, os_ = 256, 64, 2.0
    rec = noise_image_rfft(1, 64, 128, gen, dev).to(torch.complex64)
    rot = angle_rotations((1, P), gen).to(dev)
    sh = (2 * torch.randn(1, P, 2, generator=gen)).to(dev)

    def fwd():
        T.project_2d_forw(rec, rot, sh, [n, n], "linear", os_, None)

    def cpu_sample(p, threads, cpu_ops):
        rc, r0, s0 = rec.cpu(), rot[:, :p].cpu(), sh[:, :p].cpu()
        return timed_ops([("project_2d_forw", lambda: cpu_ops.project_2d_forw(
            rc, r0, s0, [n, n], "linear", os_, None))], p * n * (n // 2 + 1))

    samples = P * n * (n // 2 + 1)
    cfg = {"workload": "c1: project_2d_forw, linear", "reconstruction": [1, 128, 65], "poses": P,
           "proj": [n, n // 2 + 1], "oversampling": os_, "shifts": "2 N(0,1)"}
    return Workload("c1", cfg["workload"], [("project_2d_forw", fwd, bytes_forward(P, n, 2, "linear"), samples, P,
                                             compulsory_forward(samples, 128 * 65))], cpu_sample, cfg)


def make_c2(dev):
    """c2: 3D linear forward, 256^3-padded blob volume, 4096 poses of 128 x 65."""
    import torch
    T = torch.ops.torch_projectors
    gen = torch.Generator().manual_seed(20261201 + 2)
    P, n, os_ = 4096, 128, 2.0
    vol = blob_volume_rfft(128, 256, 32, 40.0, gen, dev)
    rot = quat_rotations(P, gen)[None].to(dev)
    sh = ((torch.rand(1, P, 2, generator=gen) * 10) - 5).to(dev)

    def fwd():
        T.project_3d_to_2d_forw(vol, rot, sh, [n, n], "linear", os_, None)

    def cpu_sample(p, threads, cpu_ops):
        vc, rc, sc = vol.cpu(), rot[:, :p].cpu(), sh[:, :p].cpu()
        return timed_ops([("project_3d_to_2d_forw", lambda: cpu_ops.project_3d_to_2d_forw(
            vc, rc, sc, [n, n], "linear", os_, None))], p * n * (n // 2 + 1))

    samples = P * n * (n // 2 + 1)
    cfg = {"workload": "c2: project_3d_to_2d_forw, linear", "volume": [1, 256, 256, 129], "poses": P,
           "proj": [n, n // 2 + 1], "oversampling": os_}
    return Workload("c2", cfg["workload"], [("project_3d_to_2d_forw", fwd, bytes_forward(P, n, 3, "linear"),
                                             samples, P, compulsory_forward(samples, 256 * 256 * 129))],
                    cpu_sample, cfg)


def make_c3(dev):
    """c3: 3D linear backprojection with weights, 8192 poses of 128 x 65 into 256^3."""
    import torch
    T = torch.ops.torch_projectors
    gen = torch.Generator().manual_seed(20261201 + 3)
    P, n, os_ = 8192, 128, 2.0
    proj = torch.randn(1, P, n, n // 2 + 1, generator=gen, dtype=torch.complex64).to(dev)
    w = ctf2_weights(1, P, n, gen).float().to(dev)
    rot = quat_rotations(P, gen)[None].to(dev)
    sh = ((torch.rand(1, P, 2, generator=gen) * 10) - 5).to(dev)

    def bp():
        T.backproject_2d_to_3d_forw(proj, w, rot, sh, "linear", os_, None)

    def cpu_sample(p, threads, cpu_ops):
        pc, wc, rc, sc = proj[:, :p].cpu(), w[:, :p].cpu(), rot[:, :p].cpu(), sh[:, :p].cpu()
        return timed_ops([("backproject_2d_to_3d_forw", lambda: cpu_ops.backproject_2d_to_3d_forw(
            pc, wc, rc, sc, "linear", os_, None))], p * n * (n // 2 + 1))

    samples = P * n * (n // 2 + 1)
    cfg = {"workload": "c3: backproject_2d_to_3d_forw (weights), linear", "volume": [1, 256, 256, 129],
           "poses": P, "proj": [n, n // 2 + 1], "oversampling": os_}
    return Workload("c3", cfg["workload"],
                    [("backproject_2d_to_3d_forw", bp, bytes_backproject(P, n, 3, "linear", 256 * 256 * 129, True),
                      samples, P, compulsory_backproject(samples, 256 * 256 * 129, True))], cpu_sample, cfg)


def make_c4(dev):
    """c4: 3D cubic forward and its backward (volume, rotation and shift gradients)."""
    import torch
    T = torch.ops.torch_projectors
    gen = torch.Generator().manual_seed(20261201 + 4)
    P, n, os_ = 2048, 256, 2.0
    vol = blob_volume_rfft(256, 512, 32, 80.0, gen, dev)
    rot = quat_rotations(P, gen)[None].to(dev).requires_grad_(True)
    sh = ((torch.rand(1, P, 2, generator=gen) * 16) - 8).to(dev).requires_grad_(True)
    g = torch.randn(1, P, n, n // 2 + 1, generator=gen, dtype=torch.complex64).to(dev)

    def fwd():
        T.project_3d_to_2d_forw(vol, rot.detach(), sh.detach(), [n, n], "cubic", os_, None)

    def back():
        T.project_3d_to_2d_back(g, vol, rot, sh, "cubic", os_, None)

    def cpu_sample(p, threads, cpu_ops):
        vc, gc = vol.cpu(), g[:, :p].cpu()
        rc = rot[:, :p].detach().cpu().requires_grad_(True)
        sc = sh[:, :p].detach().cpu().requires_grad_(True)
        return timed_ops([("project_3d_to_2d_forw", lambda: cpu_ops.project_3d_to_2d_forw(
                              vc, rc.detach(), sc.detach(), [n, n], "cubic", os_, None)),
                          ("project_3d_to_2d_back", lambda: cpu_ops.project_3d_to_2d_back(
                              gc, vc, rc, sc, "cubic", os_, None))], p * n * (n // 2 + 1))

    V = 512 * 512 * 257
    samples = P * n * (n // 2 + 1)
    cfg = {"workload": "c4: project_3d_to_2d_forw + project_3d_to_2d_back (rotation/shift grads), cubic",
           "volume": [1, 512, 512, 257], "poses": P, "proj": [n, n // 2 + 1], "oversampling": os_}
    return Workload("c4", cfg["workload"],
                    [("project_3d_to_2d_forw", fwd, bytes_forward(P, n, 3, "cubic"), samples, P,
                      compulsory_forward(samples, V)),
                     ("project_3d_to_2d_back", back, bytes_project_back(P, n, 3, "cubic", V), samples, P,
                      compulsory_project_back(samples, V))],
                    cpu_sample, cfg)


def make_c5(dev):
    """c5: batched 2D cubic, 16 images x 4096 poses: forward, backprojection and both backward ops."""
    import torch
    T = torch.ops.torch_projectors
    gen = torch.Generator().manual_seed(20261201 + 5)
    B, P, n, os_, cut = 16, 4096, 256, 2.0, 64.0
    rec = noise_image_rfft(B, 256, 512, gen, dev).to(torch.complex64)
    rot = angle_rotations((B, P), gen).to(dev)
    sh = (3 * torch.randn(B, P, 2, generator=gen)).to(dev)
    rot_g, sh_g = rot.clone().requires_grad_(True), sh.clone().requires_grad_(True)
    st = {"proj": T.project_2d_forw(rec, rot, sh, [n, n], "cubic", os_, cut)}
    ones = torch.ones(B, P, n, n // 2 + 1, device=dev)
    gd = torch.randn(B, 512, 257, generator=gen, dtype=torch.complex64).to(dev)
    gw = torch.randn(B, 512, 257, generator=gen).to(dev)

    def fwd():
        st["proj"] = T.project_2d_forw(rec, rot, sh, [n, n], "cubic", os_, cut)

    def bp():
        T.backproject_2d_forw(st["proj"], ones, rot, sh, "cubic", os_, cut)

    def bp_back():
        st["gproj"] = T.backproject_2d_back(gd, gw, st["proj"], ones, rot_g, sh_g, "cubic", os_, cut)[0]

    def p_back():
        T.project_2d_back(st["gproj"], rec, rot_g, sh_g, "cubic", os_, cut)

    bp_back()  # project_2d_back's input, so that each op can also run alone (--ops)

    def cpu_sample(p, threads, cpu_ops):
        """Item 0's first p poses through the four ops."""
        if "gproj" not in st:
            bp_back()
        rc0, r0, s0 = rec[:1].cpu(), rot[:1, :p].cpu(), sh[:1, :p].cpu()
        rg0, sg0 = r0.clone().requires_grad_(True), s0.clone().requires_grad_(True)
        pr0, gp0, on0 = st["proj"][:1, :p].cpu(), st["gproj"][:1, :p].cpu(), ones[:1, :p].cpu()
        gd0, gw0 = gd[:1].cpu(), gw[:1].cpu()
        return timed_ops([("project_2d_forw", lambda: cpu_ops.project_2d_forw(rc0, r0, s0, [n, n], "cubic", os_, cut)),
                          ("backproject_2d_forw", lambda: cpu_ops.backproject_2d_forw(
                              pr0, on0, r0, s0, "cubic", os_, cut)),
                          ("backproject_2d_back", lambda: cpu_ops.backproject_2d_back(
                              gd0, gw0, pr0, on0, rg0, sg0, "cubic", os_, cut)),
                          ("project_2d_back", lambda: cpu_ops.project_2d_back(gp0, rc0, rg0, sg0, "cubic", os_, cut))],
                         p * n * (n // 2 + 1))

    samples = B * P * n * (n // 2 + 1)
    V = B * 512 * 257
    cfg = {"workload": "c5: batched 2D cubic forward, backprojection (unit weights), both backward ops",
           "reconstruction": [B, 512, 257], "poses": P, "proj": [n, n // 2 + 1], "oversampling": os_, "cutoff": cut}
    return Workload("c5", cfg["workload"],
                    [("project_2d_forw", fwd, bytes_forward(B * P, n, 2, "cubic", cut), samples, B * P,
                      compulsory_forward(samples, V)),
                     ("backproject_2d_forw", bp, bytes_backproject(B * P, n, 2, "cubic", V, True, cut), samples,
                      B * P, compulsory_backproject(samples, V, True)),
                     ("backproject_2d_back", bp_back, bytes_backproject_back(B * P, n, 2, "cubic", True, cut),
                      samples, B * P, compulsory_backproject_back(samples, V, True)),
                     ("project_2d_back", p_back, bytes_project_back(B * P, n, 2, "cubic", V, cut), samples,
                      B * P, compulsory_project_back(samples, V))], cpu_sample, cfg, cpu_pmax=P)


def make_prep(dev):
    """prep: the reference preparation around the headline volume, both ways.

    to_fourier: 256^3 real blob volume -> pad_and_fftshift (512^3) -> rfftn ->
    [512, 512, 257] row-major; reconstruct: a (data, weight) pair of that shape
    -> normalize_reconstruction -> irfftn -> ifftshift_and_crop -> 256^3.  The
    pad, crop and normalisation are this library's kernels; the FFTs are rocFFT
    (through torch.fft).
    """
    import torch
    from torch_projectors import fourier as F
    gen = torch.Generator().manual_seed(20261201 + 7)
    n, os_ = 256, 2.0
    N = 512
    real = torch.fft.irfftn(blob_volume_rfft(n, N, 32, 80.0, gen, dev), s=(N, N, N), norm="forward")
    vol = F.ifftshift_and_crop(real, os_)[0].contiguous()  # [n, n, n]
    w = torch.rand(N, N, N // 2 + 1, generator=gen).to(dev) + 0.5
    st = {}

    def fwd():
        st["spec"] = F.to_fourier(vol, os_)

    def back():
        st["out"] = F.reconstruct(st["spec"], w, os_, 0.01)

    V = N * N * (N // 2 + 1)

    def cpu_sample(p, threads, cpu_ops):
        """The oracle's numpy restatement with numpy's FFT (one core)."""
        import numpy as np
        from oracle import fourier as OF
        vc, wc = vol.cpu().numpy(), w.cpu().numpy()
        t0 = time.perf_counter()
        spec = np.fft.rfftn(OF.pad_and_fftshift(vc, os_), axes=(0, 1, 2), norm="forward").astype(np.complex64)
        t1 = time.perf_counter()
        normed = OF.normalize_reconstruction(spec, wc, 0.01)
        back_ = np.fft.irfftn(normed, s=(N, N, N), axes=(0, 1, 2), norm="forward").astype(np.float32)
        OF.ifftshift_and_crop(back_, os_)
        t2 = time.perf_counter()
        return t2 - t0, 2 * V, {"to_fourier": t1 - t0, "reconstruct": t2 - t1}

    cfg = {"workload": "prep: to_fourier (pad_and_fftshift + rfftn) and reconstruct (normalize + irfftn + "
                       "ifftshift_and_crop)", "real_volume": [n, n, n], "padded": [N, N, N],
           "spectrum": [N, N, N // 2 + 1], "oversampling": os_}
    # minimal bytes: read the input and write the output once
    return Workload("prep", cfg["workload"],
                    [("to_fourier", fwd, n ** 3 * 4 + V * 8, V, 0, n ** 3 * 4 + V * 8),
                     ("reconstruct", back, V * (8 + 4) + n ** 3 * 4, V, 0, V * (8 + 4) + n ** 3 * 4)],
                    cpu_sample, cfg, cpu_pmax=1, cpu_kind="port", cpu_cores=1)


def make_half(dev):
    """half: the headline forward from the same volume stored as complex32 (the
    opt-in low-precision storage), beside the complex64 forward, linear and cubic."""
    import torch
    import torch_projectors as tp
    gen = torch.Generator().manual_seed(20261201 + 6)
    P, n, os_ = 2048, 256, 2.0
    vol = blob_volume_rfft(256, 512, 32, 80.0, gen, dev)
    rot = quat_rotations(P, gen)[None].to(dev)
    sh = ((torch.rand(1, P, 2, generator=gen) * 16) - 8).to(dev)
    vol16 = vol.to(torch.complex32)

    def fwd(v, interp):
        return lambda: tp.project_3d_to_2d_forw(v, rot, sh, output_shape=(n, n), interpolation=interp,
                                                oversampling=os_)

    samples = P * n * (n // 2 + 1)
    ops = []
    for interp in ("linear", "cubic"):
        for tag, v in (("complex32", vol16), ("complex64", vol)):
            ops.append((f"project_3d_to_2d_forw[{interp},{tag}]", fwd(v, interp),
                        bytes_forward(P, n, 3, interp), samples, P,
                        512 * 512 * 257 * (4 if tag == "complex32" else 8) + samples * 8))

    def cpu_sample(p_cpu, threads, cpu_ops):
        """The CPU reference on the widened volume (the storage's definition), linear."""
        vc, rc, sc = vol16.to(torch.complex64).cpu(), rot[:, :p_cpu].cpu(), sh[:, :p_cpu].cpu()
        return timed_ops([("project_3d_to_2d_forw[linear,complex32]", lambda: cpu_ops.project_3d_to_2d_forw(
            vc, rc, sc, [n, n], "linear", os_, None))], p_cpu * n * (n // 2 + 1))

    cfg = {"workload": "half: headline forward from a complex32 volume beside complex64, linear and cubic",
           "volume": [1, 512, 512, 257], "poses": P, "proj": [n, n // 2 + 1], "oversampling": os_}
    return Workload("half", cfg["workload"], ops, cpu_sample, cfg)


def make_published(dev):
    """published: the reference's published H100 rows at box 256 (volume 256^3, projections
    256 x 129, oversampling 1, the default of its benchmark scripts), P = 2048 per batch item, batch
    1 and 8, linear and cubic: forward projection, and backprojection with weights (forward op
    only).  Inputs follow its benchmark scripts (paper/results/benchmarks/forward_3d_to_2d.py,
    backward_2d_to_3d.py, benchmark_base.py:150-227): complex N(0,1) volumes and projections,
    U(0,1) weights, Euler-angle rotations, shifts 5 N(0,1)."""
    import torch
    T = torch.ops.torch_projectors
    gen = torch.Generator().manual_seed(20261201 + 8)
    n, P = 256, 2048
    V = n * n * (n // 2 + 1)
    st = {}
    for B in (1, 8):
        st[B] = dict(vol=torch.randn(B, n, n, n // 2 + 1, generator=gen, dtype=torch.complex64).to(dev),
                     rot=euler_rotations(B, P, gen).to(dev),
                     sh=(5 * torch.randn(B, P, 2, generator=gen)).to(dev),
                     proj=torch.randn(B, P, n, n // 2 + 1, generator=gen, dtype=torch.complex64).to(dev),
                     w=torch.rand(B, P, n, n // 2 + 1, generator=gen).to(dev))

    def fwd(B, interp):
        d = st[B]
        return lambda: T.project_3d_to_2d_forw(d["vol"], d["rot"], d["sh"], [n, n], interp, 1.0, None)

    def bp(B, interp):
        d = st[B]
        return lambda: T.backproject_2d_to_3d_forw(d["proj"], d["w"], d["rot"], d["sh"], interp, 1.0, None)

    # H100 proj/s (batch x poses per second), paper/results/tables/*.tex rows at box 256, 2048 poses
    h100 = {("f", 1, "linear"): (929.5e3, "project-3d-to-2d-performance.tex:54"),
            ("f", 1, "cubic"): (164.6e3, "project-3d-to-2d-performance.tex:55"),
            ("f", 8, "linear"): (1838.2e3, "project-3d-to-2d-performance.tex:64"),
            ("f", 8, "cubic"): (253.8e3, "project-3d-to-2d-performance.tex:65"),
            ("b", 1, "linear"): (135.8e3, "backproject-2d-to-3d-performance.tex:54"),
            ("b", 1, "cubic"): (18.5e3, "backproject-2d-to-3d-performance.tex:55"),
            ("b", 8, "linear"): (134.0e3, "backproject-2d-to-3d-performance.tex:64"),
            ("b", 8, "cubic"): (18.7e3, "backproject-2d-to-3d-performance.tex:65")}
    ops, published = [], {}
    for kind in ("f", "b"):
        for B in (1, 8):
            for interp in ("linear", "cubic"):
                samples = B * P * n * (n // 2 + 1)
                if kind == "f":
                    name = f"project_3d_to_2d_forw[{interp},B{B}]"
                    ops.append((name, fwd(B, interp), bytes_forward(B * P, n, 3, interp), samples, B * P,
                                compulsory_forward(samples, B * V)))
                else:
                    name = f"backproject_2d_to_3d_forw[{interp},B{B}]"
                    ops.append((name, bp(B, interp), bytes_backproject(B * P, n, 3, interp, B * V, True), samples,
                                B * P, compulsory_backproject(samples, B * V, True)))
                rate, src = h100[(kind, B, interp)]
                published[name] = {"proj_per_s": rate, "hardware": "H100 (CUDA)", "source": src}

    def cpu_sample(p, threads, cpu_ops):
        """Batch item 0's first p poses through the linear forward and backprojection."""
        d = st[1]
        vc, rc, sc = d["vol"].cpu(), d["rot"][:, :p].cpu(), d["sh"][:, :p].cpu()
        pc, wc = d["proj"][:, :p].cpu(), d["w"][:, :p].cpu()
        return timed_ops([("project_3d_to_2d_forw[linear,B1]", lambda: cpu_ops.project_3d_to_2d_forw(
                              vc, rc, sc, [n, n], "linear", 1.0, None)),
                          ("backproject_2d_to_3d_forw[linear,B1]", lambda: cpu_ops.backproject_2d_to_3d_forw(
                              pc, wc, rc, sc, "linear", 1.0, None))], p * n * (n // 2 + 1))

    cfg = {"workload": "published: box 256 (volume 256^3, projections 256 x 129), oversampling 1, 2048 poses per "
                       "item, batch 1 and 8, linear and cubic; forward and weighted backprojection",
           "volume": ["B", 256, 256, 129], "poses": P, "proj": [n, n // 2 + 1], "oversampling": 1.0,
           "shifts": "5 N(0,1)", "weights": "U(0,1)", "rotations": "Euler angles ~ U(0, 2 pi)"}
    return Workload("published", cfg["workload"], ops, cpu_sample, cfg, cpu_pmax=P, published=published)


# headline is the bench line; c1-c5 are the other BASELINE configurations,
# prep the reference preparation around the headline volume, half the
# headline forward from low-precision storage, scaled / scaled06 / scaled14 the
# headline with pose matrices that are not rotations, published the
# reference's own published rows (box 256, oversampling 1), run on request
WORKLOADS = {"headline": make_headline, "c1": make_c1, "c2": make_c2, "c3": make_c3, "c4": make_c4, "c5": make_c5,
             "prep": make_prep, "half": make_half, "scaled": make_scaled, "scaled06": make_scaled06,
             "scaled14": make_scaled14, "published": make_published}


# ----------------------------------------------------------------------------- CPU baseline
def cpu_ops_and_kind():
    from oracle import oracle as O
    ref = O.ref_ops()
    if ref is not None:
        return ref, "reference"
    return O, "port"


def cpu_model():
    """The host CPU's model name (lscpu's "Model name", else /proc/cpuinfo)."""
    import subprocess
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_threads():
    """Threads for the CPU leg: every CPU of the process's affinity, capped by OMP_NUM_THREADS when
    the environment sets it (the GPU boxes set it to the CPU share of one GPU, 16, while their
    affinity lists every core of the host)."""
    affinity = len(os.sched_getaffinity(0))
    share = os.environ.get("OMP_NUM_THREADS", "")
    if share.isdigit() and int(share) > 0:
        return min(affinity, int(share)), affinity, f"OMP_NUM_THREADS={share} (CPU share of one GPU)"
    return affinity, affinity, "every CPU of the affinity mask"


def run_cpu_baseline(wl, one_run_s=2.5, runs=5):
    """Time the workload's ops on the host cores on its first p poses.

    p doubles (or scales by the measured rate) until one run takes about one_run_s or covers every
    pose of the workload; then one warm-up run and `runs` timed runs, of which the median is
    reported.
    """
    import statistics
    import torch
    threads, affinity, rule = cpu_threads()
    torch.set_num_threads(threads)
    ops, kind = cpu_ops_and_kind()
    p = min(8, wl.cpu_pmax)
    t, _, _ = wl.cpu_sample(p, threads, ops)
    while t < one_run_s and p < wl.cpu_pmax:
        p = int(min(wl.cpu_pmax, max(2 * p, p * 1.2 * one_run_s / max(t, 1e-3))))
        t, _, _ = wl.cpu_sample(p, threads, ops)
    wl.cpu_sample(p, threads, ops)  # warm-up at the final size
    res = [wl.cpu_sample(p, threads, ops) for _ in range(runs)]
    times = [r[0] for r in res]
    med = statistics.median(times)
    t, s, parts = min(res, key=lambda r: abs(r[0] - med))
    split = ", ".join(f"{k} {v:.2f} s" for k, v in parts.items())
    kind, threads = wl.cpu_kind or kind, wl.cpu_cores or threads
    return {"value": s / med, "unit": "Fourier samples/s", "cores": threads, "kind": kind,
            "poses_per_s": p / med, "ops_s": {k: round(v, 4) for k, v in parts.items()},
            "runs_s": [round(x, 4) for x in times], "cpu_model": cpu_model(), "affinity_cpus": affinity,
            "threads_rule": rule if not wl.cpu_cores else "the workload's own one-core port",
            "sample": f"first {p} poses of the workload (item 0), every op of the step, median of {runs} runs "
                      f"after 1 warm-up ({med:.2f} s; the median run: {split}), {threads} threads"}


# ----------------------------------------------------------------------------- HBM traffic
def measured_traffic(workload):
    """HBM bytes per call of each op, and the commit they were measured at, from the committed
    rocprofv3 FETCH_SIZE/WRITE_SIZE summary.

    The counters cannot be read from inside a run, so the figures come from the
    summary profiles/hbm_traffic_<workload>.md (copy-kernel-scaled, read + write,
    summed over the op's kernels, its `traffic_bytes_per_call:` line) and the
    commit from its `measured_at_commit:` line; ({}, None) when there is none.
    """
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", f"hbm_traffic_{workload}.md")
    per_op, commit = {}, None
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_call:"):
                    per_op = json.loads(line.split(":", 1)[1])
                elif line.startswith("measured_at_commit:"):
                    commit = line.split(":", 1)[1].strip()
    except OSError:
        pass
    return per_op, commit


# ----------------------------------------------------------------------------- main
def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", default="headline", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--ops", default=None,
                    help="comma-separated op names: run only these ops of the workload's step (per-op counter "
                         "runs); the JSON then describes that step")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run and time a plain 1 GiB copy kernel (calibrates HBM byte counters, measures the copy ceiling)")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (--gpus {a.gpus} requested); more GPUs would "
              "shard the poses and all-reduce the backprojected volumes once, which is not built here",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import torch_projectors  # noqa: F401  (registers torch.ops.torch_projectors; fails without the HIP library)
    dev = torch.device("cuda:0")
    if a.copy_probe:
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.mul(src, 1.0, out=dst)  # warm-up
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(5):  # an elementwise kernel (not a runtime blit) so counters see it
            torch.mul(src, 1.0, out=dst)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / 5
        moved = 2 * src.numel() * 4
        print(json.dumps({"copy_probe_bytes_read": src.numel() * 4, "copy_probe_bytes_written": dst.numel() * 4,
                          "calls": 6, "ms_per_copy": round(ms, 4), "copy_GBps": moved / (ms / 1e3) / 1e9,
                          "copy_frac_of_peak": moved / (ms / 1e3) / 1e9 / HBM_PEAK_GBS}))
        return
    wl = WORKLOADS[a.config](dev)
    if a.ops:
        keep = a.ops.split(",")
        unknown = [k for k in keep if k not in [op[0] for op in wl.ops]]
        if unknown:
            print(f"bench.py: unknown op(s) {unknown} for --config {a.config}", file=sys.stderr)
            sys.exit(2)
        wl.ops = [op for op in wl.ops if op[0] in keep]
    torch.cuda.synchronize()
    log(f"inputs ready: {a.config}")

    for _ in range(a.warmup):
        for _, fn, *_rest in wl.ops:
            fn()
    torch.cuda.synchronize()

    nops = len(wl.ops)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(nops + 1)] for _ in range(a.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(a.steps):
        ev[s][0].record()
        for k, (_, fn, *_rest) in enumerate(wl.ops):
            fn()
            ev[s][k + 1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    log(f"timed {a.steps} steps in {wall:.2f} s")
    import statistics
    op_runs = [[ev[s][k].elapsed_time(ev[s][k + 1]) for s in range(a.steps)] for k in range(nops)]
    step_runs = [ev[s][0].elapsed_time(ev[s][nops]) for s in range(a.steps)]
    op_ms = [sum(r) / a.steps for r in op_runs]
    ms_step = sum(step_runs) / a.steps

    traffic, traffic_commit = measured_traffic(a.config)
    frac = lambda nbytes, sec: nbytes / sec / 1e9 / HBM_PEAK_GBS  # noqa: E731
    samples_step = sum(op[3] for op in wl.ops)
    per_op = {}
    for k, (name, _, nbytes, samples, poses, comp) in enumerate(wl.ops):
        sec = op_ms[k] / 1e3
        o = {"ms": round(op_ms[k], 4), "ms_median": round(statistics.median(op_runs[k]), 4),
             "samples_per_s": samples / sec, "poses_per_s": poses / sec,
             "alg_GB": nbytes / 1e9, "alg_GBps": nbytes / sec / 1e9, "alg_frac": frac(nbytes, sec),
             "compulsory_GB": comp / 1e9, "compulsory_frac": frac(comp, sec)}
        if traffic.get(name) is not None:
            o["traffic_GB"] = traffic[name] / 1e9
            o["traffic_frac"] = frac(traffic[name], sec)
        if name in wl.published:
            pub = wl.published[name]
            o["published"] = pub
            o["vs_published"] = (poses / sec) / pub["proj_per_s"]
        per_op[name] = o
    dom = max(range(nops), key=lambda k: op_ms[k])
    dname, _, dbytes, _, _, dcomp = wl.ops[dom]
    dsec = op_ms[dom] / 1e3
    achieved = dbytes / dsec / 1e9
    total_bytes = sum(op[2] for op in wl.ops)
    total_comp = sum(op[5] for op in wl.ops)

    cpu = None
    if not a.no_cpu and wl.cpu_sample is not None:
        log("cpu baseline ...")
        cpu = run_cpu_baseline(wl)
        log(f"cpu baseline: {cpu['sample']}")

    dtraffic = traffic.get(dname)
    out = {
        "metric": METRIC,
        "value": samples_step / (ms_step / 1e3),
        "unit": "Fourier samples/s",
        "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms_step, 4),
        "ms_per_step_median": round(statistics.median(step_runs), 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": wl.config,
        "poses_per_s": wl.ops[0][4] / (ms_step / 1e3),
        "step_alg_GBps": total_bytes / (ms_step / 1e3) / 1e9,
        "step_alg_frac": frac(total_bytes, ms_step / 1e3),
        "step_compulsory_frac": frac(total_comp, ms_step / 1e3),
        "wall_s": round(wall, 3),
        "ops": per_op,
        "roofline": {"bound": "hbm", "kernel": dname, "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": dtraffic,
                     "traffic_frac": frac(dtraffic, dsec) if dtraffic is not None else None,
                     "traffic_commit": traffic_commit if dtraffic is not None else None,
                     "compulsory": dcomp, "compulsory_frac": frac(dcomp, dsec),
                     "achieved_is": "algorithmic (per-tap) bytes per call / mean call time"},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
