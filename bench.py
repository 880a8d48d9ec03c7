"""Benchmark of the MI355X projector operators on one GPU.

Default workload (the headline of the metric): one step = a 3D linear
central-slice projection `project_3d_to_2d_forw` of a 2x-oversampled
512x512x257 complex64 volume onto 2048 poses (256x129 rfft projections),
followed by the weighted backprojection `backproject_2d_to_3d_forw` of those
2048 projections into a 512x512x257 data volume and its float32 weight volume.

Prints ONE JSON line: whole-step Fourier samples/s (samples = B*P*n*(n/2+1)
per op), per-op rates, the HBM roofline of the dominant op (algorithmic
bytes per call / its mean duration, measured with HIP events on the stream
the kernels run on), and the reference CPU path timed on a bounded sample of
the same inputs on the host cores.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config NAME] [--no-cpu]
Configs: headline (default, the bench line), c2..c5 (the other BASELINE.json configurations:
per-op rates and the CPU baseline on a bounded sample; no traffic figure for them).
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
    """Inputs on the GPU, a step as a list of (op name, callable, bytes, samples)."""

    def __init__(self, name, desc, ops, cpu_sample=None, config=None, cpu_pmax=None, cpu_kind=None, cpu_cores=None):
        self.name, self.desc, self.ops, self.cpu_sample, self.config = name, desc, ops, cpu_sample, config or {}
        self.cpu_pmax = cpu_pmax or ops[0][4]  # poses the CPU sample may take (one batch item's)
        # the CPU leg runs the reference build (or the oracle when absent) on `threads` cores,
        # unless the workload times its own port (numpy: one core)
        self.cpu_kind, self.cpu_cores = cpu_kind, cpu_cores


def make_headline(dev, k=0):
    import torch
    import torch_projectors as tp
    gen = torch.Generator().manual_seed(20261201 + 6)
    P, n, os_ = 2048, 256, 2.0
    vol = blob_volume_rfft(256, 512, 32, 80.0, gen, dev)
    rot = quat_rotations(P, gen)[None].to(dev)
    sh = ((torch.rand(1, P, 2, generator=gen) * 16) - 8).to(dev)
    w = ctf2_weights(1, P, n, gen).float().to(dev)
    state = {}

    def fwd():
        state["proj"] = tp.project_3d_to_2d_forw(vol, rot, sh, output_shape=(n, n), interpolation="linear",
                                                 oversampling=os_)

    def bp():
        state["bp"] = tp.backproject_2d_to_3d_forw(state["proj"], rot, weights=w, shifts=sh,
                                                   interpolation="linear", oversampling=os_)

    V = 512 * 512 * 257
    samples = P * n * (n // 2 + 1)
    ops = [("project_3d_to_2d_forw", fwd, bytes_forward(P, n, 3, "linear"), samples, P),
           ("backproject_2d_to_3d_forw", bp, bytes_backproject(P, n, 3, "linear", V, True), samples, P)]

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
    return Workload("headline", cfg["workload"], ops, cpu_sample, cfg)


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
                                             samples, P)], cpu_sample, cfg)


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
                      samples, P)], cpu_sample, cfg)


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
                    [("project_3d_to_2d_forw", fwd, bytes_forward(P, n, 3, "cubic"), samples, P),
                     ("project_3d_to_2d_back", back, bytes_project_back(P, n, 3, "cubic", V), samples, P)],
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
                    [("project_2d_forw", fwd, bytes_forward(B * P, n, 2, "cubic", cut), samples, B * P),
                     ("backproject_2d_forw", bp, bytes_backproject(B * P, n, 2, "cubic", V, True, cut), samples,
                      B * P),
                     ("backproject_2d_back", bp_back, bytes_backproject_back(B * P, n, 2, "cubic", True, cut),
                      samples, B * P),
                     ("project_2d_back", p_back, bytes_project_back(B * P, n, 2, "cubic", V, cut), samples,
                      B * P)], cpu_sample, cfg, cpu_pmax=P)


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
                    [("to_fourier", fwd, n ** 3 * 4 + V * 8, V, 0),
                     ("reconstruct", back, V * (8 + 4) + n ** 3 * 4, V, 0)],
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
                        bytes_forward(P, n, 3, interp), samples, P))

    def cpu_sample(p_cpu, threads, cpu_ops):
        """The CPU reference on the widened volume (the storage's definition), linear."""
        vc, rc, sc = vol16.to(torch.complex64).cpu(), rot[:, :p_cpu].cpu(), sh[:, :p_cpu].cpu()
        return timed_ops([("project_3d_to_2d_forw[linear,complex32]", lambda: cpu_ops.project_3d_to_2d_forw(
            vc, rc, sc, [n, n], "linear", os_, None))], p_cpu * n * (n // 2 + 1))

    cfg = {"workload": "half: headline forward from a complex32 volume beside complex64, linear and cubic",
           "volume": [1, 512, 512, 257], "poses": P, "proj": [n, n // 2 + 1], "oversampling": os_}
    return Workload("half", cfg["workload"], ops, cpu_sample, cfg)


# headline is the bench line; c2-c5 are the other BASELINE configurations,
# prep the reference preparation around the headline volume and half the
# headline forward from low-precision storage, run on request
WORKLOADS = {"headline": make_headline, "c2": make_c2, "c3": make_c3, "c4": make_c4, "c5": make_c5,
             "prep": make_prep, "half": make_half}


# ----------------------------------------------------------------------------- CPU baseline
def cpu_ops_and_kind():
    from oracle import oracle as O
    ref = O.ref_ops()
    if ref is not None:
        return ref, "reference"
    return O, "port"


def run_cpu_baseline(wl, target_s=12.0):
    """Time the workload's ops on the host cores on its first p poses.

    p doubles (or scales by the measured rate) until one run takes about half
    of target_s or covers every pose of the workload; short runs are repeated
    up to about target_s and the fastest is reported.
    """
    import torch
    threads = min(16, len(os.sched_getaffinity(0)))
    torch.set_num_threads(threads)
    ops, kind = cpu_ops_and_kind()
    p = min(8, wl.cpu_pmax)
    t, s, parts = wl.cpu_sample(p, threads, ops)
    while t < 0.5 * target_s and p < wl.cpu_pmax:
        p = int(min(wl.cpu_pmax, max(2 * p, p * 0.6 * target_s / max(t, 1e-3))))
        t, s, parts = wl.cpu_sample(p, threads, ops)
    spent, runs = t, 1
    while spent + t < target_s and runs < 5:
        t2, s2, parts2 = wl.cpu_sample(p, threads, ops)
        spent, runs = spent + t2, runs + 1
        if t2 < t:
            t, s, parts = t2, s2, parts2
    split = ", ".join(f"{k} {v:.2f} s" for k, v in parts.items())
    kind, threads = wl.cpu_kind or kind, wl.cpu_cores or threads
    return {"value": s / t, "unit": "Fourier samples/s", "cores": threads, "kind": kind,
            "poses_per_s": p / t, "ops_s": {k: round(v, 4) for k, v in parts.items()},
            "sample": f"first {p} poses of the workload (item 0), every op of the step, best of {runs} "
                      f"run(s) ({t:.2f} s: {split}), {threads} threads"}


# ----------------------------------------------------------------------------- HBM traffic
def measured_traffic(workload, op):
    """HBM bytes per call of `op`, from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary.

    The counters cannot be read from inside a run, so the figure comes from the
    summary profiles/hbm_traffic_<workload>.md (copy-kernel-scaled, read + write,
    summed over the op's kernels); None when there is none for this workload.
    """
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", f"hbm_traffic_{workload}.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_call:"):
                    return json.loads(line.split(":", 1)[1]).get(op)
    except OSError:
        pass
    return None


# ----------------------------------------------------------------------------- main
def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", default="headline", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true")
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
    op_ms = [sum(ev[s][k].elapsed_time(ev[s][k + 1]) for s in range(a.steps)) / a.steps for k in range(nops)]
    ms_step = sum(ev[s][0].elapsed_time(ev[s][nops]) for s in range(a.steps)) / a.steps

    samples_step = sum(op[3] for op in wl.ops)
    per_op = {}
    for k, (name, _, nbytes, samples, poses) in enumerate(wl.ops):
        sec = op_ms[k] / 1e3
        per_op[name] = {"ms": round(op_ms[k], 4), "samples_per_s": samples / sec, "poses_per_s": poses / sec,
                        "alg_GB": nbytes / 1e9, "alg_GBps": nbytes / sec / 1e9,
                        "hbm_frac": nbytes / sec / 1e9 / HBM_PEAK_GBS}
    dom = max(range(nops), key=lambda k: op_ms[k])
    dname, _, dbytes, _, _ = wl.ops[dom]
    achieved = dbytes / (op_ms[dom] / 1e3) / 1e9
    total_bytes = sum(op[2] for op in wl.ops)

    cpu = None
    if not a.no_cpu and wl.cpu_sample is not None:
        log("cpu baseline ...")
        cpu = run_cpu_baseline(wl)
        log(f"cpu baseline: {cpu['sample']}")

    out = {
        "metric": METRIC,
        "value": samples_step / (ms_step / 1e3),
        "unit": "Fourier samples/s",
        "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": wl.config,
        "poses_per_s": wl.ops[0][4] / (ms_step / 1e3),
        "step_alg_GBps": total_bytes / (ms_step / 1e3) / 1e9,
        "step_hbm_frac": total_bytes / (ms_step / 1e3) / 1e9 / HBM_PEAK_GBS,
        "wall_s": round(wall, 3),
        "ops": per_op,
        "roofline": {"bound": "hbm", "kernel": dname, "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": measured_traffic(a.config, dname)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
