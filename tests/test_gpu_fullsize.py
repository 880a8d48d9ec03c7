"""The BASELINE configurations at their full sizes, through the dispatcher ops.

Every output is compared whole with the oracle run on the same inputs (all host threads; poses
are independent, so this is what the reference's CPU kernels compute,
cpu/3d/projection_3d_to_2d_kernels.cpp:97-402):

* the headline, c2 and c4 forwards over all their poses (bit-identical without shifts, relative
  L2 1e-5 with them);
* the headline and c3 backprojections and the c4 reconstruction gradient over all 2048 poses,
  whole and cell by cell (tests/parity.py `check_cells`: untouched cells exactly 0, every other
  cell within 1e-5 * max|v| * sum|tap weight| of the exact sum of the reference's taps);
* c4's rotation and shift gradients of all 2048 poses;
* c5 (16 images x 4096 poses, 2.16e9 projection elements): batch item 0 over all its 4096 poses
  through the forward, the backprojection and both backward ops; item 15 on sampled poses and
  its backprojected volume (batch items are independent).

Inputs follow bench.py's synthetic recipes (seeded).  Bars as tests/parity.py: gathers
bit-identical without shifts, else relative L2 1e-5; scatters and pose gradients relative L2 1e-4.
"""
import pytest
import torch

import bench
from tests.parity import GATHER_TOL, SCATTER_TOL, check_scatter, rel_l2

pytestmark = pytest.mark.gpu

F32 = torch.float32


@pytest.fixture(scope="module")
def ops(gpu):
    import torch_projectors  # noqa: F401  (registers the dispatcher ops; fails without the HIP library)
    return torch.ops.torch_projectors


@pytest.fixture(scope="module")
def O():
    from oracle import oracle
    return oracle


def say(msg):
    print(f"[fullsize] {msg}", flush=True)


def close(got, exp, tol, what):
    err = rel_l2(got, exp)
    say(f"{what}: rel L2 {err:.2e}")
    assert err <= tol, f"{what}: relative L2 {err:.3e} > {tol:.0e}"


# ----------------------------------------------------------------------------- headline (3D linear)
@pytest.fixture(scope="module")
def headline(gpu):
    gen = torch.Generator().manual_seed(20261201 + 6)
    vol = bench.blob_volume_rfft(256, 512, 32, 80.0, gen, gpu)
    rot = bench.quat_rotations(2048, gen)[None].to(gpu)
    sh = ((torch.rand(1, 2048, 2, generator=gen) * 16) - 8).to(gpu)
    w = bench.ctf2_weights(1, 2048, 256, gen).float().to(gpu)
    return vol, rot, sh, w


def test_headline_forward_whole(headline, ops, O):
    vol, rot, sh, _ = headline
    say("headline forward, all 2048 poses against the oracle, with shifts")
    vol_c, rot_c = vol.cpu(), rot.cpu()
    proj = ops.project_3d_to_2d_forw(vol, rot, sh, [256, 256], "linear", 2.0, None)
    assert proj.shape == (1, 2048, 256, 129)
    exp = O.project_3d_to_2d_forw(vol_c, rot_c, sh.cpu(), [256, 256], "linear", 2.0, None)
    close(proj.cpu(), exp, GATHER_TOL[F32], "forward with shifts, all poses")
    say("headline forward, all 2048 poses, no shifts: bit-identical")
    proj0 = ops.project_3d_to_2d_forw(vol, rot, None, [256, 256], "linear", 2.0, None)
    exp0 = O.project_3d_to_2d_forw(vol_c, rot_c, None, [256, 256], "linear", 2.0, None)
    assert torch.equal(proj0.cpu(), exp0), "forward without shifts must be bit-identical"


def test_headline_backprojection_whole(headline, ops, O):
    vol, rot, sh, w = headline
    say("headline backprojection, 2048 poses, whole volume against the oracle")
    proj = ops.project_3d_to_2d_forw(vol, rot, sh, [256, 256], "linear", 2.0, None)
    data, wrec = ops.backproject_2d_to_3d_forw(proj, w, rot, sh, "linear", 2.0, None)
    assert data.shape == (1, 512, 512, 257) and wrec.shape == (1, 512, 512, 257)
    proj_c = proj.cpu()
    ed, ew = O.backproject_2d_to_3d_forw(proj_c, w.cpu(), rot.cpu(), sh.cpu(), "linear", 2.0, None)
    close(data.cpu(), ed, SCATTER_TOL[F32], "backprojection data")
    close(wrec.cpu(), ew, SCATTER_TOL[F32], "backprojection weights")
    say("headline backprojection, cell by cell")
    check_scatter("backproject_2d_to_3d_forw", (data, wrec), [proj_c, w, rot, sh, "linear", 2.0, None], O,
                  "headline backprojection")


# ----------------------------------------------------------------------------- c1 - c3
def test_c1_2d_linear_whole(ops, O, gpu):
    gen = torch.Generator().manual_seed(20261201 + 1)
    rec = bench.noise_image_rfft(1, 64, 128, gen, gpu).to(torch.complex64)
    rot = bench.angle_rotations((1, 256), gen).to(gpu)
    sh = (2 * torch.randn(1, 256, 2, generator=gen)).to(gpu)
    say("c1 2D linear forward and backprojection, 256 poses")
    proj = ops.project_2d_forw(rec, rot, sh, [64, 64], "linear", 2.0, None)
    exp = O.project_2d_forw(rec.cpu(), rot.cpu(), sh.cpu(), [64, 64], "linear", 2.0, None)
    close(proj.cpu(), exp, GATHER_TOL[F32], "c1 forward")
    data, _ = ops.backproject_2d_forw(proj, None, rot, sh, "linear", 2.0, None)
    ed, _ = O.backproject_2d_forw(proj.cpu(), None, rot.cpu(), sh.cpu(), "linear", 2.0, None)
    close(data.cpu(), ed, SCATTER_TOL[F32], "c1 backprojection")


def test_c2_forward_whole(ops, O, gpu):
    gen = torch.Generator().manual_seed(20261201 + 2)
    vol = bench.blob_volume_rfft(128, 256, 32, 40.0, gen, gpu)
    rot = bench.quat_rotations(4096, gen)[None].to(gpu)
    sh = ((torch.rand(1, 4096, 2, generator=gen) * 10) - 5).to(gpu)
    say("c2 forward, all 4096 poses of a 256^3 volume")
    vol_c, rot_c = vol.cpu(), rot.cpu()
    proj = ops.project_3d_to_2d_forw(vol, rot, sh, [128, 128], "linear", 2.0, None)
    exp = O.project_3d_to_2d_forw(vol_c, rot_c, sh.cpu(), [128, 128], "linear", 2.0, None)
    close(proj.cpu(), exp, GATHER_TOL[F32], "c2 forward, all poses")
    proj0 = ops.project_3d_to_2d_forw(vol, rot, None, [128, 128], "linear", 2.0, None)
    exp0 = O.project_3d_to_2d_forw(vol_c, rot_c, None, [128, 128], "linear", 2.0, None)
    assert torch.equal(proj0.cpu(), exp0), "c2 forward without shifts must be bit-identical"


def test_c3_backprojection_whole(ops, O, gpu):
    gen = torch.Generator().manual_seed(20261201 + 3)
    proj = torch.randn(1, 8192, 128, 65, generator=gen, dtype=torch.complex64).to(gpu)
    w = bench.ctf2_weights(1, 8192, 128, gen).float().to(gpu)
    rot = bench.quat_rotations(8192, gen)[None].to(gpu)
    sh = ((torch.rand(1, 8192, 2, generator=gen) * 10) - 5).to(gpu)
    say("c3 backprojection, 8192 poses, whole volume against the oracle")
    data, wrec = ops.backproject_2d_to_3d_forw(proj, w, rot, sh, "linear", 2.0, None)
    assert data.shape == (1, 256, 256, 129)
    proj_c = proj.cpu()
    ed, ew = O.backproject_2d_to_3d_forw(proj_c, w.cpu(), rot.cpu(), sh.cpu(), "linear", 2.0, None)
    close(data.cpu(), ed, SCATTER_TOL[F32], "c3 backprojection data")
    close(wrec.cpu(), ew, SCATTER_TOL[F32], "c3 backprojection weights")
    say("c3 backprojection, cell by cell")
    check_scatter("backproject_2d_to_3d_forw", (data, wrec), [proj_c, w, rot, sh, "linear", 2.0, None], O,
                  "c3 backprojection")


# ----------------------------------------------------------------------------- c4 (3D cubic, forward + backward)
@pytest.fixture(scope="module")
def c4(gpu):
    gen = torch.Generator().manual_seed(20261201 + 4)
    vol = bench.blob_volume_rfft(256, 512, 32, 80.0, gen, gpu)
    rot = bench.quat_rotations(2048, gen)[None].to(gpu)
    sh = ((torch.rand(1, 2048, 2, generator=gen) * 16) - 8).to(gpu)
    g = torch.randn(1, 2048, 256, 129, generator=gen, dtype=torch.complex64).to(gpu)
    return vol, rot, sh, g


def test_c4_cubic_forward_whole(c4, ops, O):
    vol, rot, sh, _ = c4
    say("c4 cubic forward, all 2048 poses against the oracle")
    vol_c, rot_c = vol.cpu(), rot.cpu()
    proj = ops.project_3d_to_2d_forw(vol, rot, sh, [256, 256], "cubic", 2.0, None)
    exp = O.project_3d_to_2d_forw(vol_c, rot_c, sh.cpu(), [256, 256], "cubic", 2.0, None)
    close(proj.cpu(), exp, GATHER_TOL[F32], "cubic forward, all poses")
    del proj, exp
    say("c4 cubic forward without shifts, all 2048 poses: bit-identical")
    proj0 = ops.project_3d_to_2d_forw(vol, rot, None, [256, 256], "cubic", 2.0, None)
    exp0 = O.project_3d_to_2d_forw(vol_c, rot_c, None, [256, 256], "cubic", 2.0, None)
    assert torch.equal(proj0.cpu(), exp0), "cubic forward without shifts must be bit-identical"


@pytest.fixture(scope="module")
def c4_back(c4, ops, O):
    """c4's backward on the GPU and in the oracle, all 2048 poses, rotations and shifts requiring grad."""
    vol, rot, sh, g = c4
    say("c4 cubic backward, all 2048 poses: GPU and oracle")
    rg, sg = rot.clone().requires_grad_(True), sh.clone().requires_grad_(True)
    got = ops.project_3d_to_2d_back(g, vol, rg, sg, "cubic", 2.0, None)
    assert got[0].shape == vol.shape and got[1].shape == rot.shape and got[2].shape == sh.shape
    got = tuple(t.cpu() for t in got)
    args = [g.cpu(), vol.cpu(), rot.cpu().requires_grad_(True), sh.cpu().requires_grad_(True), "cubic", 2.0, None]
    exp = O.project_3d_to_2d_back(*args)
    return got, exp, args


def test_c4_cubic_backward_whole(c4_back):
    got, exp, _ = c4_back
    close(got[0], exp[0], SCATTER_TOL[F32], "reconstruction gradient, all poses")
    close(got[1], exp[1], SCATTER_TOL[F32], "rotation gradients, all poses")
    close(got[2], exp[2], SCATTER_TOL[F32], "shift gradients, all poses")


def test_c4_reconstruction_gradient_cells(c4_back, O):
    got, _, args = c4_back
    say("c4 reconstruction gradient, all 2048 poses, cell by cell")
    check_scatter("project_3d_to_2d_back", (got[0],), [a.detach() if isinstance(a, torch.Tensor) else a for a in args],
                  O, "reconstruction gradient, all poses")


# ----------------------------------------------------------------------------- c5 (batched 2D cubic)
@pytest.fixture(scope="module")
def c5(gpu):
    gen = torch.Generator().manual_seed(20261201 + 5)
    rec = bench.noise_image_rfft(16, 256, 512, gen, gpu).to(torch.complex64)
    rot = bench.angle_rotations((16, 4096), gen).to(gpu)
    sh = (3 * torch.randn(16, 4096, 2, generator=gen)).to(gpu)
    return rec, rot, sh


ITEMS = [0, 15]
PAIRS = [(15, 2048), (15, 7)]  # sampled poses of item 15 (item 0 is compared whole)


def test_c5_batched_2d_cubic(c5, ops, O):
    rec, rot, sh = c5
    say("c5 forward: 16 x 4096 projections (2.16e9 complex elements)")
    proj = ops.project_2d_forw(rec, rot, sh, [256, 256], "cubic", 2.0, 64.0)
    assert proj.shape == (16, 4096, 256, 129) and proj.numel() > 2 ** 31
    rec_c = rec.cpu()
    r0, s0 = rot[0:1].cpu(), sh[0:1].cpu()
    say("c5 forward, item 0, all 4096 poses against the oracle")
    exp = O.project_2d_forw(rec_c[0:1], r0, s0, [256, 256], "cubic", 2.0, 64.0)
    close(proj[0:1].cpu(), exp, GATHER_TOL[F32], "forward (item 0, all poses)")
    del exp
    for b, p in PAIRS:
        exp = O.project_2d_forw(rec_c[b:b + 1], rot[b:b + 1, p:p + 1].cpu(), sh[b:b + 1, p:p + 1].cpu(), [256, 256],
                                "cubic", 2.0, 64.0)
        close(proj[b:b + 1, p:p + 1].cpu(), exp, GATHER_TOL[F32], f"forward (item {b}, pose {p})")

    say("c5 backprojection with unit weights")
    ones = torch.ones(16, 4096, 256, 129, device=proj.device, dtype=F32)
    data, wrec = ops.backproject_2d_forw(proj, ones, rot, sh, "cubic", 2.0, 64.0)
    assert data.shape == (16, 512, 257)
    for b in ITEMS:
        ed, ew = O.backproject_2d_forw(proj[b:b + 1].cpu(), ones[b:b + 1].cpu(), rot[b:b + 1].cpu(),
                                       sh[b:b + 1].cpu(), "cubic", 2.0, 64.0)
        close(data[b:b + 1].cpu(), ed, SCATTER_TOL[F32], f"backprojection data (item {b})")
        close(wrec[b:b + 1].cpu(), ew, SCATTER_TOL[F32], f"backprojection weights (item {b})")
        check_scatter("backproject_2d_forw", (data[b:b + 1], wrec[b:b + 1]),
                      [proj[b:b + 1], ones[b:b + 1], rot[b:b + 1], sh[b:b + 1], "cubic", 2.0, 64.0], O,
                      f"backprojection (item {b})")

    say("c5 backward of a loss on (data, weight)")
    gen = torch.Generator().manual_seed(20261201 + 55)
    gd = torch.randn(16, 512, 257, generator=gen, dtype=torch.complex64).to(proj.device)
    gw = torch.randn(16, 512, 257, generator=gen).to(proj.device)
    rg, sg = rot.clone().requires_grad_(True), sh.clone().requires_grad_(True)
    gproj, gwts, grot, gsh = ops.backproject_2d_back(gd, gw, proj, ones, rg, sg, "cubic", 2.0, 64.0)
    assert gproj.shape == proj.shape and gwts.shape == ones.shape
    say("c5 backproject_2d_back, item 0, all 4096 poses against the oracle")
    e = O.backproject_2d_back(gd[0:1].cpu(), gw[0:1].cpu(), proj[0:1].cpu(), ones[0:1].cpu(),
                              r0.clone().requires_grad_(True), s0.clone().requires_grad_(True), "cubic", 2.0, 64.0)
    close(gproj[0:1].cpu(), e[0], GATHER_TOL[F32], "grad_projections (item 0, all poses)")
    close(gwts[0:1].cpu(), e[1], GATHER_TOL[F32], "grad_weights (item 0, all poses)")
    close(grot[0:1].cpu(), e[2], SCATTER_TOL[F32], "grad_rotations (item 0, all poses)")
    close(gsh[0:1].cpu(), e[3], SCATTER_TOL[F32], "grad_shifts (item 0, all poses)")
    del e
    for b, p in PAIRS:
        r_c = rot[b:b + 1, p:p + 1].cpu().requires_grad_(True)
        s_c = sh[b:b + 1, p:p + 1].cpu().requires_grad_(True)
        e = O.backproject_2d_back(gd[b:b + 1].cpu(), gw[b:b + 1].cpu(), proj[b:b + 1, p:p + 1].cpu(),
                                  ones[b:b + 1, p:p + 1].cpu(), r_c, s_c, "cubic", 2.0, 64.0)
        close(gproj[b:b + 1, p:p + 1].cpu(), e[0], GATHER_TOL[F32], f"grad_projections (item {b}, pose {p})")
        close(gwts[b:b + 1, p:p + 1].cpu(), e[1], GATHER_TOL[F32], f"grad_weights (item {b}, pose {p})")
        close(grot[b:b + 1, p:p + 1].cpu(), e[2], SCATTER_TOL[F32], f"grad_rotations (item {b}, pose {p})")
        close(gsh[b:b + 1, p:p + 1].cpu(), e[3], SCATTER_TOL[F32], f"grad_shifts (item {b}, pose {p})")
    del ones, gwts

    say("c5 project_2d_back, item 0, all 4096 poses against the oracle: reconstruction, rotation and shift "
        "gradients")
    grec, grot, gsh = ops.project_2d_back(gproj, rec, rg, sg, "cubic", 2.0, 64.0)
    assert grec.shape == rec.shape and grot.shape == rot.shape and gsh.shape == sh.shape
    g0 = gproj[0:1].cpu()
    eg, er, es = O.project_2d_back(g0, rec_c[0:1], r0.clone().requires_grad_(True), s0.clone().requires_grad_(True),
                                   "cubic", 2.0, 64.0)
    close(grec[0:1].cpu(), eg, SCATTER_TOL[F32], "reconstruction gradient (item 0)")
    close(grot[0:1].cpu(), er, SCATTER_TOL[F32], "project_2d_back grad_rotations (item 0, all poses)")
    close(gsh[0:1].cpu(), es, SCATTER_TOL[F32], "project_2d_back grad_shifts (item 0, all poses)")
    check_scatter("project_2d_back", (grec[0:1],), [g0, rec_c[0:1], r0, s0, "cubic", 2.0, 64.0], O,
                  "reconstruction gradient (item 0)")
    for b, p in PAIRS:
        r_c = rot[b:b + 1, p:p + 1].cpu().requires_grad_(True)
        s_c = sh[b:b + 1, p:p + 1].cpu().requires_grad_(True)
        _, er, es = O.project_2d_back(gproj[b:b + 1, p:p + 1].cpu(), rec_c[b:b + 1], r_c, s_c, "cubic", 2.0, 64.0)
        close(grot[b:b + 1, p:p + 1].cpu(), er, SCATTER_TOL[F32], f"project_2d_back grad_rotations ({b}, {p})")
        close(gsh[b:b + 1, p:p + 1].cpu(), es, SCATTER_TOL[F32], f"project_2d_back grad_shifts ({b}, {p})")


# ----------------------------------------------------------------------------- empty inputs
def test_zero_poses(ops, gpu):
    vol = torch.randn(1, 32, 32, 17, dtype=torch.complex64, device=gpu)
    rot = torch.empty(1, 0, 3, 3, device=gpu)
    proj = ops.project_3d_to_2d_forw(vol, rot, None, [32, 32], "linear", 1.0, None)
    assert proj.shape == (1, 0, 32, 17)
    data, wrec = ops.backproject_2d_to_3d_forw(proj, torch.empty(1, 0, 32, 17, device=gpu), rot, None, "linear",
                                               2.0, None)
    torch.cuda.synchronize()
    assert data.shape == (1, 64, 64, 33) and torch.count_nonzero(data) == 0 and torch.count_nonzero(wrec) == 0
    grec, grot, gsh = ops.project_3d_to_2d_back(proj, vol, rot, None, "cubic", 1.0, None)
    assert grec.shape == vol.shape and torch.count_nonzero(grec) == 0
