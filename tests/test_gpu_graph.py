"""The headline ops (tiled 3D forward and weighted backprojection) captured in a HIP graph.

A warm-up on the capture stream creates the stream's scratch with fewer poses than the captured
calls, so the captured backprojection cannot grow its pose-bin workspace (a capturing stream can
neither wait nor allocate) and runs without bins.  Every replay, with eager work and
synchronisations between replays and new pose values written into the captured input, is compared
with eager calls of the same ops: forward projections bit for bit (they do not depend on the bins),
the backprojected volumes within relative L2 1e-5 (they differ only in the order of the fp64 sums).

The second test captures calls that do use the stream's pose bins (the warm-up had as many poses),
then grows that workspace with an eager call of twice the poses on the same stream: the replays
must still read the workspace the capture recorded, which stays allocated.

The third captures a forward that uses the stream's list of the rotation kernels' work items in
reach (made by the warm-up of the same geometry), then runs forwards of five other geometries on
the capture stream, which replace every list the stream keeps (four): the replays must still read
the list the capture recorded, and the other geometries' forwards must equal the same calls on
another stream.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a = torch.view_as_real(a) if a.is_complex() else a
    b = torch.view_as_real(b) if b.is_complex() else b
    return ((a.double() - b.double()).norm() / b.double().norm()).item()


def _rotations(P, gen):
    q = torch.randn(P, 4, generator=gen, dtype=torch.float64)
    q = q / q.norm(dim=1, keepdim=True)
    w, x, y, z = q.unbind(1)
    R = torch.stack([1 - 2 * (y * y + z * z), 2 * (x * y - z * w), 2 * (x * z + y * w),
                     2 * (x * y + z * w), 1 - 2 * (x * x + z * z), 2 * (y * z - x * w),
                     2 * (x * z - y * w), 2 * (y * z + x * w), 1 - 2 * (x * x + y * y)], 1)
    return R.reshape(1, P, 3, 3).float()


def test_forward_and_backprojection_replayed(gpu):
    T = torch.ops.torch_projectors
    gen = torch.Generator().manual_seed(8080)
    P, n, os_, N = 40, 32, 2.0, 64
    vol = torch.randn(1, N, N, N // 2 + 1, generator=gen, dtype=torch.complex64).to(gpu)
    rot = _rotations(P, gen).to(gpu)
    sh = (torch.rand(1, P, 2, generator=gen) * 4 - 2).to(gpu)
    w = torch.rand(1, P, n, n // 2 + 1, generator=gen).to(gpu)

    def step(v, r, s, ww):
        proj = T.project_3d_to_2d_forw(v, r, s, [n, n], "linear", os_, None)
        data, wrec = T.backproject_2d_to_3d_forw(proj, ww, r, s, "linear", os_, None)
        return proj, data, wrec

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        # the stream's scratch, with a pose-bin workspace for half the poses
        step(vol, rot[:, :P // 2].contiguous(), sh[:, :P // 2].contiguous(), w[:, :P // 2].contiguous())
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        proj_g, data_g, wrec_g = step(vol, rot, sh, w)
    torch.cuda.synchronize()

    gen2 = torch.Generator().manual_seed(8081)
    for replay in range(3):
        if replay == 2:
            rot.copy_(_rotations(P, gen2).to(gpu))  # new poses in the captured input
        graph.replay()
        torch.cuda.synchronize()
        proj_e, data_e, wrec_e = step(vol, rot, sh, w)  # eager, with pose bins
        torch.cuda.synchronize()
        print(f"[graph] replay {replay}", flush=True)
        assert torch.equal(proj_g, proj_e), f"replay {replay}: projections differ"
        assert _rel(data_g, data_e) <= 1e-5, f"replay {replay}: data volume {_rel(data_g, data_e):.3e}"
        assert _rel(wrec_g, wrec_e) <= 1e-5, f"replay {replay}: weight volume {_rel(wrec_g, wrec_e):.3e}"


def test_replay_after_the_bin_workspace_grew(gpu):
    T = torch.ops.torch_projectors
    gen = torch.Generator().manual_seed(8090)
    P, n, os_, N = 48, 32, 2.0, 64
    vol = torch.randn(1, N, N, N // 2 + 1, generator=gen, dtype=torch.complex64).to(gpu)
    rot = _rotations(2 * P, gen).to(gpu)
    sh = (torch.rand(1, 2 * P, 2, generator=gen) * 4 - 2).to(gpu)
    w = torch.rand(1, 2 * P, n, n // 2 + 1, generator=gen).to(gpu)
    proj = T.project_3d_to_2d_forw(vol, rot, sh, [n, n], "linear", os_, None)
    r1, s1, p1, w1 = (t[:, :P].contiguous() for t in (rot, sh, proj, w))

    def bp(p, ww, r, s):
        return T.backproject_2d_to_3d_forw(p, ww, r, s, "linear", os_, None)

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        bp(p1, w1, r1, s1)  # the stream's scratch, with a pose-bin workspace for P poses
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        data_g, wrec_g = bp(p1, w1, r1, s1)  # fits the workspace: the captured calls use the bins
    torch.cuda.synchronize()

    with torch.cuda.stream(stream):
        bp(proj, w, rot, sh)  # twice the poses: the workspace grows
    torch.cuda.synchronize()
    data_e, wrec_e = bp(p1, w1, r1, s1)
    torch.cuda.synchronize()
    for replay in range(3):
        graph.replay()
        torch.cuda.synchronize()
        print(f"[graph] replay {replay} after growth", flush=True)
        assert _rel(data_g, data_e) <= 1e-5, f"replay {replay}: data volume {_rel(data_g, data_e):.3e}"
        assert _rel(wrec_g, wrec_e) <= 1e-5, f"replay {replay}: weight volume {_rel(wrec_g, wrec_e):.3e}"
        with torch.cuda.stream(stream):
            bp(proj, w, rot, sh)  # eager work on the capture stream between replays
        torch.cuda.synchronize()


def test_fourier_transforms_replayed_after_plan_eviction(gpu):
    """hipFFT transforms captured after one eager call of their shape on the capture stream, then
    replayed after more distinct shapes on that stream than the plan cache holds (32): the plans a
    graph uses are never evicted, so every replay matches an eager transform."""
    from torch_projectors import fourier as FM
    gen = torch.Generator().manual_seed(8100)
    x = torch.randn(2, 32, 32, 32, generator=gen).to(gpu)
    others = [torch.randn(b, 8, 8, generator=gen).to(gpu) for b in range(1, 41)]
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        FM._irfftn_consuming(FM._rfftn(x, 3), 3)  # the stream's plans of both shapes
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        spec_g = FM._rfftn(x, 3)
        back_g = FM._irfftn_consuming(spec_g.clone(), 3)
    torch.cuda.synchronize()

    spec_e = FM._rfftn(x, 3)
    back_e = FM._irfftn_consuming(spec_e.clone(), 3)
    torch.cuda.synchronize()
    for replay in range(3):
        with torch.cuda.stream(stream):
            for t in others:  # eager transforms on the capture stream: the cache evicts its other plans
                FM._rfftn(t, 2)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        print(f"[graph] fourier replay {replay}", flush=True)
        assert _rel(spec_g, spec_e) <= 1e-6, f"replay {replay}: spectrum {_rel(spec_g, spec_e):.3e}"
        assert _rel(back_g, back_e) <= 1e-6, f"replay {replay}: inverse {_rel(back_g, back_e):.3e}"


def test_replay_after_the_forward_lists_turned_over(gpu):
    T = torch.ops.torch_projectors
    gen = torch.Generator().manual_seed(8100)
    P, n, os_, N = 24, 32, 2.0, 64
    vol = torch.randn(1, N, N, N // 2 + 1, generator=gen, dtype=torch.complex64).to(gpu)
    rot = _rotations(P, gen).to(gpu)
    sh = (torch.rand(1, P, 2, generator=gen) * 4 - 2).to(gpu)

    def fwd(v, r, s, m):
        return T.project_3d_to_2d_forw(v, r, s, [m, m], "linear", os_, None)

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        fwd(vol, rot, sh, n)  # the stream's area, with the list of this geometry
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        proj_g = fwd(vol, rot, sh, n)
    torch.cuda.synchronize()

    others = [(16, 64), (24, 64), (40, 64), (48, 64), (16, 32)]  # (projection size, volume size)
    vols = {m: torch.randn(1, m, m, m // 2 + 1, generator=gen, dtype=torch.complex64).to(gpu) for m in (32, 64)}
    for replay in range(3):
        with torch.cuda.stream(stream):
            outs = [fwd(vols[vn], rot, sh, pn) for pn, vn in others]  # new lists on the capture stream
        torch.cuda.synchronize()
        for (pn, vn), o in zip(others, outs):
            assert torch.equal(o, fwd(vols[vn], rot, sh, pn)), f"geometry n={pn} N={vn} differs between streams"
        graph.replay()
        torch.cuda.synchronize()
        proj_e = fwd(vol, rot, sh, n)
        torch.cuda.synchronize()
        print(f"[graph] replay {replay} after the lists turned over", flush=True)
        assert torch.equal(proj_g, proj_e), f"replay {replay}: projections differ"

