"""tp_project_3d_to_2d_forw_noalloc: the forward projection whose tiled kernels keep their per-call
pose summary and work counters in a static device array instead of allocated scratch.

Through the C ABI, two calls in a row (the second on a smaller input) must give exactly the
projections of tp_project_3d_to_2d_forw on the same inputs (the gathers are deterministic, so the
bar is bit-identity), and both must meet the oracle's bar (tests/parity.py: bit-identical without
shifts, rel-L2 1e-5 with them).  The poses mix rotations with scaled and sheared matrices (the
GEN kernels that take work from the scratch's counters) and degenerate ones (per-pixel kernels).
Each output starts as NaN, so an element the call leaves unwritten fails.
"""
import ctypes

import pytest
import torch

from tests import hip_path
from tests.parity import check_outputs
from torch_projectors import capi

pytestmark = pytest.mark.gpu

_P = ctypes.c_void_p


def _inputs(B, N, P, n, seed, mix):
    g = torch.Generator().manual_seed(seed)
    rec = torch.randn(B, N, N, N // 2 + 1, dtype=torch.complex64, generator=g)
    q = torch.randn(P, 4, generator=g, dtype=torch.float64)
    q = q / q.norm(dim=1, keepdim=True)
    w, x, y, z = q.unbind(1)
    rot = torch.stack([1 - 2 * (y * y + z * z), 2 * (x * y - z * w), 2 * (x * z + y * w),
                       2 * (x * y + z * w), 1 - 2 * (x * x + z * z), 2 * (y * z - x * w),
                       2 * (x * z - y * w), 2 * (y * z + x * w), 1 - 2 * (x * x + y * y)], 1).reshape(1, P, 3, 3)
    if mix:
        shear = torch.eye(3, dtype=torch.float64)
        shear[0, 1] = 0.15
        for p in range(P):
            k = p % 5
            if k == 1:
                rot[0, p] *= 1.02
            elif k == 2:
                rot[0, p] = shear @ rot[0, p]
            elif k == 3:
                rot[0, p] *= 0.4  # beyond the tiled scale range: per-pixel kernels
    rot = rot.float()
    shifts = (torch.rand(1, P, 2, generator=g) - 0.5) * 6
    return rec, rot, shifts


def _launch(name, rec, rot, shifts, out, n, interp, os_, stream):
    B, D, N, H = rec.shape
    capi.call(name, capi.TP_F32, hip_path._p(rec), B, D, N, H, hip_path._p(rot), rot.shape[0], rot.shape[1],
              hip_path._p(shifts), shifts.shape[0] if shifts is not None else 1, n,
              capi.TP_CUBIC if interp == "cubic" else capi.TP_LINEAR, float(os_), 0, 0.0, hip_path._p(out), stream)


def _call(name, rec, rot, shifts, n, interp, os_):
    out = hip_path._poisoned((rec.shape[0], rot.shape[1], n, n // 2 + 1), torch.complex64)
    _launch(name, rec, rot, shifts, out, n, interp, os_, hip_path._stream())
    torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.parametrize("interp", ["linear", "cubic"])
@pytest.mark.parametrize("with_shifts", [False, True])
def test_noalloc_matches_the_allocating_entry_point(gpu, oracle, interp, with_shifts):
    # the second call is smaller (box, poses, batch) than the first
    for (B, N, P, n, seed) in [(2, 64, 160, 32, 11), (1, 32, 40, 16, 12)]:
        rec, rot, shifts = _inputs(B, N, P, n, seed, mix=True)
        sh = shifts if with_shifts else None
        d_rec, d_rot = rec.to(gpu), rot.to(gpu)
        d_sh = sh.to(gpu) if sh is not None else None
        got = _call("tp_project_3d_to_2d_forw_noalloc", d_rec, d_rot, d_sh, n, interp, 2.0)
        want = _call("tp_project_3d_to_2d_forw", d_rec, d_rot, d_sh, n, interp, 2.0)
        assert not torch.isnan(torch.view_as_real(got)).any()
        assert torch.equal(got, want), (B, N, P, n)
        ref = oracle.project_3d_to_2d_forw(rec, rot, sh, (n, n), interp, 2.0, None)
        check_outputs("project_3d_to_2d_forw", (got,), (ref,), with_shifts, label=f"{interp} B{B} N{N} P{P}")


def test_noalloc_calls_in_a_row_keep_no_state(gpu):
    """A call with no rotation among its poses after one with rotations, and the reverse: the
    scratch of the earlier call must not leak into the later one (each call's pre-pass rewrites it)."""
    rec, rot, shifts = _inputs(1, 48, 64, 24, 21, mix=False)
    scaled = (rot.double() * 1.1).float()
    d_rec = rec.to(gpu)
    for r in (rot, scaled, rot, scaled):
        d_rot = r.to(gpu)
        got = _call("tp_project_3d_to_2d_forw_noalloc", d_rec, d_rot, None, 24, "linear", 2.0)
        want = _call("tp_project_3d_to_2d_forw", d_rec, d_rot, None, 24, "linear", 2.0)
        assert torch.equal(got, want)


def test_noalloc_captured_on_a_stream_no_call_has_used(gpu):
    """The entry point needs no per-stream scratch: captured in a HIP graph on a stream that no call
    has used (where the allocating entry point fails, since it would have to allocate the stream's
    scratch during capture), its replays give exactly the allocating entry point's projections,
    also after new poses are written into the captured input.  Each replay's output starts as NaN."""
    n = 24
    rec, rot, shifts = _inputs(1, 48, 96, n, 31, mix=True)
    d_rec, d_rot, d_sh = rec.to(gpu), rot.to(gpu), shifts.to(gpu)
    shape = (1, rot.shape[1], n, n // 2 + 1)
    # the first call on this device sets up its static scratch; it is made eagerly here, so that the
    # test also holds when it runs alone
    _call("tp_project_3d_to_2d_forw_noalloc", d_rec, d_rot, d_sh, n, "linear", 2.0)
    torch.cuda.synchronize()

    unused = torch.cuda.Stream()
    out0 = torch.empty(shape, dtype=torch.complex64, device=gpu)
    g0 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g0, stream=unused):
        with pytest.raises(RuntimeError, match="first call on a stream allocates"):
            _launch("tp_project_3d_to_2d_forw", d_rec, d_rot, d_sh, out0, n, "linear", 2.0,
                    _P(unused.cuda_stream))
    torch.cuda.synchronize()

    fresh = torch.cuda.Stream()
    out = hip_path._poisoned(shape, torch.complex64)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=fresh):
        _launch("tp_project_3d_to_2d_forw_noalloc", d_rec, d_rot, d_sh, out, n, "linear", 2.0, _P(fresh.cuda_stream))
    torch.cuda.synchronize()

    _, new_rot, _ = _inputs(1, 48, 96, n, 32, mix=True)
    for replay in range(3):
        if replay == 2:
            d_rot.copy_(new_rot.to(gpu))  # new poses in the captured input
        out.fill_(complex(float("nan"), float("nan")))
        graph.replay()
        torch.cuda.synchronize()
        want = _call("tp_project_3d_to_2d_forw", d_rec, d_rot, d_sh, n, "linear", 2.0)
        print(f"[noalloc] replay {replay}", flush=True)
        got = out.cpu()
        assert not torch.isnan(torch.view_as_real(got)).any(), f"replay {replay}: unwritten elements"
        assert torch.equal(got, want), f"replay {replay}: projections differ"
