"""Calls on two streams at once: every (device, stream) has its own call scratch and pose-bin
workspace, so the forward and the weighted backprojection enqueued on two streams without any
order between them must give the results of the same calls made one after the other on one
stream (projections bit for bit; volumes within relative L2 1e-5, the order of their fp64 sums
aside).  Both calls have enough poses for the pose bins, and different pose counts, so the two
streams' workspaces differ in size.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a = torch.view_as_real(a) if a.is_complex() else a
    b = torch.view_as_real(b) if b.is_complex() else b
    return ((a.double() - b.double()).norm() / b.double().norm()).item()


def _inputs(P, seed, gpu, n=32, N=64):
    g = torch.Generator().manual_seed(seed)
    vol = torch.randn(1, N, N, N // 2 + 1, generator=g, dtype=torch.complex64).to(gpu)
    rot = torch.linalg.qr(torch.randn(1, P, 3, 3, generator=g, dtype=torch.float64))[0].float().to(gpu)
    sh = (torch.rand(1, P, 2, generator=g) * 4 - 2).to(gpu)
    w = torch.rand(1, P, n, n // 2 + 1, generator=g).to(gpu)
    return vol, rot, sh, w, n


def _step(vol, rot, sh, w, n, interp):
    T = torch.ops.torch_projectors
    proj = T.project_3d_to_2d_forw(vol, rot, sh, [n, n], interp, 2.0, None)
    data, wrec = T.backproject_2d_to_3d_forw(proj, w, rot, sh, interp, 2.0, None)
    return proj, data, wrec


@pytest.mark.parametrize("interp", ["linear", "cubic"])
def test_two_streams_match_serial_calls(gpu, interp):
    a = _inputs(48, 9100, gpu)
    b = _inputs(96, 9101, gpu)
    serial = [_step(*a, interp), _step(*b, interp)]
    torch.cuda.synchronize()
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    sa.wait_stream(torch.cuda.current_stream())
    sb.wait_stream(torch.cuda.current_stream())
    for rep in range(3):
        with torch.cuda.stream(sa):
            ra = _step(*a, interp)
        with torch.cuda.stream(sb):
            rb = _step(*b, interp)
        torch.cuda.synchronize()
        print(f"[streams] {interp} round {rep}", flush=True)
        for got, exp, tag in ((ra, serial[0], "a"), (rb, serial[1], "b")):
            assert torch.equal(got[0], exp[0]), f"{tag}: projections differ"
            assert _rel(got[1], exp[1]) <= 1e-5, f"{tag}: data volume {_rel(got[1], exp[1]):.3e}"
            assert _rel(got[2], exp[2]) <= 1e-5, f"{tag}: weight volume {_rel(got[2], exp[2]):.3e}"


@pytest.mark.parametrize("shared_stream", [False, True])
def test_two_host_threads_match_serial_calls(gpu, shared_stream):
    """Two host threads enqueue at once, each on its own stream or both on one stream: the
    (device, stream) scratch table is shared between threads, and calls on one stream take its
    area's lock while they enqueue, so the results equal the serial calls'."""
    import threading
    a = _inputs(48, 9200, gpu)
    b = _inputs(80, 9201, gpu)
    serial = [_step(*a, "linear"), _step(*b, "linear")]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream()] * 2 if shared_stream else [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    results, errors = [None, None], []

    def work(i, inp):
        try:
            torch.cuda.set_device(gpu)
            with torch.cuda.stream(streams[i]):
                for _ in range(5):
                    results[i] = _step(*inp, "linear")
        except Exception as e:  # reported by the main thread
            errors.append(e)

    threads = [threading.Thread(target=work, args=(0, a)), threading.Thread(target=work, args=(1, b))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    print(f"[streams] two host threads, shared stream {shared_stream}", flush=True)
    for got, exp, tag in ((results[0], serial[0], "a"), (results[1], serial[1], "b")):
        assert torch.equal(got[0], exp[0]), f"{tag}: projections differ"
        assert _rel(got[1], exp[1]) <= 1e-5, f"{tag}: data volume {_rel(got[1], exp[1]):.3e}"
        assert _rel(got[2], exp[2]) <= 1e-5, f"{tag}: weight volume {_rel(got[2], exp[2]):.3e}"
