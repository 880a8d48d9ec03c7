"""Input layouts through the dispatcher ops on cuda:0.

The reference copies non-contiguous inputs to contiguous ones before its
kernels (cuda/3d/projection_3d_to_2d_kernels.cu:880-883), so a strided view,
an expanded (stride-0) pose tensor or a permuted shift tensor must give the
result of the same values laid out densely: bit for bit for the forward
projections (deterministic gathers), within rel-L2 1e-6 for the scatters
(the order of fp64 partial sums may differ).  Poses in float64 with a
complex64 volume are rejected, as the reference's GPU path rejects them (its
CUDA wrapper reads them through data_ptr<float>,
cuda/3d/projection_3d_to_2d_kernels.cu:987-988), and so are shifts whose
dtype differs from the rotations' (projection_utils.h:45-46) and weights
whose dtype differs from the rotations' (the reference reads weights through
the rotations' type, cpu/3d/backprojection_2d_to_3d_kernels.cpp:165-169).
"""
import pytest
import torch

from tests.parity import rel_l2

pytestmark = pytest.mark.gpu

T = torch.ops.torch_projectors


def _views(dev, dim, B=2, P=24, n=32, seed=0):
    g = torch.Generator().manual_seed(seed)
    N = 2 * n
    shape = (B, N, N // 2 + 1) if dim == 2 else (B, N, N, N // 2 + 1)
    pad = shape[:-1] + (shape[-1] + 3,)
    big = torch.randn(pad, generator=g, dtype=torch.complex64).to(dev)
    rec = big[..., :shape[-1]]                      # strided: rows longer than the data
    q = torch.linalg.qr(torch.randn(P, dim, dim, generator=g, dtype=torch.float64))[0]
    rot = q.float().to(dev)[None].expand(B, P, dim, dim)  # stride 0 over the batch
    sh = (torch.randn(2, P, B, generator=g) * 2).to(dev).permute(2, 1, 0)  # [B, P, 2], permuted
    return rec, rot, sh, n


@pytest.mark.parametrize("interp", ["linear", "cubic"])
@pytest.mark.parametrize("dim", [2, 3])
def test_strided_inputs_forward(gpu, dim, interp):
    rec, rot, sh, n = _views(gpu, dim)
    assert not rec.is_contiguous() and not rot.is_contiguous() and not sh.is_contiguous()
    f = T.project_2d_forw if dim == 2 else T.project_3d_to_2d_forw
    print(f"[layouts] forward dim={dim} {interp}", flush=True)
    got = f(rec, rot, sh, [n, n], interp, 2.0, None)
    exp = f(rec.contiguous(), rot.contiguous(), sh.contiguous(), [n, n], interp, 2.0, None)
    assert torch.equal(got, exp)
    with pytest.raises(RuntimeError, match="needs float32 rotations"):
        f(rec, rot.double(), sh.double(), [n, n], interp, 2.0, None)
    with pytest.raises(RuntimeError, match="same dtype"):
        f(rec, rot, sh.double(), [n, n], interp, 2.0, None)


@pytest.mark.parametrize("interp", ["linear", "cubic"])
@pytest.mark.parametrize("dim", [2, 3])
def test_strided_inputs_backprojection(gpu, dim, interp):
    g = torch.Generator().manual_seed(5 + dim)
    B, P, n = 2, 24, 32
    big = torch.randn(B, P, n, n // 2 + 4, generator=g, dtype=torch.complex64).to(gpu)
    proj = big[..., :n // 2 + 1]
    wbig = torch.rand(B, P, n // 2 + 1, n, generator=g).to(gpu)
    w = wbig.transpose(-1, -2)  # [B, P, n, n/2+1], transposed view
    q = torch.linalg.qr(torch.randn(P, dim, dim, generator=g, dtype=torch.float64))[0]
    rot = q.float().to(gpu)[None].expand(B, P, dim, dim)
    sh = (torch.randn(2, P, B, generator=g) * 2).to(gpu).permute(2, 1, 0)
    f = T.backproject_2d_forw if dim == 2 else T.backproject_2d_to_3d_forw
    print(f"[layouts] backprojection dim={dim} {interp}", flush=True)
    d1, w1 = f(proj, w, rot, sh, interp, 2.0, None)
    d2, w2 = f(proj.contiguous(), w.contiguous(), rot.contiguous(), sh.contiguous(), interp, 2.0, None)
    assert rel_l2(d1, d2) <= 1e-6 and rel_l2(w1, w2) <= 1e-6
    with pytest.raises(RuntimeError, match="Weights must have the rotations' dtype"):
        f(proj, w.double(), rot, sh, interp, 2.0, None)
    with pytest.raises(RuntimeError, match="needs float32 rotations"):
        f(proj, w.double(), rot.double(), sh.double(), interp, 2.0, None)
    # complex128 takes float32 poses and weights: widened exactly, weight volume in the weights' dtype
    p64 = proj.to(torch.complex128)
    d3, w3 = f(p64, w, rot, sh, interp, 2.0, None)
    d4, w4 = f(p64, w.double(), rot.double(), sh.double(), interp, 2.0, None)
    assert w3.dtype == torch.float32 and w4.dtype == torch.float64
    assert rel_l2(d3, d4) <= 1e-12 and rel_l2(w3.double(), w4) <= 1e-6


@pytest.mark.parametrize("interp", ["linear", "cubic"])
@pytest.mark.parametrize("odd_box", [False, True])
def test_volume_at_an_8_byte_boundary(gpu, oracle, interp, odd_box):
    """A contiguous volume whose first element sits 8 bytes past a 16-byte boundary (a view one
    element into a buffer), and one of odd box size (odd elements per batch item, so batch item 1
    starts off a 16-byte boundary): the tiled forward reads complex64 values at 8-byte alignment
    only, so such volumes give the projections of an aligned copy, bit for bit, and the oracle's."""
    g = torch.Generator().manual_seed(41 + odd_box)
    B, P, n = 2, 20, 32
    N = 2 * n + (1 if odd_box else 0)
    shape = (B, N, N, N // 2 + 1)
    numel = B * N * N * (N // 2 + 1)
    flat = torch.randn(numel + 1, generator=g, dtype=torch.complex64).to(gpu)
    rec = flat[1:].view(shape)
    assert rec.data_ptr() % 16 == 8 and rec.is_contiguous()
    q = torch.linalg.qr(torch.randn(P, 3, 3, generator=g, dtype=torch.float64))[0]
    rot = q.float()[None].expand(B, P, 3, 3).contiguous()
    print(f"[layouts] 8-byte boundary volume {interp} odd_box={odd_box}", flush=True)
    got = T.project_3d_to_2d_forw(rec, rot.to(gpu), None, [n, n], interp, 2.0, None)
    aligned = T.project_3d_to_2d_forw(rec.clone(), rot.to(gpu), None, [n, n], interp, 2.0, None)
    assert torch.equal(got, aligned)
    ref = oracle.project_3d_to_2d_forw(rec.cpu(), rot, None, (n, n), interp, 2.0, None)
    assert torch.equal(got.cpu(), ref)
