"""Opt-in low-precision volume storage: forward projections of a complex32
(complex-half) reconstruction and their backward ops.

The semantics are those of the fp32 path applied to the volume's exact
complex64 widening (each binary16 value is representable in fp32), so the
oracle's result on `rec.to(complex64)` is the expected one, to the same bar as
the fp32 forward: bit-identical without shifts, relative L2 1e-5 with them
(tests/parity.py).  Cases span the tile-owner gathers (rotation poses) and the
per-pixel kernels (scaled pose matrices, an oversampling factor that is not
exact in float, a cutoff), 2D and 3D, linear and cubic.  The backward ops
read the complex32 volume natively too (its rotation and shift gradients; the
reconstruction gradient, a scatter of grad_projections, is complex64 at the C
ABI): against the oracle on the widened volume with the fp32 backward's bar.
Through the dispatcher: complex64 projections, and under autograd a complex32
volume gradient and pose gradients equal to those of the widened volume.
"""
import pytest
import torch

from tests.golden.cases import _case, make_inputs
from tests.parity import check_outputs, rel_l2, scatter_cells

pytestmark = [pytest.mark.gpu, pytest.mark.filterwarnings("ignore:ComplexHalf support is experimental")]


def _cases():
    out = []
    seed = 4242
    for op, n in (("project_3d_to_2d_forw", 48), ("project_2d_forw", 64)):
        for interp in ("linear", "cubic"):
            for os_, cut, shifts, mixed in ((2.0, None, False, False), (2.0, None, True, True),
                                            (1.5, 15.0, False, True), (1.3, None, True, False)):
                seed += 1
                out.append(_case(f"half_{op}_{interp}_os{os_:g}_{'sh' if shifts else 'nosh'}"
                                 f"{'_mixed' if mixed else ''}", op, interp=interp, os=os_, cutoff=cut, B=2,
                                 B_rot=1 if mixed else 2, P=40, n=n, shifts=shifts, seed=seed, special=mixed))
    return out


CASES = _cases()


def _half(args):
    rec = args[0].detach()
    half = rec.to(torch.complex32)
    return [half] + list(args[1:]), half.to(torch.complex64)


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_half_volume_matches_widened_oracle(case, hip, oracle):
    args, tensors = make_inputs(case)
    if case["special"]:
        r = args[1].detach().clone()
        r[:, ::3] *= 1.07  # not rotations: the per-pixel kernel
        args[1] = r
    hargs, widened = _half(args)
    print(f"[half] {case['name']}", flush=True)
    got = getattr(hip, case["op"])(*hargs)
    exp = getattr(oracle, case["op"])(widened, *args[1:])
    check_outputs(case["op"], got, exp, has_shifts=tensors.get("shifts") is not None, label=case["name"])


def _back_cases():
    out = []
    seed = 4343
    for op, n in (("project_3d_to_2d_back", 40), ("project_2d_back", 48)):
        for interp in ("linear", "cubic"):
            for os_, cut, shifts, mixed in ((2.0, None, True, False), (1.5, 13.0, True, True), (1.3, None, False, True)):
                seed += 1
                out.append(_case(f"half_{op}_{interp}_os{os_:g}_{'sh' if shifts else 'nosh'}"
                                 f"{'_mixed' if mixed else ''}", op, interp=interp, os=os_, cutoff=cut, B=2,
                                 B_rot=1 if mixed else 2, P=40, n=n, shifts=shifts, seed=seed, special=mixed))
    return out


BACK_CASES = _back_cases()


@pytest.mark.parametrize("case", BACK_CASES, ids=[c["name"] for c in BACK_CASES])
def test_half_volume_backward_matches_widened_oracle(case, hip, oracle):
    args, tensors = make_inputs(case)  # (grad_projections, reconstruction, rotations, shifts, ...)
    if case["special"]:
        r = args[2].detach().clone()
        r[:, ::3] *= 1.07  # not rotations: the per-pixel kernel
        args[2] = r.requires_grad_(True)
    half = args[1].detach().to(torch.complex32)
    hargs = list(args)
    hargs[1] = half
    wargs = list(args)
    wargs[1] = half.to(torch.complex64)
    print(f"[half] {case['name']}", flush=True)
    got = getattr(hip, case["op"])(*hargs)
    exp = getattr(oracle, case["op"])(*wargs)
    assert got[0].dtype == torch.complex64
    check_outputs(case["op"], got, exp, has_shifts=tensors.get("shifts") is not None, label=case["name"],
                  cells=scatter_cells(case["op"], wargs, oracle))


@pytest.mark.parametrize("interp", ["linear", "cubic"])
@pytest.mark.parametrize("dim", [2, 3])
def test_half_volume_through_autograd(gpu, dim, interp):
    import torch_projectors as tp
    g = torch.Generator().manual_seed(77 + dim)
    n, P = 32, 24
    shape = (1, 2 * n, 2 * n // 2 + 1) if dim == 2 else (1, 2 * n, 2 * n, 2 * n // 2 + 1)
    rec = torch.randn(shape, generator=g, dtype=torch.complex64)
    rot = torch.linalg.qr(torch.randn(1, P, dim, dim, generator=g, dtype=torch.float64))[0].float()
    sh = torch.randn(1, P, 2, generator=g) * 2
    gout = torch.randn(1, P, n, n // 2 + 1, generator=g, dtype=torch.complex64).to(gpu)
    fwd = tp.project_2d_forw if dim == 2 else tp.project_3d_to_2d_forw
    print(f"[half] autograd dim={dim} {interp}", flush=True)

    runs = []
    for volume in (rec.to(torch.complex32), rec.to(torch.complex32).to(torch.complex64)):
        v = volume.to(gpu).requires_grad_(True)
        r = rot.to(gpu).requires_grad_(True)
        s = sh.to(gpu).requires_grad_(True)
        proj = fwd(v, r, shifts=s, output_shape=(n, n), interpolation=interp, oversampling=2.0)
        (torch.view_as_real(proj) * torch.view_as_real(gout)).sum().backward()
        runs.append((proj.detach(), v.grad, r.grad, s.grad))
    (p_h, gv_h, gr_h, gs_h), (p_w, gv_w, gr_w, gs_w) = runs
    assert p_h.dtype == torch.complex64 and gv_h.dtype == torch.complex32
    assert torch.equal(p_h, p_w)  # the same fp32 arithmetic on the same widened values
    assert rel_l2(gv_h.to(torch.complex64), gv_w.to(torch.complex32).to(torch.complex64)) <= 1e-3
    assert rel_l2(gr_h, gr_w) <= 1e-4 and rel_l2(gs_h, gs_w) <= 1e-4
