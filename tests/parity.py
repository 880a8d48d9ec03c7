"""Tolerances and comparison helpers shared by the parity tests.

The bar (fp32): gathers (forward projections, and the grad_projections /
grad_weights gathers of the backprojection backward) within relative L2
1e-5 of the reference, and bit-identical when no shift phase is involved
(same stencil indices, Friedel/clamp decisions, per-tap products and
summation order); scatters (data/weight volumes, reconstruction gradients)
and per-pose rotation/shift gradients, whose float-atomic or reduction
order differs, within relative L2 1e-4.  fp64 runs use 1e-12 / 1e-10.
"""
import torch

GATHER_TOL = {torch.float32: 1e-5, torch.float64: 1e-12}
SCATTER_TOL = {torch.float32: 1e-4, torch.float64: 1e-10}

# which outputs of each op are gathers (the rest are scatters or pose sums)
GATHER_OUTPUTS = {
    "project_2d_forw": {0}, "project_3d_to_2d_forw": {0},
    "backproject_2d_back": {0, 1}, "backproject_2d_to_3d_back": {0, 1},
}


def real_dtype(t):
    return torch.float64 if t.dtype in (torch.float64, torch.complex128) else torch.float32


def rel_l2(got, exp):
    g = torch.view_as_real(got) if got.is_complex() else got
    e = torch.view_as_real(exp) if exp.is_complex() else exp
    g, e = g.double(), e.double()
    den = e.norm().item()
    num = (g - e).norm().item()
    if den == 0.0:
        return num
    return num / den


def check_outputs(op, got, expected, has_shifts, label=""):
    """Compare a tuple of outputs with the expected ones under the op's bar."""
    if isinstance(got, torch.Tensor):
        got = (got,)
    if isinstance(expected, torch.Tensor):
        expected = (expected,)
    assert len(got) == len(expected), label
    for k, (g, e) in enumerate(zip(got, expected)):
        assert g.shape == e.shape, f"{label} output {k}: shape {tuple(g.shape)} vs {tuple(e.shape)}"
        assert g.dtype == e.dtype, f"{label} output {k}: dtype {g.dtype} vs {e.dtype}"
        if e.numel() == 0:
            continue
        assert torch.isfinite(torch.view_as_real(g) if g.is_complex() else g).all(), f"{label} output {k} not finite"
        gather = k in GATHER_OUTPUTS.get(op, set())
        if gather and not has_shifts:
            if not torch.equal(g, e):
                d = (g - e).abs().max().item()
                raise AssertionError(f"{label} output {k}: gather without shifts must be bit-identical, "
                                     f"max |d| = {d:.3e}")
            continue
        tol = (GATHER_TOL if gather else SCATTER_TOL)[real_dtype(e)]
        err = rel_l2(g, e)
        assert err <= tol, f"{label} output {k}: relative L2 {err:.3e} > {tol:.0e}"
