"""Tolerances and comparison helpers shared by the parity tests.

The bar (fp32): gathers (forward projections, and the grad_projections /
grad_weights gathers of the backprojection backward) within relative L2
1e-5 of the reference, and bit-identical when no shift phase is involved
(same stencil indices, Friedel/clamp decisions, per-tap products and
summation order); scatters (data/weight volumes, reconstruction gradients)
and per-pose rotation/shift gradients, whose float-atomic or reduction
order differs, within relative L2 1e-4 (scatter volumes with fp32 inputs:
of the exact sum of the reference's taps, below).  fp64 runs use 1e-12 / 1e-10.

Scatter volumes are also checked cell by cell (`check_cells`) against the
exact sum of the reference's fp32 tap values (oracle.scatter_wide: the
oracle's fp32 coordinates, stencil decisions and tap products, summed in
double; complex128 runs use the oracle's own result): a cell that sum leaves
exactly 0 (no tap reached it) must be exactly 0, and every other cell must
satisfy |got - expected| <= CELL_TOL * vmax * U, where vmax bounds |v| of the
scattered values and U is the cell's sum of |tap weight| over every sample
(the oracle's weight volume of a unit-weight backprojection with the same
poses, `scatter_cells`).  A tap dropped at a tile edge, a missed Friedel flip
or a missed x = 0 mirror moves a cell by |v| times a tap weight, far above
that bar, while the rounding of the tap products and of the final fp32 value
stays far below it.  (An fp32 sum in one order is not a sound reference for
this bar: 2048 poses adding the same DC value drift by ~3e-5 of U.)
"""
import math

import torch

GATHER_TOL = {torch.float32: 1e-5, torch.float64: 1e-12}
SCATTER_TOL = {torch.float32: 1e-4, torch.float64: 1e-10}
CELL_TOL = {torch.float32: 1e-5, torch.float64: 1e-12}

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


def _rec_box(n, os_):
    raw = int(math.ceil(n * os_))
    return raw + raw % 2


def unit_weight_volume(oracle, three_d, like_proj, rotations, interpolation, oversampling, cutoff):
    """Sum of |tap weight| per cell over every sample of these poses: the weight volume of the
    oracle's backprojection with unit weights (its x = 0 mirror included)."""
    rdt = real_dtype(like_proj)
    zeros = torch.zeros(like_proj.shape, dtype=like_proj.dtype)
    ones = torch.ones(like_proj.shape, dtype=rdt)
    fn = oracle.backproject_2d_to_3d_forw if three_d else oracle.backproject_2d_forw
    return fn(zeros, ones, rotations.detach().cpu(), None, interpolation, oversampling, cutoff)[1]


def _amax(t):
    t = t.detach().cpu()
    return (t.abs().max().item() if t.numel() else 0.0)


def scatter_cells(op, args, oracle):
    """{output index: (U or None, vmax, exact or None)} for the scatter volumes of `op` called with
    `args` (the dispatcher op's positional arguments, CPU or GPU tensors).  U is None where the op's
    volume box differs from the backprojection box of its projections (those outputs get the
    exact-zero test only); exact is the double-summed expectation for fp32 inputs (None: compare
    with the oracle's own result)."""
    three = "3d" in op
    cpu = [a.detach().cpu() if isinstance(a, torch.Tensor) else a for a in args]
    if op.startswith("backproject") and op.endswith("forw"):
        proj, w, rot, _sh, interp, os_, cut = cpu
        wide = oracle.scatter_wide(op, cpu) if proj.dtype == torch.complex64 else (None, None)
        U = unit_weight_volume(oracle, three, proj, rot, interp, os_, cut)
        cells = {0: (U, _amax(proj), wide[0])}
        if w is not None:
            cells[1] = (U, _amax(w), wide[1])
        return cells
    if op.startswith("project") and op.endswith("back"):
        gproj, rec, rot, _sh, interp, os_, cut = cpu
        wide = oracle.scatter_wide(op, cpu)[0] if gproj.dtype == torch.complex64 else None
        n = gproj.shape[-2]
        if rec.shape[-2] != _rec_box(n, os_):
            return {0: (None, _amax(gproj), wide)}
        return {0: (unit_weight_volume(oracle, three, gproj, rot, interp, os_, cut), _amax(gproj), wide)}
    return {}


def check_scatter(op, got, args, oracle, label):
    """The per-cell bar for every scatter volume in `got` (a tuple of the op's outputs)."""
    got = (got,) if isinstance(got, torch.Tensor) else got
    for k, (U, vmax, exact) in scatter_cells(op, args, oracle).items():
        assert exact is not None, "check_scatter takes fp32 inputs"
        check_cells(got[k].detach().cpu(), exact, U, vmax, f"{label} output {k}")


def check_cells(got, exp, U, vmax, label):
    """Per-cell scatter bar (module docstring)."""
    g = torch.view_as_real(got) if got.is_complex() else got.unsqueeze(-1)
    e = torch.view_as_real(exp) if exp.is_complex() else exp.unsqueeze(-1)
    untouched = (e == 0).all(-1)
    stray = untouched & (g != 0).any(-1)
    if stray.any():
        first = tuple(int(i) for i in stray.nonzero()[0])
        raise AssertionError(f"{label}: {int(stray.sum())} cells are nonzero where the oracle's are exactly 0 "
                             f"(first at {first})")
    if U is None or vmax == 0.0:
        return
    d = (g.double() - e.double()).norm(dim=-1)
    scale = vmax * U.double()
    tol = CELL_TOL[real_dtype(got)]
    bad = d > tol * scale
    if bad.any():
        ratio = torch.where(scale > 0, d / scale.clamp_min(1e-300), torch.where(d > 0, float("inf"), 0.0))
        worst = tuple(int(i) for i in (ratio == ratio.max()).nonzero()[0])
        raise AssertionError(f"{label}: {int(bad.sum())} cells exceed {tol:.0e} * vmax * U; worst |d| / (vmax U) "
                             f"= {ratio.max().item():.3e} at {worst} (U {U[worst].item():.3e}, got {got[worst].item()}, "
                             f"expected {exp[worst].item()})")


def check_outputs(op, got, expected, has_shifts, label="", cells=None):
    """Compare a tuple of outputs with the expected ones under the op's bar; `cells`
    (from scatter_cells) adds the per-cell check of the scatter volumes."""
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
        # a scatter volume with fp32 inputs is compared with the exact sum of the reference's taps:
        # the oracle's own fp32 sum, in one order as the reference's atomics, departs from it with
        # the number of contributions per cell (2.2e-4 rel-L2 for 66000 poses of unit-range weights)
        exact = cells[k][2] if (cells and k in cells and not gather) else None
        err = rel_l2(g, e if exact is None else exact)
        assert err <= tol, f"{label} output {k}: relative L2 {err:.3e} > {tol:.0e}"
        if cells and k in cells:
            U, vmax, exact = cells[k]
            check_cells(g, e if exact is None else exact, U, vmax, f"{label} output {k}")
