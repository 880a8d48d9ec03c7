"""Pose matrices other than rotations through the tiled kernels (C ABI against the oracle).

The reference treats every pose matrix alike (cpu/3d/projection_3d_to_2d_kernels.cpp:180-188,
cpu/2d/projection_2d_kernels.cpp:173-178).  The tiled kernels take every matrix whose first two
columns (3D) or two columns (2D) have singular values in [0.5, 2] (scaled, anisotropically
magnified, sheared); the per-pixel kernels take the rest (stronger scalings, degenerate matrices).
These cases mix all of them in one call, and run calls whose poses all enlarge (samples beyond the
unit-scale radius: the forward's wider tile grid, up to twice as far out) or all shrink.  Bar: tests/parity.py, with the
per-cell check of the scatter volumes.
"""
import math

import pytest
import torch

from tests.golden.cases import _case, make_inputs
from tests.parity import check_outputs, scatter_cells

pytestmark = pytest.mark.gpu

ROT_ARG = {"project_3d_to_2d_forw": 1, "project_2d_forw": 1, "project_3d_to_2d_back": 2, "project_2d_back": 2,
           "backproject_2d_to_3d_forw": 2, "backproject_2d_forw": 2,
           "backproject_2d_to_3d_back": 4, "backproject_2d_back": 4}


def _classes(dim):
    """Maps R -> pose matrix, and whether the tiled kernels take the result."""
    eye = torch.eye(dim, dtype=torch.float64)
    shear = eye.clone()
    shear[0, 1] = 0.15
    aniso = torch.diag(torch.tensor([1.03, 0.97, 1.0][:dim], dtype=torch.float64))

    def parallel(R):  # columns 0 and 1 equal: a degenerate matrix
        R = R.clone()
        R[..., :, 1] = R[..., :, 0]
        return R

    strong = torch.diag(torch.tensor([1.8, 0.55, 1.0][:dim], dtype=torch.float64))
    return [(lambda R: R, True), (lambda R: 1.02 * R, True), (lambda R: 0.85 * R, True), (lambda R: 1.2 * R, True),
            (lambda R: aniso @ R, True), (lambda R: shear @ R, True), (lambda R: R @ shear, True),
            (lambda R: 1.4 * R, True), (lambda R: 0.6 * R, True), (lambda R: 1.9 * R, True),
            (lambda R: strong @ R, True),
            (lambda R: 2.3 * R, False), (lambda R: 0.4 * R, False), (parallel, False)]


def _apply(args, case, mode):
    idx = ROT_ARG[case["op"]]
    rot = args[idx]
    dim = rot.shape[-1]
    r = rot.detach().double().clone()
    classes = _classes(dim)
    if mode == "mixed":
        for p in range(r.shape[1]):
            f, _ = classes[p % len(classes)]
            r[:, p] = f(r[:, p])
    else:
        s = {"enlarge": 1.2, "shrink": 0.85, "enlarge_strong": 1.9, "shrink_strong": 0.55}[mode]
        r = s * r
    args[idx] = r.to(rot.dtype).requires_grad_(rot.requires_grad)
    return args


CASES = []
seed = 4400
for op in ROT_ARG:
    three = "3d" in op
    for mode in ("mixed", "enlarge", "shrink", "enlarge_strong", "shrink_strong"):
        for interp in ("linear", "cubic"):
            seed += 1
            n = (40 if interp == "linear" else 24) if three else 48
            P = 27 if mode == "mixed" else 9
            c = _case(f"{op}_{mode}_{interp}", op, interp=interp, os=2.0, n=n, P=P, B=1, seed=seed)
            c["mode"] = mode
            CASES.append(c)
    seed += 1
    c = _case(f"{op}_mixed_cut_bcast", op, os=1.5, n=32 if three else 48, P=18, B=2, B_rot=1, cutoff=11.0, seed=seed)
    c["mode"] = "mixed"
    CASES.append(c)


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_pose_classes_match_oracle(case, hip, oracle):
    args, tensors = make_inputs(case)
    args = _apply(args, case, case["mode"])
    print(f"[poses] {case['name']}", flush=True)
    got = getattr(hip, case["op"])(*args)
    exp = getattr(oracle, case["op"])(*args)
    check_outputs(case["op"], got, exp, has_shifts=tensors.get("shifts") is not None, label=case["name"],
                  cells=scatter_cells(case["op"], args, oracle))


def test_pose_class_predicate_bounds():
    """The classes above sit where the tests assume: singular values of the first two columns."""
    for dim in (2, 3):
        g = torch.Generator().manual_seed(dim)
        q = torch.linalg.qr(torch.randn(dim, dim, generator=g, dtype=torch.float64))[0]
        for f, tiled in _classes(dim):
            sv = torch.linalg.svdvals(f(q)[:, :2])
            inside = bool((sv >= 0.5 - 1e-9).all() and (sv <= 2.0 + 1e-9).all())
            assert inside == tiled, (dim, sv)
        assert math.isclose(float(torch.linalg.svdvals(1.02 * q[:, :2]).max()), 1.02)
