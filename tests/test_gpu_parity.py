"""The HIP library (C ABI) against the CPU oracle on seeded medium-size inputs.

The golden fixtures pin tiny boxes; these cases span many 16^3 tiles of the
tile-owner kernels, both pose classes (rotations take the tiled path; scaled
matrices take the per-pixel kernels), batch broadcasting, cutoffs, both
interpolations and oversampling factors, for all eight ops.  Bar:
tests/parity.py (gathers bit-identical without shifts).
"""
import pytest
import torch

from tests.golden.cases import _case, make_inputs
from tests.parity import check_outputs, scatter_cells

pytestmark = pytest.mark.gpu

OPS3 = ["project_3d_to_2d_forw", "project_3d_to_2d_back", "backproject_2d_to_3d_forw", "backproject_2d_to_3d_back"]
OPS2 = ["project_2d_forw", "project_2d_back", "backproject_2d_forw", "backproject_2d_back"]


def _scale_some_poses(args, case):
    """Turn every third rotation into a scaled matrix (not a rotation)."""
    idx = {"project_3d_to_2d_forw": 1, "project_2d_forw": 1, "project_3d_to_2d_back": 2, "project_2d_back": 2,
           "backproject_2d_to_3d_forw": 2, "backproject_2d_forw": 2,
           "backproject_2d_to_3d_back": 4, "backproject_2d_back": 4}[case["op"]]
    rot = args[idx]
    rg = rot.requires_grad
    r = rot.detach().clone()
    r[:, ::3] *= 1.07
    args[idx] = r.requires_grad_(rg)
    return args


CASES = []
for op in OPS3:
    CASES += [
        _case(f"{op}_lin_os2", op, n=64, P=40, B=1, os=2.0, seed=11),
        _case(f"{op}_lin_os2_noshift", op, n=48, P=24, B=1, os=2.0, shifts=False, seed=12),
        _case(f"{op}_cub_os2", op, interp="cubic", n=32, P=20, B=1, os=2.0, seed=13),
        _case(f"{op}_lin_os1.5_cut", op, n=40, P=24, B=2, B_rot=1, os=1.5, cutoff=13.0, seed=14),
        _case(f"{op}_cub_os1_bcast", op, interp="cubic", n=32, P=16, B=2, B_rot=1, B_shift=1, os=1.0, seed=15),
        _case(f"{op}_lin_os2_mixed", op, n=48, P=30, B=1, os=2.0, seed=16, special=True),
        _case(f"{op}_lin_os2_noweights", op, n=40, P=16, B=1, os=2.0, weights=False, grad_weight_rec=False,
              rg_rot=False, seed=17),
        _case(f"{op}_cub_os2_bigcut", op, interp="cubic", n=24, P=12, B=1, os=2.0, cutoff=40.0, seed=18),
    ]
for op in OPS2:
    CASES += [
        _case(f"{op}_lin_os2", op, n=64, P=64, B=2, os=2.0, seed=21),
        _case(f"{op}_cub_os2_cut", op, interp="cubic", n=64, P=48, B=2, B_rot=1, os=2.0, cutoff=16.0, seed=22),
        _case(f"{op}_lin_os1.5_mixed", op, n=48, P=40, B=1, os=1.5, seed=23),
    ]


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_hip_matches_oracle(case, hip, oracle):
    args, tensors = make_inputs(case)
    if "mixed" in case["name"]:
        args = _scale_some_poses(args, case)
    print(f"[parity] {case['name']}", flush=True)
    got = getattr(hip, case["op"])(*args)
    exp = getattr(oracle, case["op"])(*args)
    check_outputs(case["op"], got, exp, has_shifts=tensors.get("shifts") is not None, label=case["name"],
                  cells=scatter_cells(case["op"], args, oracle))
