"""The cubic 3D kernels' carried sample windows, through the C ABI, against the oracle.

The cubic tiled scatter (backprojection and the reconstruction gradient of project_3d_to_2d_back)
and the cubic tiled forward do not deposit a wave's last, partly filled window of samples at the
end of a batch: the next batch's samples fill it. A wave keeps two pose sets for that (batch j in
set j mod 2), deposits a window that would still hold samples of batch j - 1 when batch j ends,
runs an empty block for a batch without rows while a window is carried, and deposits every window
at the end of a pass or cull phase. The cases below walk those paths:

* pose counts on and around the batch sizes (4 poses per scatter batch, 5 per forward batch;
  4 waves per workgroup) and past the 16 poses from which the scatters use pose bins;
* every pose the same rotation (all batches give a tile the same rows) and poses spread over a
  few degrees (most batches give most tiles nothing);
* more poses than one cull phase holds (the scatter culls 512 per phase, the forward 2048);
* every other matrix scaled (the kernels for tiled poses that are not rotations) and a cutoff.

Bars as tests/parity.py (gathers bit-identical without shifts, 1e-5 with them; scatters 1e-4 and
the per-cell check against the exact sum of the oracle's taps).
"""
import math

import pytest
import torch

from tests.golden.cases import _case, make_inputs
from tests.parity import check_outputs, scatter_cells
from tests.random_cases import scale_poses

pytestmark = pytest.mark.gpu

OPS = ("backproject_2d_to_3d_forw", "project_3d_to_2d_back", "project_3d_to_2d_forw")
ROT_ARG = {"project_3d_to_2d_forw": 1, "project_3d_to_2d_back": 2, "backproject_2d_to_3d_forw": 2}


def _rot_about_z(deg):
    a = math.radians(deg)
    return torch.tensor([[math.cos(a), -math.sin(a), 0.0], [math.sin(a), math.cos(a), 0.0], [0.0, 0.0, 1.0]],
                        dtype=torch.float64)


def _tilted(P, spread_deg, seed):
    """P rotations within `spread_deg` of one tilted orientation."""
    g = torch.Generator().manual_seed(seed)
    base = _rot_about_z(23.0) @ torch.tensor([[1.0, 0.0, 0.0], [0.0, math.cos(0.7), -math.sin(0.7)],
                                               [0.0, math.sin(0.7), math.cos(0.7)]], dtype=torch.float64)
    out = []
    for _ in range(P):
        d = float(torch.rand(1, generator=g)) * spread_deg
        out.append(_rot_about_z(d) @ base)
    return torch.stack(out)


def _cases():
    out = []
    seed = 31000
    for op in OPS:
        for P in (1, 3, 4, 5, 6, 9, 11, 17, 21, 37):
            seed += 1
            out.append(_case(f"carry_{op}_P{P}", op, interp="cubic", os=2.0, B=1, P=P, n=16, seed=seed))
        for kind in ("same", "spread"):
            seed += 1
            c = _case(f"carry_{op}_{kind}", op, interp="cubic", os=2.0, B=1, P=24, n=20, seed=seed)
            c["poses"] = kind
            out.append(c)
        seed += 1
        c = _case(f"carry_{op}_scaled_cut", op, interp="cubic", os=1.5, cutoff=6.5, B=2, P=13, n=20, seed=seed)
        c["scaled"] = True
        out.append(c)
    # more poses than one cull phase: 600 for the scatters (512 a phase), 2100 for the forward
    for op, P in (("backproject_2d_to_3d_forw", 600), ("project_3d_to_2d_back", 600), ("project_3d_to_2d_forw", 2100)):
        seed += 1
        out.append(_case(f"carry_{op}_phases_P{P}", op, interp="cubic", os=2.0, B=1, P=P, n=8, seed=seed))
    return out


CASES = _cases()


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_cubic_carried_windows_match_oracle(case, hip, oracle):
    args, tensors = make_inputs(case)
    op = case["op"]
    if case.get("poses"):
        i = ROT_ARG[op]
        R = args[i].detach()
        P = R.shape[1]
        rots = _tilted(1, 0.0, case["seed"]).expand(P, 3, 3) if case["poses"] == "same" else \
            _tilted(P, 3.0, case["seed"])
        args[i] = rots.to(R.dtype).unsqueeze(0).expand_as(R).contiguous().requires_grad_(R.requires_grad)
    if case.get("scaled"):
        args = scale_poses(args, case)
    print(f"[carry] {case['name']} P={case['P']} n={case['n']} os={case['os']}", flush=True)
    got = getattr(hip, op)(*args)
    exp = getattr(oracle, op)(*args)
    check_outputs(op, got, exp, has_shifts=tensors.get("shifts") is not None, label=case["name"],
                  cells=scatter_cells(op, args, oracle))
