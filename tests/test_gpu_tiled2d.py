"""The fp32 2D operators at pose counts that split the tile-owner work into pose ranges.

Rotation poses take the tiled kernels: the scatter for backproject_2d_forw
and project_2d_back's reconstruction gradient, the gather for
project_2d_forw, project_2d_back's rotation/shift gradients and
backproject_2d_back.  Both split every tile's poses into ranges of >= 128
when there are few tiles; the random and golden cases have too few poses for
that.  These cases run hundreds of poses through the C ABI
against the oracle, with every third pose matrix scaled (those take the
per-pixel kernel), broadcast rotations, cutoffs inside and beyond the disc and
oversampling factors that leave the tile grid ragged.  Bar: tests/parity.py.
"""
import pytest

from tests.golden.cases import _case, make_inputs
from tests.parity import check_outputs, scatter_cells

pytestmark = pytest.mark.gpu


def _cases():
    out = []
    seed = 90210
    for op in ("backproject_2d_forw", "project_2d_back", "project_2d_forw", "backproject_2d_back"):
        for interp in ("linear", "cubic"):
            for n, os_, cut, P, B, B_rot in ((48, 2.0, None, 700, 2, 2), (64, 1.5, 20.0, 400, 1, 1),
                                             (40, 3.0, 1000.0, 300, 3, 1), (32, 0.75, 9.5, 513, 1, 1)):
                seed += 1
                out.append(_case(f"tiled2d_{op}_{interp}_n{n}_os{os_:g}_P{P}", op, interp=interp, os=os_, cutoff=cut,
                                 B=B, P=P, n=n, B_rot=B_rot, seed=seed, weights=(seed % 2 == 0)))
    return out


CASES = _cases()


def _scale_some(args, case):
    """Scale every third pose matrix by 1.05 (not a rotation: the per-pixel path)."""
    idx = 2
    r = args[idx].detach().clone()
    r[:, ::3] *= 1.05
    args[idx] = r.requires_grad_(args[idx].requires_grad)
    return args


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_tiled2d_matches_oracle(case, hip, oracle):
    args, tensors = make_inputs(case)
    args = _scale_some(args, case)
    print(f"[tiled2d] {case['name']} B={case['B']} B_rot={case['B_rot']}", flush=True)
    got = getattr(hip, case["op"])(*args)
    exp = getattr(oracle, case["op"])(*args)
    check_outputs(case["op"], got, exp, has_shifts=tensors.get("shifts") is not None, label=case["name"],
                  cells=scatter_cells(case["op"], args, oracle))
