"""Oversampling factors that are not float values (1.1, 1.3, 1.7, 2.2).

The tiled 3D kernels form c*os in float when float(os) == os (every factor
of the golden and random cases) and in double otherwise, as the reference
does (double product rounded to float); these cases take the second path.
Bar: tests/parity.py.
"""
import pytest

from tests.golden.cases import _case, make_inputs
from tests.parity import check_outputs, scatter_cells

pytestmark = pytest.mark.gpu


def _cases():
    out = []
    seed = 555000
    for op in ("project_3d_to_2d_forw", "backproject_2d_to_3d_forw", "project_3d_to_2d_back",
               "backproject_2d_to_3d_back", "project_2d_forw", "backproject_2d_forw"):
        for interp in ("linear", "cubic"):
            for os_, cut in ((1.1, None), (1.3, 7.5), (1.7, None), (2.2, 11.0)):
                seed += 1
                out.append(_case(f"osx_{op}_{interp}_os{os_:g}", op, interp=interp, os=os_, cutoff=cut, B=2, P=7,
                                 n=24, seed=seed, weights=(seed % 2 == 0)))
    return out


CASES = _cases()


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_inexact_oversampling(case, hip, oracle):
    args, tensors = make_inputs(case)
    print(f"[osx] {case['name']}", flush=True)
    got = getattr(hip, case["op"])(*args)
    exp = getattr(oracle, case["op"])(*args)
    check_outputs(case["op"], got, exp, has_shifts=tensors.get("shifts") is not None, label=case["name"],
                  cells=scatter_cells(case["op"], args, oracle))
