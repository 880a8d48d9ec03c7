"""The HIP library, called through its C ABI, against the reference's golden
vectors (tests/golden/*.npz: one call of a reference CPU op each, compiled
from the reference sources and run on one thread).

Every op, linear and cubic, oversampling 1 / 1.5 / 2, with and without
shifts and weights, broadcast rotations/shifts, radius cutoffs, box edges,
impulse volumes and complex128.  Bar: tests/parity.py.
"""
import os

import pytest

from tests.golden.cases import build_args
from tests.parity import check_outputs, scatter_cells
from tests.test_oracle_golden import GOLDEN, load_fixture

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p)[:-4] for p in GOLDEN])
def test_hip_matches_reference_golden(path, hip, oracle):
    case, tensors, expected = load_fixture(path)
    args = build_args(case, tensors)
    print(f"[golden] {case['name']} op={case['op']} dtype={case['dtype']}", flush=True)
    got = getattr(hip, case["op"])(*args)
    check_outputs(case["op"], got, expected, has_shifts=tensors.get("shifts") is not None, label=case["name"],
                  cells=scatter_cells(case["op"], args, oracle))
