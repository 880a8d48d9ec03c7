"""The HIP library (C ABI) against the oracle on random configurations.

The same seeded configuration generator as tests/test_oracle_ref_random.py
(where the oracle is pinned bit for bit to the reference's compiled CPU
kernels), plus empty pose sets and cutoffs of +inf, NaN and beyond any int
(the tiled kernels cap each row's columns by the disc only where that cap is
a finite int), 3D scatters with enough poses for the per-call pose bins, odd projection
sizes, and calls of 66000 poses (past the bins' 16-bit lists).
Bar: tests/parity.py.
"""
import pytest

from tests.golden.cases import make_inputs
from tests.parity import check_outputs, scatter_cells
from tests.random_cases import (binned_cases, large_shift_cases, many_pose_cases, nonfinite_cutoff_cases, odd_cases,
                                random_cases, reflect_cases, reflect_poses, scale_poses)

pytestmark = pytest.mark.gpu

CASES = (random_cases(160, seed=424242) + random_cases(40, seed=777, min_p=0) + nonfinite_cutoff_cases()
         + binned_cases() + odd_cases() + many_pose_cases()
         + large_shift_cases() + reflect_cases())


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_hip_matches_oracle_random(case, hip, oracle):
    args, tensors = make_inputs(case)
    if case["scaled"]:
        args = scale_poses(args, case)
    if case.get("reflect"):
        args = reflect_poses(args, case)
    print(f"[random] {case['name']} n={case['n']} os={case['os']} cut={case['cutoff']} P={case['P']}", flush=True)
    got = getattr(hip, case["op"])(*args)
    exp = getattr(oracle, case["op"])(*args)
    check_outputs(case["op"], got, exp, has_shifts=tensors.get("shifts") is not None, label=case["name"],
                  cells=scatter_cells(case["op"], args, oracle))
