"""The oracle against the reference's own compiled CPU kernels on random configurations (CPU).

oracle/_ref is built from the reference sources in the build container
(oracle/build_ref.py); where it is absent these tests skip.  Both sides run on
one thread, so every output must be bit-identical, as for the golden vectors.
"""
import pytest
import torch

from oracle import oracle as O
from tests.golden.cases import make_inputs
from tests.random_cases import (large_shift_cases, nonfinite_cutoff_cases, odd_cases, random_cases, reflect_cases,
                                reflect_poses, scale_poses)

CASES = (random_cases(160, seed=424242) + random_cases(40, seed=777, min_p=0) + nonfinite_cutoff_cases()
         + odd_cases() + large_shift_cases() + reflect_cases())


@pytest.fixture(scope="module")
def ref():
    ops = O.ref_ops()
    if ops is None:
        pytest.skip("oracle/_ref (the reference's compiled CPU kernels) is not built here")
    return ops


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_oracle_matches_reference_build(case, ref):
    args, _ = make_inputs(case)
    if case["scaled"]:
        args = scale_poses(args, case)
    if case.get("reflect"):
        args = reflect_poses(args, case)
    threads = torch.get_num_threads()
    torch.set_num_threads(1)
    try:
        exp = getattr(ref, case["op"])(*args)
    finally:
        torch.set_num_threads(threads)
    got = getattr(O, case["op"])(*args, num_threads=1)
    if isinstance(got, torch.Tensor):
        got, exp = (got,), (exp,)
    assert len(got) == len(exp)
    for k, (g, e) in enumerate(zip(got, exp)):
        assert g.shape == e.shape, (k, g.shape, e.shape)
        assert g.dtype == e.dtype, (k, g.dtype, e.dtype)
        assert torch.equal(g, e), f"output {k}: max |d| = {(g - e).abs().max().item():.3e}"
        if case["name"].startswith("cut"):
            assert e.numel() == 0 or torch.count_nonzero(e) > 0, f"output {k} is all zero"
