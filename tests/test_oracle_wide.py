"""The double-summed scatter of the oracle (oracle.scatter_wide) against its fp32 one (CPU).

scatter_wide is the per-cell expectation of tests/parity.py `check_cells`.  It
must hold the same taps as the fp32 oracle (which is pinned bit for bit to the
reference): the same cells untouched (exactly 0), and every other cell within
the error of an fp32 summation, 2^-20 * vmax * U (U the cell's sum of |tap
weight|).  A dropped or extra tap, a lost conjugation or a lost x = 0 mirror in
the wide path moves a cell by |v| times a tap weight and fails here.
"""
import pytest
import torch

from oracle import oracle as O
from tests.golden.cases import BPFORW, PBACK, make_inputs
from tests.parity import scatter_cells
from tests.random_cases import random_cases

CASES = [c for c in random_cases(160, seed=31337) if c["op"] in BPFORW + PBACK and c["dtype"] == "f32"]


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_wide_scatter_holds_the_same_taps(case):
    args, _ = make_inputs(case)
    op = case["op"]
    exp = getattr(O, op)(*args, num_threads=1)
    exp = (exp,) if isinstance(exp, torch.Tensor) else exp
    for k, (U, vmax, wide) in scatter_cells(op, args, O).items():
        e = torch.view_as_real(exp[k]) if exp[k].is_complex() else exp[k].unsqueeze(-1)
        w = torch.view_as_real(wide) if wide.is_complex() else wide.unsqueeze(-1)
        assert wide.dtype in (torch.complex128, torch.float64) and wide.shape == exp[k].shape
        assert torch.equal((e == 0).all(-1), (w == 0).all(-1)), f"output {k}: untouched cells differ"
        if U is not None:
            d = (e.double() - w).norm(dim=-1)
            assert (d <= 2.0 ** -20 * vmax * U.double()).all(), f"output {k}: max |d| {d.max().item():.3e}"
