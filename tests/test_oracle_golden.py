"""The oracle against the reference's golden vectors (CPU only).

Each fixture in tests/golden/ holds one call of a reference CPU op (compiled
from the reference sources, one thread).  The oracle, also run on one thread,
must reproduce every output bit for bit: same sample coordinates, stencils,
Friedel flips, clamps, per-tap products and summation order.
"""
import glob
import json
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.golden.cases import build_args

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))


def load_fixture(path):
    z = np.load(path, allow_pickle=False)
    case = json.loads(str(z["meta"]))
    tensors = {k[3:]: torch.from_numpy(z[k].copy()) for k in z.files if k.startswith("in_")}
    outs = [torch.from_numpy(z[k].copy()) for k in sorted((k for k in z.files if k.startswith("out_")),
                                                          key=lambda s: int(s[4:]))]
    for name in ("shifts", "weights", "grad_weight_rec"):
        tensors.setdefault(name, None)
    return case, tensors, outs


def test_fixture_set_is_complete():
    ops = {json.loads(str(np.load(p)["meta"]))["op"] for p in GOLDEN}
    assert ops == set(O.OPS)
    assert len(GOLDEN) >= 60


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p)[:-4] for p in GOLDEN])
def test_oracle_matches_reference_golden(path):
    case, tensors, expected = load_fixture(path)
    args = build_args(case, tensors)
    got = getattr(O, case["op"])(*args, num_threads=1)
    if isinstance(got, torch.Tensor):
        got = (got,)
    assert len(got) == len(expected)
    for k, (g, e) in enumerate(zip(got, expected)):
        assert g.shape == e.shape, (k, g.shape, e.shape)
        assert g.dtype == e.dtype, (k, g.dtype, e.dtype)
        assert torch.equal(g, e), f"output {k} differs: max |d| = {(g - e).abs().max().item():.3e}"
