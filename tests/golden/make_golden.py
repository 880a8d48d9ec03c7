"""Write the golden vectors in tests/golden/*.npz.

Inputs are small seeded tensors; outputs come from the reference's own CPU
kernels (csrc/cpu/**, compiled unmodified by oracle/build_ref.py into
oracle/_ref/ and registered as torch.ops.torch_projectors_ref), run with one
thread so that their scatter sums have a fixed order.  Each file holds one
call: `meta` (JSON: op, non-tensor arguments, requires_grad flags), the input
tensors `in_<name>` and the outputs `out_<k>`.

Run in the build container (needs /root/reference):
    python oracle/build_ref.py && python tests/golden/make_golden.py
"""
import json
import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from tests.golden.cases import CASES, make_inputs  # noqa: E402


def to_np(t):
    return t.detach().cpu().numpy()


def main():
    from oracle import oracle as O
    ref = O.ref_ops()
    if ref is None:
        raise SystemExit("oracle/_ref/libtp_ref.so missing: run python oracle/build_ref.py first")
    torch.set_num_threads(1)
    for old in os.listdir(HERE):
        if old.endswith(".npz"):
            os.remove(os.path.join(HERE, old))
    total = 0
    for case in CASES:
        args, tensors = make_inputs(case)
        op = getattr(ref, case["op"])
        outs = op(*args)
        if isinstance(outs, torch.Tensor):
            outs = (outs,)
        payload = {f"in_{k}": to_np(v) for k, v in tensors.items() if v is not None}
        for k, o in enumerate(outs):
            payload[f"out_{k}"] = to_np(o)
        payload["meta"] = np.array(json.dumps(case))
        path = os.path.join(HERE, case["name"] + ".npz")
        np.savez_compressed(path, **payload)
        total += os.path.getsize(path)
    print(f"wrote {len(CASES)} fixtures, {total / 1e6:.2f} MB")


if __name__ == "__main__":
    main()
