"""The Catmull-Rom weight functions of tp_device.hh on the host.

`tests/cubic_weights_check.hip` is built with hipcc for the host only, with the
library's floating-point flags, and walks every float f in [0, 1]:

* `cubic_w_tap(f, j)`, which evaluates only tap j's piece of the weight, must
  equal `cubic_w(f - (j - 1))` (the reference's piecewise formula,
  csrc/cpu/common/cubic_kernels.h:25-43) bit for bit, in float and in double;
* the fp32 polynomials `cubic_w_fast` / `cubic_dw_fast` of the gradient sums must
  stay within 4 ulps (relative, where the weight is at least 1e-6) and 2.5e-7
  (absolute) of the piecewise weight and derivative (cubic_kernels.h:50-67)
  evaluated in double.
"""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRC = os.path.join(HERE, "cubic_weights_check.hip")
HIP_SRC = os.path.join(ROOT, "torch-projectors_amd", "csrc", "hip")
INCLUDE = os.path.join(ROOT, "include")
ULP = 2.0 ** -24


def _hipcc():
    for c in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if c and os.path.exists(c):
            return c
    return None


def test_cubic_weight_pieces_and_polynomials(tmp_path):
    hipcc = _hipcc()
    if hipcc is None:
        pytest.skip("hipcc not found")
    exe = str(tmp_path / "cubic_weights_check")
    subprocess.run([hipcc, "--cuda-host-only", "-O2", "-std=c++17", "-ffp-contract=off", "-fno-fast-math",
                    "-I", HIP_SRC, "-I", INCLUDE, "-o", exe, SRC, "-lpthread"],
                   check=True, capture_output=True, timeout=600)
    out = subprocess.run([exe], check=True, capture_output=True, text=True, timeout=900).stdout.split()
    vals = {out[i]: float(out[i + 1]) for i in range(0, len(out) - 1, 2)}
    assert vals["values"] == 0x3F800001  # every float in [0, 1]
    assert vals["tap_mismatch_f32"] == 0
    assert vals["tap_mismatch_f64"] == 0
    assert vals["w_fast_rel"] <= 4 * ULP, vals
    assert vals["dw_fast_rel"] <= 4 * ULP, vals
    assert vals["w_fast_abs"] <= 2.5e-7, vals
    assert vals["dw_fast_abs"] <= 2.5e-7, vals
