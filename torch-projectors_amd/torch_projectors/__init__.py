"""torch_projectors for MI355X (gfx950).

Differentiable Fourier-space projection operators with the public API of the
reference package (torch_projectors/__init__.py:28-29): the dispatcher ops
`torch.ops.torch_projectors.*` are implemented by hand-written HIP kernels in
libtorch_projectors_hip.so and registered under PyTorch-ROCm's GPU key by
_C.so.  Importing fails loudly when the native library has not been built.
"""
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_EXT = os.path.join(_HERE, "_C.so")
LIBRARY_PATH = os.path.join(_HERE, "libtorch_projectors_hip.so")

if not os.path.exists(_EXT) or not os.path.exists(LIBRARY_PATH):
    raise ImportError(
        "torch_projectors: native library not built (expected _C.so and libtorch_projectors_hip.so in "
        f"{_HERE}); run `python torch-projectors_amd/build.py`")
torch.ops.load_library(_EXT)

from . import ops  # noqa: E402  (registers the autograd stubs)
from .ops import (  # noqa: E402
    backproject_2d_forw,
    backproject_2d_to_3d_back,
    backproject_2d_to_3d_forw,
    project_2d_back,
    project_2d_forw,
    project_3d_to_2d_back,
    project_3d_to_2d_forw,
)

__version__ = "0.1.0+gfx950"

__all__ = ["project_2d_forw", "project_2d_back", "project_3d_to_2d_forw", "project_3d_to_2d_back",
           "backproject_2d_forw", "backproject_2d_to_3d_forw", "backproject_2d_to_3d_back"]
