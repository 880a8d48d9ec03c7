"""The drop-in boundary without a GPU: dispatcher schemas identical to the
reference's, Python-side argument checks with the reference's ValueErrors
(torch_projectors/ops.py), and no silent CPU path."""
import pytest
import torch

import torch_projectors as tp

# csrc/torch_projectors.cpp:23-36 of the reference
REFERENCE_SCHEMAS = {
    "project_2d_forw": "project_2d_forw(Tensor reconstruction, Tensor rotations, Tensor? shifts, int[] output_shape, str interpolation, float oversampling, float? fourier_radius_cutoff) -> Tensor",
    "project_2d_back": "project_2d_back(Tensor grad_projections, Tensor reconstruction, Tensor rotations, Tensor? shifts, str interpolation, float oversampling, float? fourier_radius_cutoff) -> (Tensor, Tensor, Tensor)",
    "backproject_2d_forw": "backproject_2d_forw(Tensor projections, Tensor? weights, Tensor rotations, Tensor? shifts, str interpolation, float oversampling, float? fourier_radius_cutoff) -> (Tensor, Tensor)",
    "backproject_2d_back": "backproject_2d_back(Tensor grad_data_rec, Tensor? grad_weight_rec, Tensor projections, Tensor? weights, Tensor rotations, Tensor? shifts, str interpolation, float oversampling, float? fourier_radius_cutoff) -> (Tensor, Tensor, Tensor, Tensor)",
    "project_3d_to_2d_forw": "project_3d_to_2d_forw(Tensor reconstruction, Tensor rotations, Tensor? shifts, int[] output_shape, str interpolation, float oversampling, float? fourier_radius_cutoff) -> Tensor",
    "project_3d_to_2d_back": "project_3d_to_2d_back(Tensor grad_projections, Tensor reconstruction, Tensor rotations, Tensor? shifts, str interpolation, float oversampling, float? fourier_radius_cutoff) -> (Tensor, Tensor, Tensor)",
    "backproject_2d_to_3d_forw": "backproject_2d_to_3d_forw(Tensor projections, Tensor? weights, Tensor rotations, Tensor? shifts, str interpolation, float oversampling, float? fourier_radius_cutoff) -> (Tensor, Tensor)",
    "backproject_2d_to_3d_back": "backproject_2d_to_3d_back(Tensor grad_data_rec, Tensor? grad_weight_rec, Tensor projections, Tensor? weights, Tensor rotations, Tensor? shifts, str interpolation, float oversampling, float? fourier_radius_cutoff) -> (Tensor, Tensor, Tensor, Tensor)",
}


@pytest.mark.parametrize("name", sorted(REFERENCE_SCHEMAS))
def test_schema_matches_reference(name):
    schema = str(getattr(torch.ops.torch_projectors, name).default._schema)
    assert schema == "torch_projectors::" + REFERENCE_SCHEMAS[name]


@pytest.mark.parametrize("name", sorted(REFERENCE_SCHEMAS))
def test_gpu_kernel_registered_and_no_cpu_kernel(name):
    op = f"torch_projectors::{name}"
    assert torch._C._dispatch_has_kernel_for_dispatch_key(op, "CUDA")
    assert not torch._C._dispatch_has_kernel_for_dispatch_key(op, "CPU")


def test_public_names():
    assert tp.__all__ == ["project_2d_forw", "project_2d_back", "project_3d_to_2d_forw", "project_3d_to_2d_back",
                          "backproject_2d_forw", "backproject_2d_to_3d_forw", "backproject_2d_to_3d_back"]


def test_cpu_tensors_fail_loudly():
    rec = torch.zeros(1, 8, 8, 5, dtype=torch.complex64)
    rot = torch.eye(3).reshape(1, 1, 3, 3)
    with pytest.raises(NotImplementedError):
        tp.project_3d_to_2d_forw(rec, rot)


def c64(*shape):
    return torch.zeros(*shape, dtype=torch.complex64)


@pytest.mark.parametrize("call,msg", [
    (lambda: tp.project_3d_to_2d_forw(c64(1, 7, 7, 4), torch.eye(3)[None, None]), "must be even"),
    (lambda: tp.project_3d_to_2d_forw(c64(1, 8, 8, 4), torch.eye(3)[None, None]), "shape mismatch"),
    (lambda: tp.project_3d_to_2d_forw(c64(8, 8, 5), torch.eye(3)[None, None]), "4D tensor"),
    (lambda: tp.project_3d_to_2d_forw(c64(1, 8, 8, 5), torch.eye(3)[None, None], output_shape=(6, 4)),
     "must be square"),
    (lambda: tp.project_3d_to_2d_forw(c64(1, 8, 8, 5), torch.eye(3)[None, None], output_shape=(5, 5)),
     "must be even"),
    (lambda: tp.project_2d_forw(c64(8,), torch.eye(2)[None, None]), "at least 2 dimensions"),
    (lambda: tp.project_2d_forw(c64(1, 10, 5), torch.eye(2)[None, None]), "shape mismatch"),
    (lambda: tp.backproject_2d_forw(c64(1, 8, 5), torch.eye(2)[None, None]), "4D tensor"),
    (lambda: tp.backproject_2d_to_3d_forw(c64(1, 1, 8, 5), torch.eye(3)[None, None],
                                          weights=torch.zeros(1, 1, 8, 4)), "must match projections shape"),
    (lambda: tp.backproject_2d_to_3d_forw(c64(1, 1, 8, 5), torch.eye(3)[None, None],
                                          weights=torch.zeros(1, 1, 8, 5, dtype=torch.int32)), "real-valued"),
    (lambda: tp.project_3d_to_2d_forw(c64(2, 8, 8, 5), torch.eye(3).expand(3, 1, 3, 3)), "Batch size of rotations"),
])
def test_python_argument_checks(call, msg):
    with pytest.raises(ValueError, match=msg):
        call()
