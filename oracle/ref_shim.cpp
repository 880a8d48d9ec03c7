// TEST INFRASTRUCTURE — NOT PART OF THE PRODUCT.
//
// Registers the reference's own CPU kernels (compiled from
// /root/reference/csrc/cpu/**, unmodified) under the dispatcher namespace
// `torch_projectors_ref`, so that they can be loaded next to the product's
// `torch_projectors` namespace.  The schemas are those of the reference
// (csrc/torch_projectors.cpp:23-36); only the namespace differs.  Built by
// oracle/build_ref.py into oracle/_ref/ (git-ignored); used by
// tests/golden/make_golden.py, the oracle cross-check test and, when present,
// bench.py's cpu_baseline leg.
#include <torch/library.h>

#include "cpu/2d/backprojection_2d_kernels.h"
#include "cpu/2d/projection_2d_kernels.h"
#include "cpu/3d/backprojection_2d_to_3d_kernels.h"
#include "cpu/3d/projection_3d_to_2d_kernels.h"

TORCH_LIBRARY(torch_projectors_ref, m) {
    m.def("project_2d_forw(Tensor reconstruction, Tensor rotations, Tensor? shifts, int[] output_shape, str interpolation, float oversampling, float? fourier_radius_cutoff) -> Tensor");
    m.def("project_2d_back(Tensor grad_projections, Tensor reconstruction, Tensor rotations, Tensor? shifts, str interpolation, float oversampling, float? fourier_radius_cutoff) -> (Tensor, Tensor, Tensor)");
    m.def("backproject_2d_forw(Tensor projections, Tensor? weights, Tensor rotations, Tensor? shifts, str interpolation, float oversampling, float? fourier_radius_cutoff) -> (Tensor, Tensor)");
    m.def("backproject_2d_back(Tensor grad_data_rec, Tensor? grad_weight_rec, Tensor projections, Tensor? weights, Tensor rotations, Tensor? shifts, str interpolation, float oversampling, float? fourier_radius_cutoff) -> (Tensor, Tensor, Tensor, Tensor)");
    m.def("project_3d_to_2d_forw(Tensor reconstruction, Tensor rotations, Tensor? shifts, int[] output_shape, str interpolation, float oversampling, float? fourier_radius_cutoff) -> Tensor");
    m.def("project_3d_to_2d_back(Tensor grad_projections, Tensor reconstruction, Tensor rotations, Tensor? shifts, str interpolation, float oversampling, float? fourier_radius_cutoff) -> (Tensor, Tensor, Tensor)");
    m.def("backproject_2d_to_3d_forw(Tensor projections, Tensor? weights, Tensor rotations, Tensor? shifts, str interpolation, float oversampling, float? fourier_radius_cutoff) -> (Tensor, Tensor)");
    m.def("backproject_2d_to_3d_back(Tensor grad_data_rec, Tensor? grad_weight_rec, Tensor projections, Tensor? weights, Tensor rotations, Tensor? shifts, str interpolation, float oversampling, float? fourier_radius_cutoff) -> (Tensor, Tensor, Tensor, Tensor)");
}

TORCH_LIBRARY_IMPL(torch_projectors_ref, CPU, m) {
    m.impl("project_2d_forw", &project_2d_forw_cpu);
    m.impl("project_2d_back", &project_2d_back_cpu);
    m.impl("backproject_2d_forw", &backproject_2d_forw_cpu);
    m.impl("backproject_2d_back", &backproject_2d_back_cpu);
    m.impl("project_3d_to_2d_forw", &project_3d_to_2d_forw_cpu);
    m.impl("project_3d_to_2d_back", &project_3d_to_2d_back_cpu);
    m.impl("backproject_2d_to_3d_forw", &backproject_2d_to_3d_forw_cpu);
    m.impl("backproject_2d_to_3d_back", &backproject_2d_to_3d_back_cpu);
}
