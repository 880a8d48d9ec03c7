// PyTorch dispatcher registration of the MI355X projector library.
//
// Defines the namespace `torch_projectors` with the reference's eight op
// schemas, verbatim (csrc/torch_projectors.cpp:21-37), and registers the HIP
// implementations under the CUDA dispatch key, which is PyTorch-ROCm's GPU
// key (the reference registers its CUDA kernels there,
// csrc/torch_projectors.cpp:77-95).  Each implementation validates its
// arguments with the reference's conditions and messages
// (validate_projection_inputs, cpu/common/projection_utils.h:23-48, and the
// per-op checks in cpu/{2d,3d}/*.cpp), allocates the outputs, and calls the C
// ABI of libtorch_projectors_hip.so on PyTorch's current stream.  No CPU
// kernels are registered: CPU tensors fail in the dispatcher.
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/library.h>
#include <torch/torch.h>

#include <cmath>
#include <string>
#include <tuple>

#include "../../include/torch_projectors_hip.h"

namespace {

using at::Tensor;
using c10::optional;

void validate_inputs(const std::string& interpolation, const Tensor& reconstruction, const Tensor& rotations,
                     const optional<Tensor>& shifts, int64_t rec_dims, int64_t rot_size) {
    TORCH_CHECK(interpolation == "linear" || interpolation == "cubic",
                "Supported interpolation methods: 'linear', 'cubic'");
    TORCH_CHECK(reconstruction.is_complex(), "Reconstruction must be a complex tensor");
    TORCH_CHECK(reconstruction.dim() == rec_dims, "Reconstruction must have " + std::to_string(rec_dims) +
                                                      " dimensions");
    TORCH_CHECK(rotations.dim() == 4 && rotations.size(2) == rot_size && rotations.size(3) == rot_size,
                "Rotations must be (B_rot, P, " + std::to_string(rot_size) + ", " + std::to_string(rot_size) + ")");
    if (shifts.has_value()) {
        TORCH_CHECK(shifts->dim() == 3, "Shifts must be (B_shift, P, 2)");
        TORCH_CHECK(shifts->size(2) == 2, "Shifts must have 2 components (x, y)");
        TORCH_CHECK(shifts->scalar_type() == rotations.scalar_type(), "Shifts and rotations must have the same dtype");
    }
}

void check_shift_batch(const optional<Tensor>& shifts, int64_t B, int64_t P, const char* what) {
    if (!shifts.has_value()) return;
    TORCH_CHECK(shifts->size(0) == B || shifts->size(0) == 1,
                std::string("Batch size of shifts must be 1 or same as ") + what);
    TORCH_CHECK(shifts->size(1) == P, "Number of poses in shifts must match rotations");
}

// Real-valued inputs against the complex input's dtype, as the reference's two
// paths accept them.  Rotations are dispatched as float or double
// (AT_DISPATCH_FLOATING_TYPES, cpu/3d/projection_3d_to_2d_kernels.cpp:126), and
// weights / grad_weight_rec are read through the rotations' type
// (cpu/3d/backprojection_2d_to_3d_kernels.cpp:165-169, :388-397).  Complex64
// calls take the reference's GPU path, which reads rotations, shifts and weights
// as float (cuda/3d/projection_3d_to_2d_kernels.cu:987-988) and raises for
// double; complex128 calls fall back to its CPU code, which also takes float
// rotations: those are widened exactly to double here, the same values the
// CPU code's promotion gives.
void check_real_dtypes(c10::ScalarType cplx, const Tensor& rotations, const optional<Tensor>& weights,
                       const optional<Tensor>& grad_weight_rec = c10::nullopt) {
    const auto rt = rotations.scalar_type();
    TORCH_CHECK(rt == at::kFloat || rt == at::kDouble, "Rotations must be float32 or float64, got ", rt);
    TORCH_CHECK(cplx == at::kComplexDouble || rt == at::kFloat, "A ", cplx,
                " input needs float32 rotations and shifts (the reference's GPU path reads them as float), got ", rt);
    if (weights.has_value())
        TORCH_CHECK(weights->scalar_type() == rt, "Weights must have the rotations' dtype (", rt, "), got ",
                    weights->scalar_type());
    if (grad_weight_rec.has_value())
        TORCH_CHECK(grad_weight_rec->scalar_type() == rt, "grad_weight_rec must have the rotations' dtype (", rt,
                    "), got ", grad_weight_rec->scalar_type());
}

// The kernels read every real-valued input in the complex tensor's value
// type (check_real_dtypes admits only float32 -> float64 widening).
struct Prep {
    Tensor t;
    const void* ptr() const { return t.defined() ? t.data_ptr() : nullptr; }
};
Prep prep(const Tensor& t, c10::ScalarType st, const c10::Device& dev) {
    TORCH_CHECK(t.device() == dev, "all tensors must be on the same GPU (", dev, "), got one on ", t.device());
    return {t.to(st).contiguous()};
}
Prep prep_opt(const optional<Tensor>& t, c10::ScalarType st, const c10::Device& dev) {
    if (!t.has_value()) return {};
    return prep(*t, st, dev);
}

int dtype_code(const Tensor& complex_tensor) {
    const auto st = complex_tensor.scalar_type();
    TORCH_CHECK(st == at::kComplexFloat || st == at::kComplexDouble, "complex64 or complex128 tensors expected, got ",
                st);
    return st == at::kComplexFloat ? TP_F32 : TP_F64;
}

// Opt-in low-precision volume storage (no counterpart in the reference): a
// complex32 reconstruction is read natively by the projection and its backward
// (TP_F16S: every value widened exactly to fp32 on load, complex64 projections
// and fp32 gradient arithmetic); the backward returns the reconstruction
// gradient as complex32, the dtype autograd expects for that input.
bool is_half_volume(const Tensor& reconstruction) { return reconstruction.scalar_type() == at::kComplexHalf; }

int interp_code(const std::string& s) { return s == "cubic" ? TP_CUBIC : TP_LINEAR; }

void* current_stream(const c10::Device& dev) {
    return static_cast<void*>(c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(dev.index()).stream());
}

void check_rc(int rc) { TORCH_CHECK(rc == TP_OK, "torch_projectors HIP backend: ", tp_last_error()); }

int64_t rec_boxsize_for(int64_t n, double os) { return tp_backproject_rec_boxsize(n, os); }

// Gradient outputs for rotations / shifts, gated on requires_grad as in the
// reference (GradientTensors, projection_utils.h:99-132).
struct PoseGrads {
    bool need_rot, need_shift;
    Tensor rot, shift;  // in the working real type
};
PoseGrads pose_grads(const Tensor& rotations, const optional<Tensor>& shifts, const Prep& rot, const Prep& sh) {
    PoseGrads g;
    g.need_rot = rotations.requires_grad();
    g.need_shift = shifts.has_value() && shifts->requires_grad();
    if (g.need_rot) g.rot = at::empty_like(rot.t);
    if (g.need_shift) g.shift = at::empty_like(sh.t);
    return g;
}
Tensor finish_rot(const PoseGrads& g, const Tensor& rotations) {
    if (!g.need_rot) return torch::empty({0}, rotations.options());
    return g.rot.to(rotations.scalar_type());
}
Tensor finish_shift(const PoseGrads& g, const Tensor& rotations, const optional<Tensor>& shifts,
                    const Tensor& like) {
    if (!g.need_shift) return torch::empty({0}, like.options().dtype(rotations.scalar_type()));
    return g.shift.to(shifts->scalar_type());
}

// ------------------------------------------------------------------ forward projection
Tensor project_forw(int dim, const Tensor& reconstruction, const Tensor& rotations, const optional<Tensor>& shifts,
                    at::IntArrayRef output_shape, const std::string& interpolation, double oversampling,
                    const optional<double>& fourier_radius_cutoff) {
    validate_inputs(interpolation, reconstruction, rotations, shifts, dim + 1, dim);
    const int64_t B = reconstruction.size(0);
    const int64_t B_rot = rotations.size(0), P = rotations.size(1);
    TORCH_CHECK(B_rot == B || B_rot == 1, "Batch size of rotations must be 1 or same as reconstruction");
    check_shift_batch(shifts, B, P, "reconstruction");
    TORCH_CHECK(output_shape.size() >= 1, "output_shape must have at least one entry");
    const int64_t n = output_shape[0];
    const auto dev = reconstruction.device();
    c10::hip::HIPGuardMasqueradingAsCUDA guard(dev);
    const bool half = is_half_volume(reconstruction);
    const int dt = half ? TP_F16S : dtype_code(reconstruction);
    const auto cplx = half ? at::kComplexFloat : reconstruction.scalar_type();
    check_real_dtypes(cplx, rotations, c10::nullopt);
    const auto real = c10::toRealValueType(cplx);
    const Tensor rec = reconstruction.contiguous();
    const Prep rot = prep(rotations, real, dev), sh = prep_opt(shifts, real, dev);
    Tensor out = at::empty({B, P, n, n / 2 + 1}, reconstruction.options().dtype(cplx));
    const int has_cut = fourier_radius_cutoff.has_value();
    const double cut = fourier_radius_cutoff.value_or(0.0);
    int rc;
    if (dim == 2)
        rc = tp_project_2d_forw(dt, rec.data_ptr(), B, rec.size(1), rec.size(2), rot.ptr(), B_rot, P, sh.ptr(),
                                sh.t.defined() ? sh.t.size(0) : 1, n, interp_code(interpolation), oversampling,
                                has_cut, cut, out.data_ptr(), current_stream(dev));
    else
        rc = tp_project_3d_to_2d_forw(dt, rec.data_ptr(), B, rec.size(1), rec.size(2), rec.size(3), rot.ptr(), B_rot,
                                      P, sh.ptr(), sh.t.defined() ? sh.t.size(0) : 1, n, interp_code(interpolation),
                                      oversampling, has_cut, cut, out.data_ptr(), current_stream(dev));
    check_rc(rc);
    return out;
}

// ------------------------------------------------------------------ projection backward
std::tuple<Tensor, Tensor, Tensor> project_back(int dim, const Tensor& grad_projections, const Tensor& reconstruction,
                                                const Tensor& rotations, const optional<Tensor>& shifts,
                                                const std::string& interpolation, double oversampling,
                                                const optional<double>& fourier_radius_cutoff) {
    validate_inputs(interpolation, reconstruction, rotations, shifts, dim + 1, dim);
    TORCH_CHECK(grad_projections.is_complex(), "Projections must be a complex tensor");
    TORCH_CHECK(grad_projections.dim() == 4, "Projections must be a 4D tensor (B, P, H, W/2+1)");
    const int64_t B = grad_projections.size(0), P = grad_projections.size(1);
    const int64_t n = grad_projections.size(2), hp = grad_projections.size(3);
    TORCH_CHECK(reconstruction.size(0) == B, "grad_projections and reconstruction batch sizes differ");
    TORCH_CHECK(rotations.size(1) == P, "Number of poses in rotations must match grad_projections");
    const int64_t B_rot = rotations.size(0);
    TORCH_CHECK(B_rot == B || B_rot == 1, "Batch size of rotations must be 1 or same as reconstruction");
    check_shift_batch(shifts, B, P, "reconstruction");
    const bool half = is_half_volume(reconstruction);
    TORCH_CHECK(grad_projections.scalar_type() == (half ? at::kComplexFloat : reconstruction.scalar_type()),
                half ? "grad_projections must be complex64 for a complex32 reconstruction"
                     : "grad_projections and reconstruction must have the same dtype");
    const auto dev = reconstruction.device();
    c10::hip::HIPGuardMasqueradingAsCUDA guard(dev);
    TORCH_CHECK(grad_projections.device() == dev, "all tensors must be on the same GPU");
    const Tensor g = grad_projections.contiguous();
    const Tensor rec = reconstruction.contiguous();
    const int dt = half ? TP_F16S : dtype_code(rec);
    const auto cplx = half ? at::kComplexFloat : rec.scalar_type();
    check_real_dtypes(cplx, rotations, c10::nullopt);
    const auto real = c10::toRealValueType(cplx);
    const Prep rot = prep(rotations, real, dev), sh = prep_opt(shifts, real, dev);
    PoseGrads pg = pose_grads(rotations, shifts, rot, sh);
    Tensor grec = at::empty(rec.sizes(), grad_projections.options());
    const int has_cut = fourier_radius_cutoff.has_value();
    const double cut = fourier_radius_cutoff.value_or(0.0);
    void* grot = pg.need_rot ? pg.rot.data_ptr() : nullptr;
    void* gsh = pg.need_shift ? pg.shift.data_ptr() : nullptr;
    const int64_t Bs = sh.t.defined() ? sh.t.size(0) : 1;
    int rc;
    if (dim == 2)
        rc = tp_project_2d_back(dt, g.data_ptr(), B, P, n, hp, rec.data_ptr(), rec.size(1), rec.size(2), rot.ptr(),
                                B_rot, sh.ptr(), Bs, interp_code(interpolation), oversampling, has_cut, cut,
                                grec.data_ptr(), grot, gsh, current_stream(dev));
    else
        rc = tp_project_3d_to_2d_back(dt, g.data_ptr(), B, P, n, hp, rec.data_ptr(), rec.size(1), rec.size(2),
                                      rec.size(3), rot.ptr(), B_rot, sh.ptr(), Bs, interp_code(interpolation),
                                      oversampling, has_cut, cut, grec.data_ptr(), grot, gsh, current_stream(dev));
    check_rc(rc);
    return {half ? grec.to(at::kComplexHalf) : grec, finish_rot(pg, rotations),
            finish_shift(pg, rotations, shifts, grad_projections)};
}

// ------------------------------------------------------------------ backprojection
std::tuple<Tensor, Tensor> backproject_forw(int dim, const Tensor& projections, const optional<Tensor>& weights,
                                            const Tensor& rotations, const optional<Tensor>& shifts,
                                            const std::string& interpolation, double oversampling,
                                            const optional<double>& fourier_radius_cutoff) {
    TORCH_CHECK(projections.is_complex(), "Projections must be a complex tensor");
    TORCH_CHECK(projections.dim() == 4, "Projections must be (B, P, height, width/2+1)");
    validate_inputs(interpolation, projections, rotations, shifts, 4, dim);
    if (weights.has_value()) {
        TORCH_CHECK(weights->is_floating_point(), "Weights must be a real-valued tensor");
        TORCH_CHECK(weights->dim() == 4, "Weights must be (B, P, height, width/2+1)");
        TORCH_CHECK(weights->sizes() == projections.sizes(), "Weights and projections must have the same shape");
    }
    const int64_t B = projections.size(0), P = projections.size(1);
    const int64_t n = projections.size(2), hp = projections.size(3);
    const int64_t B_rot = rotations.size(0);
    TORCH_CHECK(B_rot == B || B_rot == 1, "Batch size of rotations must be 1 or same as projections");
    TORCH_CHECK(rotations.size(1) == P, "Number of poses in rotations must match projections");
    check_shift_batch(shifts, B, P, "projections");
    const auto dev = projections.device();
    c10::hip::HIPGuardMasqueradingAsCUDA guard(dev);
    const int dt = dtype_code(projections);
    check_real_dtypes(projections.scalar_type(), rotations, weights);
    const auto real = c10::toRealValueType(projections.scalar_type());
    const Tensor pr = projections.contiguous();
    const Prep rot = prep(rotations, real, dev), sh = prep_opt(shifts, real, dev), w = prep_opt(weights, real, dev);
    const int64_t N = rec_boxsize_for(n, oversampling);
    TORCH_CHECK(N >= 2, "oversampling gives a reconstruction box below 2");
    std::vector<int64_t> shape = dim == 2 ? std::vector<int64_t>{B, N, N / 2 + 1}
                                          : std::vector<int64_t>{B, N, N, N / 2 + 1};
    Tensor data = at::empty(shape, projections.options());
    Tensor wrec = w.t.defined() ? at::empty(shape, w.t.options()) : Tensor();
    const int has_cut = fourier_radius_cutoff.has_value();
    const double cut = fourier_radius_cutoff.value_or(0.0);
    const int64_t Bs = sh.t.defined() ? sh.t.size(0) : 1;
    void* wptr = wrec.defined() ? wrec.data_ptr() : nullptr;
    int rc;
    if (dim == 2)
        rc = tp_backproject_2d_forw(dt, pr.data_ptr(), B, P, n, hp, w.ptr(), rot.ptr(), B_rot, sh.ptr(), Bs,
                                    interp_code(interpolation), oversampling, has_cut, cut, data.data_ptr(), wptr,
                                    current_stream(dev));
    else
        rc = tp_backproject_2d_to_3d_forw(dt, pr.data_ptr(), B, P, n, hp, w.ptr(), rot.ptr(), B_rot, sh.ptr(), Bs,
                                          interp_code(interpolation), oversampling, has_cut, cut, data.data_ptr(),
                                          wptr, current_stream(dev));
    check_rc(rc);
    if (!wrec.defined()) return {data, torch::empty({0}, projections.options().dtype(rotations.scalar_type()))};
    return {data, wrec.to(weights->scalar_type())};
}

// ------------------------------------------------------------------ backprojection backward
std::tuple<Tensor, Tensor, Tensor, Tensor> backproject_back(
    int dim, const Tensor& grad_data_rec, const optional<Tensor>& grad_weight_rec, const Tensor& projections,
    const optional<Tensor>& weights, const Tensor& rotations, const optional<Tensor>& shifts,
    const std::string& interpolation, double oversampling, const optional<double>& fourier_radius_cutoff) {
    TORCH_CHECK(grad_data_rec.is_complex(), "grad_data_rec must be a complex tensor");
    TORCH_CHECK(grad_data_rec.dim() == dim + 1,
                dim == 2 ? "grad_data_rec must be (B, height, width/2+1)" : "grad_data_rec must be (B, D, H, W/2+1)");
    validate_inputs(interpolation, projections, rotations, shifts, 4, dim);
    if (grad_weight_rec.has_value()) {
        TORCH_CHECK(grad_weight_rec->is_floating_point(), "grad_weight_rec must be a real-valued tensor");
        TORCH_CHECK(grad_weight_rec->dim() == dim + 1, dim == 2 ? "grad_weight_rec must be (B, height, width/2+1)"
                                                                : "grad_weight_rec must be (B, D, H, W/2+1)");
        TORCH_CHECK(grad_weight_rec->sizes() == grad_data_rec.sizes(),
                    "grad_weight_rec and grad_data_rec must have same shape");
    }
    const int64_t B = projections.size(0), P = projections.size(1);
    const int64_t n = projections.size(2), hp = projections.size(3);
    const int64_t N = rec_boxsize_for(n, oversampling);
    if (dim == 3) {
        TORCH_CHECK(grad_data_rec.size(1) == N, "grad_data_rec depth must match expected reconstruction size");
        TORCH_CHECK(grad_data_rec.size(2) == N, "grad_data_rec height must match expected reconstruction size");
        TORCH_CHECK(grad_data_rec.size(3) == N / 2 + 1, "grad_data_rec width must match expected reconstruction size");
    } else {
        TORCH_CHECK(grad_data_rec.size(1) == N, "grad_data_rec height must match expected reconstruction size");
        TORCH_CHECK(grad_data_rec.size(2) == N / 2 + 1, "grad_data_rec width must match expected reconstruction size");
    }
    TORCH_CHECK(grad_data_rec.size(0) == B, "grad_data_rec and projections batch sizes differ");
    if (weights.has_value())
        TORCH_CHECK(weights->sizes() == projections.sizes(), "Weights and projections must have the same shape");
    const int64_t B_rot = rotations.size(0);
    TORCH_CHECK(B_rot == B || B_rot == 1, "Batch size of rotations must be 1 or same as projections");
    TORCH_CHECK(rotations.size(1) == P, "Number of poses in rotations must match projections");
    check_shift_batch(shifts, B, P, "projections");
    TORCH_CHECK(projections.scalar_type() == grad_data_rec.scalar_type(),
                "projections and grad_data_rec must have the same dtype");
    const auto dev = projections.device();
    c10::hip::HIPGuardMasqueradingAsCUDA guard(dev);
    const int dt = dtype_code(projections);
    check_real_dtypes(projections.scalar_type(), rotations, weights, grad_weight_rec);
    const auto real = c10::toRealValueType(projections.scalar_type());
    TORCH_CHECK(grad_data_rec.device() == dev, "all tensors must be on the same GPU");
    const Tensor gd = grad_data_rec.contiguous(), pr = projections.contiguous();
    const Prep gw = prep_opt(grad_weight_rec, real, dev), w = prep_opt(weights, real, dev);
    const Prep rot = prep(rotations, real, dev), sh = prep_opt(shifts, real, dev);
    PoseGrads pg = pose_grads(rotations, shifts, rot, sh);
    Tensor gproj = at::empty_like(pr);
    Tensor gweights = w.t.defined() ? at::empty_like(w.t) : Tensor();
    const int has_cut = fourier_radius_cutoff.has_value();
    const double cut = fourier_radius_cutoff.value_or(0.0);
    const int64_t Bs = sh.t.defined() ? sh.t.size(0) : 1;
    void* grot = pg.need_rot ? pg.rot.data_ptr() : nullptr;
    void* gsh = pg.need_shift ? pg.shift.data_ptr() : nullptr;
    void* gwp = gweights.defined() ? gweights.data_ptr() : nullptr;
    int rc;
    if (dim == 2)
        rc = tp_backproject_2d_back(dt, gd.data_ptr(), gw.ptr(), gd.size(1), gd.size(2), pr.data_ptr(), B, P, n, hp,
                                    w.ptr(), rot.ptr(), B_rot, sh.ptr(), Bs, interp_code(interpolation),
                                    oversampling, has_cut, cut, gproj.data_ptr(), gwp, grot, gsh,
                                    current_stream(dev));
    else
        rc = tp_backproject_2d_to_3d_back(dt, gd.data_ptr(), gw.ptr(), gd.size(2), gd.size(3), pr.data_ptr(), B, P, n,
                                          hp, w.ptr(), rot.ptr(), B_rot, sh.ptr(), Bs, interp_code(interpolation),
                                          oversampling, has_cut, cut, gproj.data_ptr(), gwp, grot, gsh,
                                          current_stream(dev));
    check_rc(rc);
    Tensor gw_out = gweights.defined() ? gweights.to(weights->scalar_type())
                                       : torch::empty({0}, projections.options().dtype(rotations.scalar_type()));
    return {gproj, gw_out, finish_rot(pg, rotations), finish_shift(pg, rotations, shifts, gproj)};
}

// ------------------------------------------------------------------ op entry points (schema signatures)
Tensor project_2d_forw_hip(const Tensor& reconstruction, const Tensor& rotations, const optional<Tensor>& shifts,
                           const at::IntArrayRef output_shape, const std::string& interpolation,
                           const double oversampling, const optional<double>& fourier_radius_cutoff) {
    return project_forw(2, reconstruction, rotations, shifts, output_shape, interpolation, oversampling,
                        fourier_radius_cutoff);
}
Tensor project_3d_to_2d_forw_hip(const Tensor& reconstruction, const Tensor& rotations,
                                 const optional<Tensor>& shifts, const at::IntArrayRef output_shape,
                                 const std::string& interpolation, const double oversampling,
                                 const optional<double>& fourier_radius_cutoff) {
    return project_forw(3, reconstruction, rotations, shifts, output_shape, interpolation, oversampling,
                        fourier_radius_cutoff);
}
std::tuple<Tensor, Tensor, Tensor> project_2d_back_hip(const Tensor& grad_projections, const Tensor& reconstruction,
                                                       const Tensor& rotations, const optional<Tensor>& shifts,
                                                       const std::string& interpolation, const double oversampling,
                                                       const optional<double>& fourier_radius_cutoff) {
    return project_back(2, grad_projections, reconstruction, rotations, shifts, interpolation, oversampling,
                        fourier_radius_cutoff);
}
std::tuple<Tensor, Tensor, Tensor> project_3d_to_2d_back_hip(const Tensor& grad_projections,
                                                             const Tensor& reconstruction, const Tensor& rotations,
                                                             const optional<Tensor>& shifts,
                                                             const std::string& interpolation,
                                                             const double oversampling,
                                                             const optional<double>& fourier_radius_cutoff) {
    return project_back(3, grad_projections, reconstruction, rotations, shifts, interpolation, oversampling,
                        fourier_radius_cutoff);
}
std::tuple<Tensor, Tensor> backproject_2d_forw_hip(const Tensor& projections, const optional<Tensor>& weights,
                                                   const Tensor& rotations, const optional<Tensor>& shifts,
                                                   const std::string& interpolation, const double oversampling,
                                                   const optional<double>& fourier_radius_cutoff) {
    return backproject_forw(2, projections, weights, rotations, shifts, interpolation, oversampling,
                            fourier_radius_cutoff);
}
std::tuple<Tensor, Tensor> backproject_2d_to_3d_forw_hip(const Tensor& projections, const optional<Tensor>& weights,
                                                         const Tensor& rotations, const optional<Tensor>& shifts,
                                                         const std::string& interpolation, const double oversampling,
                                                         const optional<double>& fourier_radius_cutoff) {
    return backproject_forw(3, projections, weights, rotations, shifts, interpolation, oversampling,
                            fourier_radius_cutoff);
}
std::tuple<Tensor, Tensor, Tensor, Tensor> backproject_2d_back_hip(
    const Tensor& grad_data_rec, const optional<Tensor>& grad_weight_rec, const Tensor& projections,
    const optional<Tensor>& weights, const Tensor& rotations, const optional<Tensor>& shifts,
    const std::string& interpolation, const double oversampling, const optional<double>& fourier_radius_cutoff) {
    return backproject_back(2, grad_data_rec, grad_weight_rec, projections, weights, rotations, shifts, interpolation,
                            oversampling, fourier_radius_cutoff);
}
std::tuple<Tensor, Tensor, Tensor, Tensor> backproject_2d_to_3d_back_hip(
    const Tensor& grad_data_rec, const optional<Tensor>& grad_weight_rec, const Tensor& projections,
    const optional<Tensor>& weights, const Tensor& rotations, const optional<Tensor>& shifts,
    const std::string& interpolation, const double oversampling, const optional<double>& fourier_radius_cutoff) {
    return backproject_back(3, grad_data_rec, grad_weight_rec, projections, weights, rotations, shifts, interpolation,
                            oversampling, fourier_radius_cutoff);
}

}  // namespace

TORCH_LIBRARY(torch_projectors, m) {
    m.def("project_2d_forw(Tensor reconstruction, Tensor rotations, Tensor? shifts, int[] output_shape, str interpolation, float oversampling, float? fourier_radius_cutoff) -> Tensor");
    m.def("project_2d_back(Tensor grad_projections, Tensor reconstruction, Tensor rotations, Tensor? shifts, str interpolation, float oversampling, float? fourier_radius_cutoff) -> (Tensor, Tensor, Tensor)");
    m.def("backproject_2d_forw(Tensor projections, Tensor? weights, Tensor rotations, Tensor? shifts, str interpolation, float oversampling, float? fourier_radius_cutoff) -> (Tensor, Tensor)");
    m.def("backproject_2d_back(Tensor grad_data_rec, Tensor? grad_weight_rec, Tensor projections, Tensor? weights, Tensor rotations, Tensor? shifts, str interpolation, float oversampling, float? fourier_radius_cutoff) -> (Tensor, Tensor, Tensor, Tensor)");
    m.def("project_3d_to_2d_forw(Tensor reconstruction, Tensor rotations, Tensor? shifts, int[] output_shape, str interpolation, float oversampling, float? fourier_radius_cutoff) -> Tensor");
    m.def("project_3d_to_2d_back(Tensor grad_projections, Tensor reconstruction, Tensor rotations, Tensor? shifts, str interpolation, float oversampling, float? fourier_radius_cutoff) -> (Tensor, Tensor, Tensor)");
    m.def("backproject_2d_to_3d_forw(Tensor projections, Tensor? weights, Tensor rotations, Tensor? shifts, str interpolation, float oversampling, float? fourier_radius_cutoff) -> (Tensor, Tensor)");
    m.def("backproject_2d_to_3d_back(Tensor grad_data_rec, Tensor? grad_weight_rec, Tensor projections, Tensor? weights, Tensor rotations, Tensor? shifts, str interpolation, float oversampling, float? fourier_radius_cutoff) -> (Tensor, Tensor, Tensor, Tensor)");
}

TORCH_LIBRARY_IMPL(torch_projectors, CUDA, m) {
    m.impl("project_2d_forw", &project_2d_forw_hip);
    m.impl("project_2d_back", &project_2d_back_hip);
    m.impl("backproject_2d_forw", &backproject_2d_forw_hip);
    m.impl("backproject_2d_back", &backproject_2d_back_hip);
    m.impl("project_3d_to_2d_forw", &project_3d_to_2d_forw_hip);
    m.impl("project_3d_to_2d_back", &project_3d_to_2d_back_hip);
    m.impl("backproject_2d_to_3d_forw", &backproject_2d_to_3d_forw_hip);
    m.impl("backproject_2d_to_3d_back", &backproject_2d_to_3d_back_hip);
}
