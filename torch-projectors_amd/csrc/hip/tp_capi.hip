// C ABI of libtorch_projectors_hip.so (declared in include/torch_projectors_hip.h).
//
// Each entry point validates its arguments with the conditions of the
// reference (validate_projection_inputs, projection_utils.h:23-48, and the
// per-op TORCH_CHECKs), derives the launch geometry, zero-fills the outputs
// that are accumulated, and enqueues the kernels on the caller's stream.
// Nothing is synchronised and nothing is allocated.
#include <cmath>
#include <string>

#include "../../../include/torch_projectors_hip.h"
#include "tp_launch.hh"

namespace {

thread_local std::string g_err;

int fail(const std::string& m) {
    g_err = m;
    return TP_ERR_INVALID;
}

int hip_fail(hipError_t e, const char* what) {
    g_err = std::string(what) + ": " + hipGetErrorString(e);
    return TP_ERR_HIP;
}

constexpr int64_t kInt32Max = 2147483647;

// Shared argument checks; fills the pose part of `g`.
int check_common(int dtype, int interp, int64_t B, int64_t P, int64_t B_rot, const void* shifts, int64_t B_shift,
                 tp::Geom& g) {
    if (dtype != TP_F32 && dtype != TP_F64) return fail("dtype must be TP_F32 or TP_F64");
    if (interp != TP_LINEAR && interp != TP_CUBIC) return fail("Supported interpolation methods: 'linear', 'cubic'");
    if (B < 0 || P < 0) return fail("batch and pose counts must be non-negative");
    if (B_rot != B && B_rot != 1) return fail("Batch size of rotations must be 1 or same as reconstruction");
    if (shifts && B_shift != B && B_shift != 1)
        return fail("Batch size of shifts must be 1 or same as reconstruction");
    g.B = B;
    g.P = P;
    g.B_rot = B_rot;
    g.B_shift = shifts ? B_shift : 1;
    return TP_OK;
}

int set_proj(int64_t n, tp::Geom& g) {
    if (n < 1) return fail("projection box size must be positive");
    const int64_t hp = n / 2 + 1;
    if (n * hp > kInt32Max) return fail("projection too large (n*(n/2+1) must be < 2^31)");
    g.n = int(n);
    g.hp = int(hp);
    g.npix = int(n * hp);
    g.chunks = int((g.npix + tp::kBlock - 1) / tp::kBlock);
    g.work = g.B * g.P * g.chunks;
    g.phase_k = -2.0 * M_PI / double(n);
    return TP_OK;
}

int set_rec(int dim, int64_t N, int64_t H, tp::Geom& g) {
    if (N < 2) return fail("reconstruction box size must be at least 2");
    if (H != N / 2 + 1) return fail("reconstruction last dimension must be boxsize/2+1");
    const int64_t vol = dim == 2 ? N * H : N * N * H;
    if (vol > kInt32Max) return fail("reconstruction too large (elements per batch item must be < 2^31)");
    g.N = int(N);
    g.H = int(H);
    g.vol = vol;
    return TP_OK;
}

// Squared cutoff radius, rounded in the real type like the reference
// (cpu/3d/projection_3d_to_2d_kernels.cpp:145-149): default radius n/2.
void set_cut(int dtype, int has_cut, double cut, tp::Geom& g) {
    const double radius = has_cut ? cut : double(g.n) / 2.0;
    if (dtype == TP_F32) {
        const float rf = float(radius);
        const float r2 = rf * rf;
        g.cut2 = double(r2);
    } else {
        g.cut2 = radius * radius;
    }
}

int64_t rec_box(int64_t n, double os) {
    const int64_t raw = static_cast<int64_t>(std::ceil(double(n) * os));
    return raw + (raw % 2);
}

int64_t cx_words(int dtype, int64_t elems) { return elems * (dtype == TP_F32 ? 2 : 4); }
int64_t re_words(int dtype, int64_t elems) { return elems * (dtype == TP_F32 ? 1 : 2); }

int zero(void* p, int64_t words, hipStream_t s) {
    if (!p || words <= 0) return TP_OK;
    const hipError_t e = tp::launch_zero(p, words, s);
    return e == hipSuccess ? TP_OK : hip_fail(e, "zero-fill launch");
}

int need(const void* p, const char* name) {
    if (!p) return fail(std::string(name) + " must not be NULL");
    return TP_OK;
}

#define TP_TRY(expr)                 \
    do {                             \
        const int rc_ = (expr);      \
        if (rc_ != TP_OK) return rc_; \
    } while (0)

int launched(hipError_t e, const char* what) { return e == hipSuccess ? TP_OK : hip_fail(e, what); }

int project_forw(int dim, int dtype, const void* rec, int64_t B, int64_t D, int64_t N, int64_t H, const void* rot,
                 int64_t B_rot, int64_t P, const void* shifts, int64_t B_shift, int64_t n, int interp, double os,
                 int has_cut, double cut, void* out, void* stream) {
    tp::Geom g{};
    TP_TRY(check_common(dtype, interp, B, P, B_rot, shifts, B_shift, g));
    if (dim == 3 && D != N) return fail("reconstruction depth must equal its height");
    TP_TRY(set_rec(dim, N, H, g));
    TP_TRY(set_proj(n, g));
    set_cut(dtype, has_cut, cut, g);
    g.os = os;
    if (g.work == 0) return TP_OK;
    TP_TRY(need(rec, "reconstruction"));
    TP_TRY(need(rot, "rotations"));
    TP_TRY(need(out, "projections"));
    hipStream_t s = static_cast<hipStream_t>(stream);
    return launched(tp::launch_project_forw(dim, dtype, interp == TP_CUBIC, g, rec, rot, shifts, out, s),
                    "projection launch");
}

int project_back(int dim, int dtype, const void* gproj, int64_t B, int64_t P, int64_t n, int64_t hp, const void* rec,
                 int64_t D, int64_t N, int64_t H, const void* rot, int64_t B_rot, const void* shifts,
                 int64_t B_shift, int interp, double os, int has_cut, double cut, void* grec, void* grot,
                 void* gshift, void* stream) {
    tp::Geom g{};
    TP_TRY(check_common(dtype, interp, B, P, B_rot, shifts, B_shift, g));
    if (dim == 3 && D != N) return fail("reconstruction depth must equal its height");
    if (hp != n / 2 + 1) return fail("grad_projections last dimension must be boxsize/2+1");
    if (gshift && !shifts) return fail("grad_shifts requested without shifts");
    TP_TRY(set_rec(dim, N, H, g));
    TP_TRY(set_proj(n, g));
    set_cut(dtype, has_cut, cut, g);
    g.os = os;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (g.B > 0) TP_TRY(need(grec, "grad_reconstruction"));
    TP_TRY(zero(grec, cx_words(dtype, g.B * g.vol), s));
    TP_TRY(zero(grot, re_words(dtype, g.B_rot * g.P * dim * dim), s));
    TP_TRY(zero(gshift, re_words(dtype, g.B_shift * g.P * 2), s));
    if (g.work == 0) return TP_OK;
    TP_TRY(need(gproj, "grad_projections"));
    TP_TRY(need(rec, "reconstruction"));
    TP_TRY(need(rot, "rotations"));
    return launched(tp::launch_project_back(dim, dtype, interp == TP_CUBIC, g, gproj, rec, rot, shifts, grec, grot,
                                            gshift, s),
                    "projection backward launch");
}

int backproject_forw(int dim, int dtype, const void* proj, int64_t B, int64_t P, int64_t n, int64_t hp,
                     const void* weights, const void* rot, int64_t B_rot, const void* shifts, int64_t B_shift,
                     int interp, double os, int has_cut, double cut, void* data, void* wrec, void* stream) {
    tp::Geom g{};
    TP_TRY(check_common(dtype, interp, B, P, B_rot, shifts, B_shift, g));
    if (hp != n / 2 + 1) return fail("projections last dimension must be boxsize/2+1");
    if ((weights == nullptr) != (wrec == nullptr))
        return fail("weight_reconstruction must be given exactly when weights are");
    const int64_t N = rec_box(n, os);
    TP_TRY(set_rec(dim, N, N / 2 + 1, g));
    TP_TRY(set_proj(n, g));
    set_cut(dtype, has_cut, cut, g);
    g.os = os;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (g.B > 0) TP_TRY(need(data, "data_reconstruction"));
    TP_TRY(zero(data, cx_words(dtype, g.B * g.vol), s));
    TP_TRY(zero(wrec, re_words(dtype, g.B * g.vol), s));
    if (g.work == 0) return TP_OK;
    TP_TRY(need(proj, "projections"));
    TP_TRY(need(rot, "rotations"));
    return launched(
        tp::launch_backproject_forw(dim, dtype, interp == TP_CUBIC, g, proj, weights, rot, shifts, data, wrec, s),
        "backprojection launch");
}

int backproject_back(int dim, int dtype, const void* gdata, const void* gw, int64_t N, int64_t H, const void* proj,
                     int64_t B, int64_t P, int64_t n, int64_t hp, const void* weights, const void* rot,
                     int64_t B_rot, const void* shifts, int64_t B_shift, int interp, double os, int has_cut,
                     double cut, void* gproj, void* gweights, void* grot, void* gshift, void* stream) {
    tp::Geom g{};
    TP_TRY(check_common(dtype, interp, B, P, B_rot, shifts, B_shift, g));
    if (hp != n / 2 + 1) return fail("projections last dimension must be boxsize/2+1");
    if (gweights && !weights) return fail("grad_weights requested without weights");
    if (gshift && !shifts) return fail("grad_shifts requested without shifts");
    TP_TRY(set_rec(dim, N, H, g));
    TP_TRY(set_proj(n, g));
    set_cut(dtype, has_cut, cut, g);
    g.os = os;
    hipStream_t s = static_cast<hipStream_t>(stream);
    TP_TRY(zero(grot, re_words(dtype, g.B_rot * g.P * dim * dim), s));
    TP_TRY(zero(gshift, re_words(dtype, g.B_shift * g.P * 2), s));
    if (g.work == 0) return TP_OK;
    TP_TRY(need(gdata, "grad_data_rec"));
    TP_TRY(need(proj, "projections"));
    TP_TRY(need(rot, "rotations"));
    TP_TRY(need(gproj, "grad_projections"));
    return launched(tp::launch_backproject_back(dim, dtype, interp == TP_CUBIC, g, gdata, gw, proj, rot, shifts,
                                                gproj, gweights, grot, gshift, s),
                    "backprojection backward launch");
}

}  // namespace

extern "C" {

const char* tp_last_error(void) { return g_err.c_str(); }

int tp_abi_version(void) { return 1; }

int64_t tp_backproject_rec_boxsize(int64_t proj_boxsize, double oversampling) {
    return rec_box(proj_boxsize, oversampling);
}

int tp_project_2d_forw(int dtype, const void* reconstruction, int64_t B, int64_t rec_boxsize,
                       int64_t rec_boxsize_half, const void* rotations, int64_t B_rot, int64_t P, const void* shifts,
                       int64_t B_shift, int64_t proj_boxsize, int interpolation, double oversampling, int has_cutoff,
                       double fourier_radius_cutoff, void* projections, void* stream) {
    g_err.clear();
    return project_forw(2, dtype, reconstruction, B, rec_boxsize, rec_boxsize, rec_boxsize_half, rotations, B_rot, P,
                        shifts, B_shift, proj_boxsize, interpolation, oversampling, has_cutoff,
                        fourier_radius_cutoff, projections, stream);
}

int tp_project_3d_to_2d_forw(int dtype, const void* reconstruction, int64_t B, int64_t rec_depth,
                             int64_t rec_boxsize, int64_t rec_boxsize_half, const void* rotations, int64_t B_rot,
                             int64_t P, const void* shifts, int64_t B_shift, int64_t proj_boxsize, int interpolation,
                             double oversampling, int has_cutoff, double fourier_radius_cutoff, void* projections,
                             void* stream) {
    g_err.clear();
    return project_forw(3, dtype, reconstruction, B, rec_depth, rec_boxsize, rec_boxsize_half, rotations, B_rot, P,
                        shifts, B_shift, proj_boxsize, interpolation, oversampling, has_cutoff,
                        fourier_radius_cutoff, projections, stream);
}

int tp_project_2d_back(int dtype, const void* grad_projections, int64_t B, int64_t P, int64_t proj_boxsize,
                       int64_t proj_boxsize_half, const void* reconstruction, int64_t rec_boxsize,
                       int64_t rec_boxsize_half, const void* rotations, int64_t B_rot, const void* shifts,
                       int64_t B_shift, int interpolation, double oversampling, int has_cutoff,
                       double fourier_radius_cutoff, void* grad_reconstruction, void* grad_rotations,
                       void* grad_shifts, void* stream) {
    g_err.clear();
    return project_back(2, dtype, grad_projections, B, P, proj_boxsize, proj_boxsize_half, reconstruction,
                        rec_boxsize, rec_boxsize, rec_boxsize_half, rotations, B_rot, shifts, B_shift, interpolation,
                        oversampling, has_cutoff, fourier_radius_cutoff, grad_reconstruction, grad_rotations,
                        grad_shifts, stream);
}

int tp_project_3d_to_2d_back(int dtype, const void* grad_projections, int64_t B, int64_t P, int64_t proj_boxsize,
                             int64_t proj_boxsize_half, const void* reconstruction, int64_t rec_depth,
                             int64_t rec_boxsize, int64_t rec_boxsize_half, const void* rotations, int64_t B_rot,
                             const void* shifts, int64_t B_shift, int interpolation, double oversampling,
                             int has_cutoff, double fourier_radius_cutoff, void* grad_reconstruction,
                             void* grad_rotations, void* grad_shifts, void* stream) {
    g_err.clear();
    return project_back(3, dtype, grad_projections, B, P, proj_boxsize, proj_boxsize_half, reconstruction, rec_depth,
                        rec_boxsize, rec_boxsize_half, rotations, B_rot, shifts, B_shift, interpolation,
                        oversampling, has_cutoff, fourier_radius_cutoff, grad_reconstruction, grad_rotations,
                        grad_shifts, stream);
}

int tp_backproject_2d_forw(int dtype, const void* projections, int64_t B, int64_t P, int64_t proj_boxsize,
                           int64_t proj_boxsize_half, const void* weights, const void* rotations, int64_t B_rot,
                           const void* shifts, int64_t B_shift, int interpolation, double oversampling,
                           int has_cutoff, double fourier_radius_cutoff, void* data_reconstruction,
                           void* weight_reconstruction, void* stream) {
    g_err.clear();
    return backproject_forw(2, dtype, projections, B, P, proj_boxsize, proj_boxsize_half, weights, rotations, B_rot,
                            shifts, B_shift, interpolation, oversampling, has_cutoff, fourier_radius_cutoff,
                            data_reconstruction, weight_reconstruction, stream);
}

int tp_backproject_2d_to_3d_forw(int dtype, const void* projections, int64_t B, int64_t P, int64_t proj_boxsize,
                                 int64_t proj_boxsize_half, const void* weights, const void* rotations,
                                 int64_t B_rot, const void* shifts, int64_t B_shift, int interpolation,
                                 double oversampling, int has_cutoff, double fourier_radius_cutoff,
                                 void* data_reconstruction, void* weight_reconstruction, void* stream) {
    g_err.clear();
    return backproject_forw(3, dtype, projections, B, P, proj_boxsize, proj_boxsize_half, weights, rotations, B_rot,
                            shifts, B_shift, interpolation, oversampling, has_cutoff, fourier_radius_cutoff,
                            data_reconstruction, weight_reconstruction, stream);
}

int tp_backproject_2d_back(int dtype, const void* grad_data_rec, const void* grad_weight_rec, int64_t rec_boxsize,
                           int64_t rec_boxsize_half, const void* projections, int64_t B, int64_t P,
                           int64_t proj_boxsize, int64_t proj_boxsize_half, const void* weights,
                           const void* rotations, int64_t B_rot, const void* shifts, int64_t B_shift,
                           int interpolation, double oversampling, int has_cutoff, double fourier_radius_cutoff,
                           void* grad_projections, void* grad_weights, void* grad_rotations, void* grad_shifts,
                           void* stream) {
    g_err.clear();
    return backproject_back(2, dtype, grad_data_rec, grad_weight_rec, rec_boxsize, rec_boxsize_half, projections, B,
                            P, proj_boxsize, proj_boxsize_half, weights, rotations, B_rot, shifts, B_shift,
                            interpolation, oversampling, has_cutoff, fourier_radius_cutoff, grad_projections,
                            grad_weights, grad_rotations, grad_shifts, stream);
}

int tp_backproject_2d_to_3d_back(int dtype, const void* grad_data_rec, const void* grad_weight_rec,
                                 int64_t rec_boxsize, int64_t rec_boxsize_half, const void* projections, int64_t B,
                                 int64_t P, int64_t proj_boxsize, int64_t proj_boxsize_half, const void* weights,
                                 const void* rotations, int64_t B_rot, const void* shifts, int64_t B_shift,
                                 int interpolation, double oversampling, int has_cutoff,
                                 double fourier_radius_cutoff, void* grad_projections, void* grad_weights,
                                 void* grad_rotations, void* grad_shifts, void* stream) {
    g_err.clear();
    return backproject_back(3, dtype, grad_data_rec, grad_weight_rec, rec_boxsize, rec_boxsize_half, projections, B,
                            P, proj_boxsize, proj_boxsize_half, weights, rotations, B_rot, shifts, B_shift,
                            interpolation, oversampling, has_cutoff, fourier_radius_cutoff, grad_projections,
                            grad_weights, grad_rotations, grad_shifts, stream);
}

}  // extern "C"
