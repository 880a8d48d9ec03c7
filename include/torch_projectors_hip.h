/*
 * torch_projectors_hip.h — C ABI of the MI355X (gfx950) projector library
 * libtorch_projectors_hip.so.
 *
 * One entry point per dispatcher op of the reference
 * (csrc/torch_projectors.cpp:23-36).  Each replaces the reference's
 * `*_cuda` host wrapper for that op; the wrapper it replaces is cited above
 * each declaration.  Tensors become (pointer, sizes) pairs:
 *
 *   - every array is dense, row-major, in device memory of the current HIP
 *     device, and must not alias another argument;
 *   - complex arrays are interleaved (re, im) pairs of the real type chosen
 *     by `dtype` (TP_F32: complex64 / float32, TP_F64: complex128 / float64);
 *     rotations, shifts and weights use that same real type;
 *   - an optional input is passed as NULL when absent; an array with no
 *     elements may be passed as NULL too;
 *   - an optional gradient output is passed as NULL when it is not wanted
 *     (the reference decides this from `requires_grad`, projection_utils.h:112-113);
 *   - every output element is written by the call (no pre-zeroing needed);
 *   - work is enqueued on `stream` (a hipStream_t; NULL = default stream) and
 *     the call returns without synchronising.
 *
 * Shapes (n = projection box, N = reconstruction box, h = N/2+1, hp = n/2+1):
 *   2D reconstruction  [B, N, h]        3D reconstruction [B, N, N, h]
 *   projections        [B, P, n, hp]    weights           [B, P, n, hp] (real)
 *   rotations          [B_rot, P, 2, 2] or [B_rot, P, 3, 3], B_rot in {1, B}
 *   shifts             [B_shift, P, 2], B_shift in {1, B}; component 0 pairs
 *                      with the row frequency, component 1 with the column
 *   rotation/shift gradients have the shape of rotations/shifts.
 *
 * `interpolation` is TP_LINEAR or TP_CUBIC; `has_cutoff` = 0 means the
 * reference default cutoff n/2 (cpu/3d/projection_3d_to_2d_kernels.cpp:147-149).
 *
 * Return value: TP_OK, or an error code with a message in tp_last_error()
 * (thread-local).  Argument errors are detected before anything is enqueued.
 */
#ifndef TORCH_PROJECTORS_HIP_H
#define TORCH_PROJECTORS_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TP_OK 0
#define TP_ERR_INVALID 1 /* invalid argument (shape, dtype, pointer) */
#define TP_ERR_HIP 2     /* HIP runtime / launch failure */

#define TP_F32 0 /* complex64 + float32 */
#define TP_F64 1 /* complex128 + float64 */
/* Forward projections and their gradients only (tp_project_2d_forw,
 * tp_project_3d_to_2d_forw, tp_project_2d_back, tp_project_3d_to_2d_back):
 * the reconstruction is stored as complex half (interleaved binary16 pairs,
 * torch.complex32); rotations, shifts, projections, grad_projections and the
 * gradient outputs (grad_reconstruction complex64) are TP_F32, and every
 * stored value is widened exactly to fp32 before the TP_F32 arithmetic.  No
 * counterpart in the reference: an opt-in low-precision volume storage that
 * halves the volume's footprint and the bytes its staging reads. */
#define TP_F16S 2

#define TP_LINEAR 0
#define TP_CUBIC 1

/* Message of the last failed call on this thread ("" if none). */
const char* tp_last_error(void);

/* ABI version of this header (bumped on any signature change). */
int tp_abi_version(void);

/* Reconstruction box produced by the backprojection ops: ceil(n*os) rounded
 * up to even (cpu/3d/backprojection_2d_to_3d_kernels.cpp:129-132). */
int64_t tp_backproject_rec_boxsize(int64_t proj_boxsize, double oversampling);

/* ---------------------------------------------------------------- 2D -> 2D */

/* Replaces project_2d_forw_cuda (cuda/2d/projection_2d_kernels.cu:633-758). */
int tp_project_2d_forw(int dtype,
                       const void* reconstruction, int64_t B, int64_t rec_boxsize, int64_t rec_boxsize_half,
                       const void* rotations, int64_t B_rot, int64_t P,
                       const void* shifts, int64_t B_shift,
                       int64_t proj_boxsize,
                       int interpolation, double oversampling, int has_cutoff, double fourier_radius_cutoff,
                       void* projections,
                       void* stream);

/* Replaces project_2d_back_cuda (cuda/2d/projection_2d_kernels.cu:760-920).
 * grad_reconstruction has the reconstruction's shape. */
int tp_project_2d_back(int dtype,
                       const void* grad_projections, int64_t B, int64_t P, int64_t proj_boxsize, int64_t proj_boxsize_half,
                       const void* reconstruction, int64_t rec_boxsize, int64_t rec_boxsize_half,
                       const void* rotations, int64_t B_rot,
                       const void* shifts, int64_t B_shift,
                       int interpolation, double oversampling, int has_cutoff, double fourier_radius_cutoff,
                       void* grad_reconstruction, void* grad_rotations, void* grad_shifts,
                       void* stream);

/* Replaces backproject_2d_forw_cuda (cuda/2d/backprojection_2d_kernels.cu:827-977).
 * Outputs have shape [B, N, N/2+1] with N = tp_backproject_rec_boxsize(n, os);
 * weight_reconstruction must be non-NULL exactly when weights is (when
 * B * P == 0, weights may be NULL with weight_reconstruction given: it is
 * zero-filled). */
int tp_backproject_2d_forw(int dtype,
                           const void* projections, int64_t B, int64_t P, int64_t proj_boxsize, int64_t proj_boxsize_half,
                           const void* weights,
                           const void* rotations, int64_t B_rot,
                           const void* shifts, int64_t B_shift,
                           int interpolation, double oversampling, int has_cutoff, double fourier_radius_cutoff,
                           void* data_reconstruction, void* weight_reconstruction,
                           void* stream);

/* Replaces backproject_2d_back_cuda (cuda/2d/backprojection_2d_kernels.cu:979-1191).
 * grad_weights (shape of weights) may only be non-NULL when weights is; it is
 * all zeros when grad_weight_rec is NULL. */
int tp_backproject_2d_back(int dtype,
                           const void* grad_data_rec, const void* grad_weight_rec, int64_t rec_boxsize, int64_t rec_boxsize_half,
                           const void* projections, int64_t B, int64_t P, int64_t proj_boxsize, int64_t proj_boxsize_half,
                           const void* weights,
                           const void* rotations, int64_t B_rot,
                           const void* shifts, int64_t B_shift,
                           int interpolation, double oversampling, int has_cutoff, double fourier_radius_cutoff,
                           void* grad_projections, void* grad_weights, void* grad_rotations, void* grad_shifts,
                           void* stream);

/* ---------------------------------------------------------------- 3D <-> 2D */

/* Replaces project_3d_to_2d_forw_cuda (cuda/3d/projection_3d_to_2d_kernels.cu:814-1015).
 * rec_depth must equal rec_boxsize. */
int tp_project_3d_to_2d_forw(int dtype,
                             const void* reconstruction, int64_t B, int64_t rec_depth, int64_t rec_boxsize, int64_t rec_boxsize_half,
                             const void* rotations, int64_t B_rot, int64_t P,
                             const void* shifts, int64_t B_shift,
                             int64_t proj_boxsize,
                             int interpolation, double oversampling, int has_cutoff, double fourier_radius_cutoff,
                             void* projections,
                             void* stream);

/* Bytes of the static device scratch array of tp_project_3d_to_2d_forw_noalloc
 * (one copy per GPU, held until the process ends). */
#define TP_NOALLOC_SCRATCH_BYTES 256

/* No counterpart in the reference.  tp_project_3d_to_2d_forw for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc): same arguments, same results, but
 * the tiled kernels' per-call pose summary and work counters live in a static
 * device array of TP_NOALLOC_SCRATCH_BYTES per GPU instead of a scratch area
 * that the first call on each stream allocates; the call itself allocates
 * nothing.  The scratch it needs does not depend on the input sizes (a call
 * needing more than the array would be rejected with TP_ERR_INVALID); the
 * ordinary size limits of tp_project_3d_to_2d_forw apply.  Every call on one
 * GPU shares that GPU's array, and each call's first kernel rewrites what the
 * later ones read, so calls ordered on one stream are safe, while calls that
 * overlap on one GPU (different streams with no order between them) race. */
int tp_project_3d_to_2d_forw_noalloc(int dtype,
                                     const void* reconstruction, int64_t B, int64_t rec_depth, int64_t rec_boxsize,
                                     int64_t rec_boxsize_half,
                                     const void* rotations, int64_t B_rot, int64_t P,
                                     const void* shifts, int64_t B_shift,
                                     int64_t proj_boxsize,
                                     int interpolation, double oversampling, int has_cutoff,
                                     double fourier_radius_cutoff,
                                     void* projections,
                                     void* stream);

/* Replaces project_3d_to_2d_back_cuda (cuda/3d/projection_3d_to_2d_kernels.cu:1018-1179). */
int tp_project_3d_to_2d_back(int dtype,
                             const void* grad_projections, int64_t B, int64_t P, int64_t proj_boxsize, int64_t proj_boxsize_half,
                             const void* reconstruction, int64_t rec_depth, int64_t rec_boxsize, int64_t rec_boxsize_half,
                             const void* rotations, int64_t B_rot,
                             const void* shifts, int64_t B_shift,
                             int interpolation, double oversampling, int has_cutoff, double fourier_radius_cutoff,
                             void* grad_reconstruction, void* grad_rotations, void* grad_shifts,
                             void* stream);

/* Replaces backproject_2d_to_3d_forw_cuda (cuda/3d/backprojection_2d_to_3d_kernels.cu:1001-1188).
 * Outputs have shape [B, N, N, N/2+1] with N = tp_backproject_rec_boxsize(n, os);
 * weights and weight_reconstruction pair as for tp_backproject_2d_forw. */
int tp_backproject_2d_to_3d_forw(int dtype,
                                 const void* projections, int64_t B, int64_t P, int64_t proj_boxsize, int64_t proj_boxsize_half,
                                 const void* weights,
                                 const void* rotations, int64_t B_rot,
                                 const void* shifts, int64_t B_shift,
                                 int interpolation, double oversampling, int has_cutoff, double fourier_radius_cutoff,
                                 void* data_reconstruction, void* weight_reconstruction,
                                 void* stream);

/* Replaces backproject_2d_to_3d_back_cuda (cuda/3d/backprojection_2d_to_3d_kernels.cu:1191-1404). */
int tp_backproject_2d_to_3d_back(int dtype,
                                 const void* grad_data_rec, const void* grad_weight_rec, int64_t rec_boxsize, int64_t rec_boxsize_half,
                                 const void* projections, int64_t B, int64_t P, int64_t proj_boxsize, int64_t proj_boxsize_half,
                                 const void* weights,
                                 const void* rotations, int64_t B_rot,
                                 const void* shifts, int64_t B_shift,
                                 int interpolation, double oversampling, int has_cutoff, double fourier_radius_cutoff,
                                 void* grad_projections, void* grad_weights, void* grad_rotations, void* grad_shifts,
                                 void* stream);

/* ---------------------------------------------------------------- reference preparation
 *
 * The real-space steps around the projectors that the reference performs
 * with tensor ops in its helpers pad_and_fftshift / ifftshift_and_crop
 * (tests/test_utils.py:174-247, 250-293; README.md:106-143), as single-pass
 * kernels, plus the normalisation of a backprojected (data, weight) pair
 * (no counterpart in the reference, whose dual volumes exist for it:
 * paper/main.tex:72).  The FFTs between them are library calls (rocFFT).
 * Elements are moved as opaque words of elem_bytes = 2, 4, 8 or 16 bytes (any
 * real or complex dtype).  Axes: `dim` (2 or 3) equal-role spatial axes after
 * one flattened batch axis, row-major. */

/* pad_and_fftshift's output edge: int(boxsize * oversampling), plus one if odd
 * (tests/test_utils.py:217-220).  Its zero padding before the data is
 * (padded - boxsize) / 2, rounded down (:223-225). */
int64_t tp_padded_boxsize(int64_t boxsize, double oversampling);

/* ifftshift_and_crop's output edge: int(boxsize / oversampling)
 * (tests/test_utils.py:281-286); the crop starts at (boxsize - cropped) / 2. */
int64_t tp_cropped_boxsize(int64_t boxsize, double oversampling);

/* dst[batch, N^dim] = fftshift over every spatial axis of src[batch, n^dim]
 * zero-padded to N with pad_before zeros in front (replaces F.pad + fftshift,
 * tests/test_utils.py:227-245).  Requires n <= N <= 2^30 and
 * 0 <= pad_before <= N - n. */
int tp_fftshift_pad(int elem_bytes, const void* src, int64_t batch, int dim, int64_t boxsize,
                    int64_t padded_boxsize, int64_t pad_before, void* dst, void* stream);

/* dst = ifftshift over every spatial axis of src[batch, len0, len1(, len2)],
 * keeping indices [crop_start, crop_start + crop_len) of each axis, clipped
 * to the axis like a Python slice (replaces ifftshift + slicing,
 * tests/test_utils.py:271-293).  dst has the clipped lengths.  The adjoint
 * of tp_fftshift_pad with pad_before = crop_start for even lengths. */
int tp_ifftshift_crop(int elem_bytes, const void* src, int64_t batch, int dim, int64_t len0, int64_t len1,
                      int64_t len2, int64_t crop_start, int64_t crop_len, void* dst, void* stream);

/* rfftn with norm="forward" (scaled by 1/boxsize^dim) of `batch` real boxes
 * [batch, boxsize^dim] into [batch, boxsize^(dim-1), boxsize/2+1] complex,
 * both row-major, through hipFFT (rocFFT) with plans cached per shape for the
 * life of the process (replaces torch.fft.rfftn in the reference's recipe,
 * README.md:115-116).  `real` is left unchanged. */
int tp_rfftn(int dtype, int dim, int64_t batch, int64_t boxsize, const void* real, void* spectrum, void* stream);

/* The inverse (irfftn with norm="forward": unscaled) of tp_rfftn's layout.
 * `spectrum` is overwritten (the library's complex-to-real transforms use
 * their input as scratch). */
int tp_irfftn(int dtype, int dim, int64_t batch, int64_t boxsize, void* spectrum, void* real, void* stream);

/* out[e] = data[e] / (weights[e] + reg) component-wise where weights[e] + reg > 0,
 * else 0: a Wiener-style normalisation of a backprojected pair (data complex,
 * weights real, both of `dtype`, `elems` elements).  No counterpart in the
 * reference (its dual data/weight volumes exist for this step,
 * paper/main.tex:72); for callers that reconstruct after backprojection.
 * out may alias data. */
int tp_normalize_reconstruction(int dtype, const void* data, const void* weights, int64_t elems, double reg,
                                void* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TORCH_PROJECTORS_HIP_H */
