"""Public API and autograd wiring of the projector operators.

Signatures, defaults, argument checks (ValueError) and autograd behaviour
follow the reference's torch_projectors/ops.py:
  - project_2d_forw / project_3d_to_2d_forw          ops.py:6-38, 119-174
  - backproject_2d_forw / backproject_2d_to_3d_forw  ops.py:61-117, 208-264
  - project_2d_back / project_3d_to_2d_back          ops.py:40-59, 176-206
  - backproject_2d_to_3d_back                        ops.py:266-296
  - autograd Functions                               ops.py:300-514
  - no-op autograd registrations of the other ops    ops.py:516-574
The arithmetic runs in `torch.ops.torch_projectors.*` (the HIP library).
"""
from typing import Optional

import torch

_OPS = torch.ops.torch_projectors


# ----------------------------------------------------------------------------- checks
def _check_rfft_box(boxsize, boxsize_half, what):
    if boxsize % 2 != 0:
        raise ValueError(f"{what} ({boxsize}) must be even. Only even dimensions are supported.")
    if boxsize != (boxsize_half - 1) * 2:
        noun = "Reconstruction" if what == "Boxsize" else "Projection"
        raise ValueError(f"{noun} shape mismatch: expected boxsize {boxsize} to match "
                         f"2*(boxsize_half-1) = {(boxsize_half - 1) * 2}")


def _resolve_output_shape(output_shape, boxsize):
    if output_shape is None:
        return (boxsize, boxsize)
    if len(output_shape) != 2 or output_shape[0] != output_shape[1]:
        raise ValueError(f"Output shape {output_shape} must be square (height == width)")
    if output_shape[0] % 2 != 0:
        raise ValueError(f"Output boxsize {output_shape[0]} must be even")
    return output_shape


def _check_projections(projections, weights):
    if projections.dim() != 4:
        raise ValueError("Projections must be a 4D tensor (B, P, height, width/2+1)")
    _, _, n, n_half = projections.shape
    _check_rfft_box(n, n_half, "Projection boxsize")
    if weights is not None:
        if weights.shape != projections.shape:
            raise ValueError(f"Weights shape {weights.shape} must match projections shape {projections.shape}")
        if not weights.is_floating_point():
            raise ValueError("Weights must be real-valued (floating point)")


def _batched_poses(rotations, shifts):
    """Prepend the batch dims the dispatcher ops expect: [B_rot, P, k, k] and [B_shift, P, 2]."""
    while rotations.dim() < 4:
        rotations = rotations.unsqueeze(0)
    if shifts is not None:
        while shifts.dim() < 3:
            shifts = shifts.unsqueeze(0)
    return rotations, shifts


def _check_rot_batch(rotations, B, what):
    if rotations.size(0) != B and rotations.size(0) != 1:
        raise ValueError(f"Batch size of rotations must be 1 or match {what}")


# ----------------------------------------------------------------------------- public API
def project_2d_forw(reconstruction: torch.Tensor, rotations: torch.Tensor, shifts: Optional[torch.Tensor] = None,
                    output_shape: Optional[tuple] = None, interpolation: str = 'linear',
                    oversampling: float = 1.0, fourier_radius_cutoff: Optional[float] = None) -> torch.Tensor:
    """Project 2D Fourier reconstructions [B, H, W/2+1] to rotated, shifted 2D
    projections [B, P, n, n/2+1] (rotations [B_rot, P, 2, 2], shifts [B_shift, P, 2])."""
    if reconstruction.dim() < 2:
        raise ValueError("Reconstruction must have at least 2 dimensions")
    _check_rfft_box(reconstruction.shape[-2], reconstruction.shape[-1], "Boxsize")
    output_shape = _resolve_output_shape(output_shape, reconstruction.shape[-2])
    return _Project2D.apply(reconstruction, rotations, shifts, output_shape, interpolation, oversampling,
                            fourier_radius_cutoff)


def project_2d_back(projections: torch.Tensor, reconstruction: torch.Tensor, rotations: torch.Tensor,
                    shifts: Optional[torch.Tensor] = None, interpolation: str = 'linear',
                    oversampling: float = 1.0) -> torch.Tensor:
    """Gradient of project_2d_forw w.r.t. the reconstruction only."""
    grad_reconstruction, _, _ = _OPS.project_2d_back(projections, reconstruction, rotations, shifts, interpolation,
                                                     oversampling, None)
    return grad_reconstruction


def backproject_2d_forw(projections: torch.Tensor, rotations: torch.Tensor, weights: Optional[torch.Tensor] = None,
                        shifts: Optional[torch.Tensor] = None, interpolation: str = 'linear',
                        oversampling: float = 1.0, fourier_radius_cutoff: Optional[float] = None):
    """Accumulate 2D projections [B, P, n, n/2+1] (and optional real weights of the
    same shape) into 2D reconstructions [B, N, N/2+1], N = ceil(n*os) rounded up to
    even.  Returns (data_reconstruction, weight_reconstruction or an empty tensor)."""
    _check_projections(projections, weights)
    return _Backproject2D.apply(projections, weights, rotations, shifts, interpolation, oversampling,
                                fourier_radius_cutoff)


def project_3d_to_2d_forw(reconstruction: torch.Tensor, rotations: torch.Tensor,
                          shifts: Optional[torch.Tensor] = None, output_shape: Optional[tuple] = None,
                          interpolation: str = 'linear', oversampling: float = 1.0,
                          fourier_radius_cutoff: Optional[float] = None) -> torch.Tensor:
    """Central-slice projection of 3D Fourier volumes [B, D, H, W/2+1] to 2D
    projections [B, P, n, n/2+1] (rotations [B_rot, P, 3, 3], shifts [B_shift, P, 2])."""
    if reconstruction.dim() != 4:
        raise ValueError("Reconstruction must be a 4D tensor (B, D, H, W/2+1)")
    _check_rfft_box(reconstruction.shape[2], reconstruction.shape[3], "Boxsize")
    output_shape = _resolve_output_shape(output_shape, reconstruction.shape[2])
    return _Project3DTo2D.apply(reconstruction, rotations, shifts, output_shape, interpolation, oversampling,
                                fourier_radius_cutoff)


def project_3d_to_2d_back(projections: torch.Tensor, reconstruction: torch.Tensor, rotations: torch.Tensor,
                          shifts: Optional[torch.Tensor] = None, interpolation: str = 'linear',
                          oversampling: float = 1.0) -> torch.Tensor:
    """Gradient of project_3d_to_2d_forw w.r.t. the 3D reconstruction only."""
    grad_reconstruction, _, _ = _OPS.project_3d_to_2d_back(projections, reconstruction, rotations, shifts,
                                                           interpolation, oversampling, None)
    return grad_reconstruction


def backproject_2d_to_3d_forw(projections: torch.Tensor, rotations: torch.Tensor,
                              weights: Optional[torch.Tensor] = None, shifts: Optional[torch.Tensor] = None,
                              interpolation: str = 'linear', oversampling: float = 1.0,
                              fourier_radius_cutoff: Optional[float] = None):
    """Accumulate 2D projections [B, P, n, n/2+1] (and optional real weights) into
    3D volumes [B, N, N, N/2+1] through the central-slice theorem.  Returns
    (data_reconstruction, weight_reconstruction or an empty tensor)."""
    _check_projections(projections, weights)
    return _Backproject2DTo3D.apply(projections, weights, rotations, shifts, interpolation, oversampling,
                                    fourier_radius_cutoff)


def backproject_2d_to_3d_back(reconstruction: torch.Tensor, projections: torch.Tensor, rotations: torch.Tensor,
                              shifts: Optional[torch.Tensor] = None, interpolation: str = 'linear',
                              oversampling: float = 1.0) -> torch.Tensor:
    """Gradient of backproject_2d_to_3d_forw w.r.t. the projections, given the
    gradient `reconstruction` of the data volume.

    The reference's wrapper (ops.py:266-296) passes 7 arguments to the 9-argument
    schema and cannot be called; this one passes no weights and no weight gradient,
    which is what its docstring describes."""
    grad_projections, _, _, _ = _OPS.backproject_2d_to_3d_back(reconstruction, None, projections, None, rotations,
                                                               shifts, interpolation, oversampling, None)
    return grad_projections


# ----------------------------------------------------------------------------- autograd
class _Project2D(torch.autograd.Function):
    @staticmethod
    def forward(ctx, reconstruction, rotations, shifts, output_shape, interpolation, oversampling,
                fourier_radius_cutoff):
        if reconstruction.dim() == 2:
            reconstruction = reconstruction.unsqueeze(0)
        rotations, shifts = _batched_poses(rotations, shifts)
        _check_rot_batch(rotations, reconstruction.size(0), "reconstruction")
        projection = _OPS.project_2d_forw(reconstruction, rotations, shifts, output_shape, interpolation,
                                          oversampling, fourier_radius_cutoff)
        ctx.save_for_backward(reconstruction, rotations, shifts)
        ctx.interpolation, ctx.oversampling, ctx.fourier_radius_cutoff = interpolation, oversampling, \
            fourier_radius_cutoff
        return projection

    @staticmethod
    def backward(ctx, grad_output):
        reconstruction, rotations, shifts = ctx.saved_tensors
        g_rec, g_rot, g_shift = _OPS.project_2d_back(grad_output.contiguous(), reconstruction, rotations, shifts,
                                                     ctx.interpolation, ctx.oversampling, ctx.fourier_radius_cutoff)
        return g_rec, g_rot, (None if shifts is None else g_shift), None, None, None, None


class _Project3DTo2D(torch.autograd.Function):
    @staticmethod
    def forward(ctx, reconstruction, rotations, shifts, output_shape, interpolation, oversampling,
                fourier_radius_cutoff):
        if reconstruction.dim() == 3:
            reconstruction = reconstruction.unsqueeze(0)
        rotations, shifts = _batched_poses(rotations, shifts)
        _check_rot_batch(rotations, reconstruction.size(0), "reconstruction")
        projection = _OPS.project_3d_to_2d_forw(reconstruction, rotations, shifts, output_shape, interpolation,
                                                oversampling, fourier_radius_cutoff)
        ctx.save_for_backward(reconstruction, rotations, shifts)
        ctx.interpolation, ctx.oversampling, ctx.fourier_radius_cutoff = interpolation, oversampling, \
            fourier_radius_cutoff
        return projection

    @staticmethod
    def backward(ctx, grad_output):
        reconstruction, rotations, shifts = ctx.saved_tensors
        g_rec, g_rot, g_shift = _OPS.project_3d_to_2d_back(grad_output.contiguous(), reconstruction, rotations,
                                                           shifts, ctx.interpolation, ctx.oversampling,
                                                           ctx.fourier_radius_cutoff)
        return g_rec, g_rot, (None if shifts is None else g_shift), None, None, None, None


class _BackprojectBase(torch.autograd.Function):
    """Shared forward/backward of the two backprojection Functions."""
    _forw = None
    _back = None

    @classmethod
    def _forward(cls, ctx, projections, weights, rotations, shifts, interpolation, oversampling,
                 fourier_radius_cutoff):
        if projections.dim() == 3:
            projections = projections.unsqueeze(0)
        rotations, shifts = _batched_poses(rotations, shifts)
        if weights is not None and weights.dim() == 3:
            weights = weights.unsqueeze(0)
        _check_rot_batch(rotations, projections.size(0), "projections")
        data, weight = cls._forw(projections, weights, rotations, shifts, interpolation, oversampling,
                                 fourier_radius_cutoff)
        ctx.save_for_backward(projections, weights, rotations, shifts)
        ctx.interpolation, ctx.oversampling, ctx.fourier_radius_cutoff = interpolation, oversampling, \
            fourier_radius_cutoff
        return data, weight

    @classmethod
    def _backward(cls, ctx, grad_data_rec, grad_weight_rec):
        projections, weights, rotations, shifts = ctx.saved_tensors
        if grad_weight_rec is not None and grad_weight_rec.numel() == 0:
            grad_weight_rec = None
        g_proj, g_w, g_rot, g_shift = cls._back(
            grad_data_rec.contiguous(), grad_weight_rec.contiguous() if grad_weight_rec is not None else None,
            projections, weights, rotations, shifts, ctx.interpolation, ctx.oversampling, ctx.fourier_radius_cutoff)
        return (g_proj, None if weights is None else g_w, g_rot, None if shifts is None else g_shift,
                None, None, None)


class _Backproject2D(_BackprojectBase):
    _forw = staticmethod(_OPS.backproject_2d_forw)
    _back = staticmethod(_OPS.backproject_2d_back)

    @staticmethod
    def forward(ctx, projections, weights, rotations, shifts, interpolation, oversampling, fourier_radius_cutoff):
        return _Backproject2D._forward(ctx, projections, weights, rotations, shifts, interpolation, oversampling,
                                       fourier_radius_cutoff)

    @staticmethod
    def backward(ctx, grad_data_rec, grad_weight_rec):
        return _Backproject2D._backward(ctx, grad_data_rec, grad_weight_rec)


class _Backproject2DTo3D(_BackprojectBase):
    _forw = staticmethod(_OPS.backproject_2d_to_3d_forw)
    _back = staticmethod(_OPS.backproject_2d_to_3d_back)

    @staticmethod
    def forward(ctx, projections, weights, rotations, shifts, interpolation, oversampling, fourier_radius_cutoff):
        return _Backproject2DTo3D._forward(ctx, projections, weights, rotations, shifts, interpolation,
                                           oversampling, fourier_radius_cutoff)

    @staticmethod
    def backward(ctx, grad_data_rec, grad_weight_rec):
        return _Backproject2DTo3D._backward(ctx, grad_data_rec, grad_weight_rec)


# The ops that are only reached from the Functions above get no-op autograd
# registrations, as in the reference (ops.py:516-574).
def _no_grad_backward(ctx, *grads):
    return None


for _name in ("project_2d_back", "backproject_2d_forw", "backproject_2d_back", "project_3d_to_2d_back",
              "backproject_2d_to_3d_forw", "backproject_2d_to_3d_back"):
    torch.library.register_autograd(f"torch_projectors::{_name}", _no_grad_backward,
                                    setup_context=lambda ctx, inputs, output: None)
