"""TEST INFRASTRUCTURE — the CPU oracle behind the public operator signatures.

The four differentiable operators of the reference's Python API
(torch_projectors/ops.py:29-264 of the reference) with the oracle's forward
and backward functions under torch.autograd, so the property checks of
tests/reference_props.py run on the CPU restatement as they do on the HIP
operators; pad_and_fftshift and ifftshift_and_crop are oracle/fourier.py's.  Rotation/shift gradients are requested exactly when autograd
needs them, as the reference's backward does (ops.py:430-514).  Tensors are
CPU tensors; poses are [B_rot, P, d, d] and shifts [B_shift, P, 2].
"""
from oracle import fourier as OF
from oracle import oracle as O

import torch


# A test may set this to f(kind, grads) -> grads to plant a mistake in the
# oracle's backward and show that a check notices it; kind is "project" or
# "backproject", grads the tuple the oracle's backward function returned.
plant = None


def _planted(kind, grads):
    return grads if plant is None else plant(kind, grads)


def _need(t, flag):
    return None if t is None else t.detach().requires_grad_(bool(flag))


class _Project(torch.autograd.Function):
    @staticmethod
    def forward(ctx, forw, back, reconstruction, rotations, shifts, output_shape, interpolation, oversampling,
                cutoff):
        ctx.back, ctx.tail = back, (interpolation, oversampling, cutoff)
        ctx.save_for_backward(reconstruction, rotations, shifts)
        return forw(reconstruction.detach(), rotations.detach(), None if shifts is None else shifts.detach(),
                    output_shape, interpolation, oversampling, cutoff)

    @staticmethod
    def backward(ctx, grad):
        rec, rot, sh = ctx.saved_tensors
        need = ctx.needs_input_grad
        g_rec, g_rot, g_sh = _planted("project", ctx.back(grad.contiguous(), rec.detach(), _need(rot, need[3]),
                                                          _need(sh, need[4]), *ctx.tail))
        return (None, None, g_rec, g_rot if need[3] else None, g_sh if need[4] else None,
                None, None, None, None)


class _Backproject(torch.autograd.Function):
    @staticmethod
    def forward(ctx, forw, back, projections, weights, rotations, shifts, interpolation, oversampling, cutoff):
        ctx.back, ctx.tail = back, (interpolation, oversampling, cutoff)
        ctx.save_for_backward(projections, weights, rotations, shifts)
        return forw(projections.detach(), None if weights is None else weights.detach(), rotations.detach(),
                    None if shifts is None else shifts.detach(), interpolation, oversampling, cutoff)

    @staticmethod
    def backward(ctx, g_data, g_weight):
        proj, w, rot, sh = ctx.saved_tensors
        need = ctx.needs_input_grad
        if g_weight is not None and (w is None or g_weight.numel() == 0):
            g_weight = None
        g_proj, g_w, g_rot, g_sh = _planted("backproject", ctx.back(
            g_data.contiguous(), None if g_weight is None else g_weight.contiguous(), proj.detach(),
            None if w is None else w.detach(), _need(rot, need[4]), _need(sh, need[5]), *ctx.tail))
        return (None, None, g_proj, g_w if (w is not None and need[3]) else None,
                g_rot if need[4] else None, g_sh if need[5] else None, None, None, None)


def project_2d_forw(reconstruction, rotations, shifts=None, output_shape=None, interpolation="linear",
                    oversampling=1.0, fourier_radius_cutoff=None):
    n = reconstruction.shape[-2]
    shape = tuple(output_shape) if output_shape is not None else (n, n)
    return _Project.apply(O.project_2d_forw, O.project_2d_back, reconstruction, rotations, shifts, shape,
                          interpolation, oversampling, fourier_radius_cutoff)


def project_3d_to_2d_forw(reconstruction, rotations, shifts=None, output_shape=None, interpolation="linear",
                          oversampling=1.0, fourier_radius_cutoff=None):
    n = reconstruction.shape[-2]
    shape = tuple(output_shape) if output_shape is not None else (n, n)
    return _Project.apply(O.project_3d_to_2d_forw, O.project_3d_to_2d_back, reconstruction, rotations, shifts,
                          shape, interpolation, oversampling, fourier_radius_cutoff)


def backproject_2d_forw(projections, rotations, weights=None, shifts=None, interpolation="linear",
                        oversampling=1.0, fourier_radius_cutoff=None):
    return _Backproject.apply(O.backproject_2d_forw, O.backproject_2d_back, projections, weights, rotations,
                              shifts, interpolation, oversampling, fourier_radius_cutoff)


def backproject_2d_to_3d_forw(projections, rotations, weights=None, shifts=None, interpolation="linear",
                              oversampling=1.0, fourier_radius_cutoff=None):
    return _Backproject.apply(O.backproject_2d_to_3d_forw, O.backproject_2d_to_3d_back, projections, weights,
                              rotations, shifts, interpolation, oversampling, fourier_radius_cutoff)


def pad_and_fftshift(tensor, oversampling_factor):
    return torch.from_numpy(OF.pad_and_fftshift(tensor.detach().cpu().numpy(), oversampling_factor))


def ifftshift_and_crop(real_tensor, oversampling_factor):
    return torch.from_numpy(OF.ifftshift_and_crop(real_tensor.detach().cpu().numpy(), oversampling_factor).copy())
