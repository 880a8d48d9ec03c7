"""Drive the HIP library through its C ABI with the oracle's call signatures.

Each function takes the arguments of the matching dispatcher op (CPU or GPU
tensors), copies them to `cuda:0`, calls the `tp_*` entry point through
ctypes on PyTorch's current stream, synchronises, and returns CPU tensors
shaped like the oracle's outputs (oracle/oracle.py), so a test can compare
the two directly.  Rotation/shift gradients are requested exactly when the
input tensors require grad, as the reference does (projection_utils.h:107-131).
"""
import ctypes

import torch

from torch_projectors import capi

DEV = "cuda:0"
_P = ctypes.c_void_p


def _dt(t):
    if t.dtype == torch.complex64:
        return capi.TP_F32
    if t.dtype == torch.complex128:
        return capi.TP_F64
    if t.dtype == torch.complex32:  # a complex-half volume (the projections and their gradients)
        return capi.TP_F16S
    raise RuntimeError("complex64, complex128 or (volume) complex32 expected")


def _proj_dtype(rec):
    return torch.complex64 if rec.dtype == torch.complex32 else rec.dtype


def _interp(s):
    return {"linear": capi.TP_LINEAR, "cubic": capi.TP_CUBIC}[s]


def _g(t):
    return None if t is None else t.detach().to(DEV).contiguous()


def _p(t):
    return _P(t.data_ptr()) if t is not None else _P(None)


def _stream():
    return _P(torch.cuda.current_stream().cuda_stream)


def _tail(interpolation, oversampling, cutoff):
    return [_interp(interpolation), float(oversampling), int(cutoff is not None),
            0.0 if cutoff is None else float(cutoff)]


def _done(*outs):
    torch.cuda.synchronize()
    res = tuple(o.cpu() if o is not None else None for o in outs)
    return res[0] if len(res) == 1 else res


def _poisoned(shape, dtype):
    """An output buffer filled with NaN: every entry point writes every element of its outputs, so an
    element left unwritten shows up as a NaN in the comparison instead of passing on stale zeros."""
    fill = complex(float("nan"), float("nan")) if dtype.is_complex else float("nan")
    return torch.full(tuple(shape), fill, dtype=dtype, device=DEV)


def _grad_outputs(rotations, shifts, like):
    need_rot = rotations.requires_grad
    need_sh = shifts is not None and shifts.requires_grad
    grot = _poisoned(rotations.shape, rotations.dtype) if need_rot else None
    gsh = _poisoned(shifts.shape, shifts.dtype) if need_sh else None
    return grot, gsh


def _empty_like_cpu(t, dtype):
    return t if t is not None else torch.empty(0, dtype=dtype)


def project_2d_forw(reconstruction, rotations, shifts, output_shape, interpolation, oversampling,
                    fourier_radius_cutoff):
    rec, rot, sh = _g(reconstruction), _g(rotations), _g(shifts)
    B, N, H = rec.shape
    n = int(output_shape[0])
    out = _poisoned((B, rot.shape[1], n, n // 2 + 1), _proj_dtype(rec))
    capi.call("tp_project_2d_forw", _dt(rec), _p(rec), B, N, H, _p(rot), rot.shape[0], rot.shape[1], _p(sh),
              sh.shape[0] if sh is not None else 1, n, *_tail(interpolation, oversampling, fourier_radius_cutoff),
              _p(out), _stream())
    return _done(out)


def project_3d_to_2d_forw(reconstruction, rotations, shifts, output_shape, interpolation, oversampling,
                          fourier_radius_cutoff):
    rec, rot, sh = _g(reconstruction), _g(rotations), _g(shifts)
    B, D, N, H = rec.shape
    n = int(output_shape[0])
    out = _poisoned((B, rot.shape[1], n, n // 2 + 1), _proj_dtype(rec))
    capi.call("tp_project_3d_to_2d_forw", _dt(rec), _p(rec), B, D, N, H, _p(rot), rot.shape[0], rot.shape[1],
              _p(sh), sh.shape[0] if sh is not None else 1, n,
              *_tail(interpolation, oversampling, fourier_radius_cutoff), _p(out), _stream())
    return _done(out)


def _project_back(name, dims, grad_projections, reconstruction, rotations, shifts, interpolation, oversampling,
                  fourier_radius_cutoff):
    g, rec, rot, sh = _g(grad_projections), _g(reconstruction), _g(rotations), _g(shifts)
    B, P, n, hp = g.shape
    grec = _poisoned(rec.shape, _proj_dtype(rec))  # complex64 for a complex-half volume
    grot, gsh = _grad_outputs(rotations, shifts, grec)
    rec_dims = list(rec.shape[1:])
    capi.call(name, _dt(rec), _p(g), B, P, n, hp, _p(rec), *rec_dims, _p(rot), rot.shape[0], _p(sh),
              sh.shape[0] if sh is not None else 1, *_tail(interpolation, oversampling, fourier_radius_cutoff),
              _p(grec), _p(grot), _p(gsh), _stream())
    grec, grot, gsh = _done(grec, grot, gsh)
    rdt = rotations.dtype
    return grec, _empty_like_cpu(grot, rdt), _empty_like_cpu(gsh, rdt)


def project_2d_back(*args):
    return _project_back("tp_project_2d_back", 2, *args)


def project_3d_to_2d_back(*args):
    return _project_back("tp_project_3d_to_2d_back", 3, *args)


def _backproject_forw(name, dims, projections, weights, rotations, shifts, interpolation, oversampling,
                      fourier_radius_cutoff):
    pr, w, rot, sh = _g(projections), _g(weights), _g(rotations), _g(shifts)
    B, P, n, hp = pr.shape
    N = capi.rec_boxsize(n, oversampling)
    shape = (B, N, N // 2 + 1) if dims == 2 else (B, N, N, N // 2 + 1)
    data = _poisoned(shape, pr.dtype)
    wrec = _poisoned(shape, w.dtype) if w is not None else None
    capi.call(name, _dt(pr), _p(pr), B, P, n, hp, _p(w), _p(rot), rot.shape[0], _p(sh),
              sh.shape[0] if sh is not None else 1, *_tail(interpolation, oversampling, fourier_radius_cutoff),
              _p(data), _p(wrec), _stream())
    data, wrec = _done(data, wrec)
    return data, _empty_like_cpu(wrec, rotations.dtype)


def backproject_2d_forw(*args):
    return _backproject_forw("tp_backproject_2d_forw", 2, *args)


def backproject_2d_to_3d_forw(*args):
    return _backproject_forw("tp_backproject_2d_to_3d_forw", 3, *args)


def _backproject_back(name, grad_data_rec, grad_weight_rec, projections, weights, rotations, shifts, interpolation,
                      oversampling, fourier_radius_cutoff):
    gd, gw, pr, w = _g(grad_data_rec), _g(grad_weight_rec), _g(projections), _g(weights)
    rot, sh = _g(rotations), _g(shifts)
    B, P, n, hp = pr.shape
    N, H = gd.shape[-2], gd.shape[-1]
    gproj = _poisoned(pr.shape, pr.dtype)
    gweights = _poisoned(w.shape, w.dtype) if w is not None else None
    grot, gsh = _grad_outputs(rotations, shifts, pr)
    capi.call(name, _dt(pr), _p(gd), _p(gw), N, H, _p(pr), B, P, n, hp, _p(w), _p(rot), rot.shape[0], _p(sh),
              sh.shape[0] if sh is not None else 1, *_tail(interpolation, oversampling, fourier_radius_cutoff),
              _p(gproj), _p(gweights), _p(grot), _p(gsh), _stream())
    gproj, gweights, grot, gsh = _done(gproj, gweights, grot, gsh)
    rdt = rotations.dtype
    return gproj, _empty_like_cpu(gweights, rdt), _empty_like_cpu(grot, rdt), _empty_like_cpu(gsh, rdt)


def backproject_2d_back(*args):
    return _backproject_back("tp_backproject_2d_back", *args)


def backproject_2d_to_3d_back(*args):
    return _backproject_back("tp_backproject_2d_to_3d_back", *args)
