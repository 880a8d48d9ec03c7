"""TEST INFRASTRUCTURE — NOT PART OF THE PRODUCT.

ctypes binding of the CPU oracle (oracle/tp_oracle.cpp) with the call
signatures of the reference's dispatcher ops (csrc/torch_projectors.cpp:23-36):
CPU tensors in, CPU tensors out, rotation/shift gradients gated on
`requires_grad` exactly as projection_utils.h:107-131 does.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg import this module.

`ref_ops()` returns the reference's own compiled CPU kernels (oracle/_ref,
built by oracle/build_ref.py) registered under `torch.ops.torch_projectors_ref`,
or None when that build is absent.
"""
import ctypes
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libtp_oracle.so")
REF_LIB_PATH = os.path.join(HERE, "_ref", "libtp_ref.so")

_lib = None
_ref_loaded = False

c_void_p, c_int, c_int64, c_double = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_double


def build():
    """Compile the oracle with its Makefile (g++ only)."""
    import subprocess
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _lib.tpo_last_error.restype = ctypes.c_char_p
        _lib.tpo_backproject_rec_boxsize.restype = c_int64
        _lib.tpo_backproject_rec_boxsize.argtypes = [c_int64, c_double]
    return _lib


def ref_ops():
    """The reference's compiled CPU ops, or None if oracle/_ref was not built."""
    global _ref_loaded
    if not _ref_loaded:
        if not os.path.exists(REF_LIB_PATH):
            return None
        torch.ops.load_library(REF_LIB_PATH)
        _ref_loaded = True
    return torch.ops.torch_projectors_ref


def _p(t):
    return c_void_p(t.data_ptr()) if t is not None else c_void_p(None)


def _i(v):
    return c_int64(int(v))


def _dtype(t):
    if t.dtype == torch.complex64:
        return 0
    if t.dtype == torch.complex128:
        return 1
    raise RuntimeError("complex64 or complex128 expected")


def _interp(s):
    if s == "linear":
        return 0
    if s == "cubic":
        return 1
    raise RuntimeError("Supported interpolation methods: 'linear', 'cubic'")


def _real(t):
    return torch.float32 if t.dtype == torch.complex64 else torch.float64


def _c(t):
    return None if t is None else t.detach().contiguous()


def _call(name, *args):
    f = getattr(lib(), name)
    rc = f(*args)
    if rc != 0:
        raise RuntimeError(lib().tpo_last_error().decode())


def _tail(interpolation, oversampling, cutoff, num_threads):
    return [c_int(_interp(interpolation)), c_double(oversampling), c_int(cutoff is not None),
            c_double(0.0 if cutoff is None else cutoff)]


def rec_boxsize(n, oversampling):
    return int(lib().tpo_backproject_rec_boxsize(n, oversampling))


def project_2d_forw(reconstruction, rotations, shifts, output_shape, interpolation, oversampling,
                    fourier_radius_cutoff, num_threads=0):
    rec, rot, sh = _c(reconstruction), _c(rotations), _c(shifts)
    B, N, H = rec.shape
    n = int(output_shape[0])
    out = torch.empty(B, rot.shape[1], n, n // 2 + 1, dtype=rec.dtype)
    _call("tpo_project_2d_forw", c_int(_dtype(rec)), _p(rec), _i(B), _i(N), _i(H), _p(rot), _i(rot.shape[0]),
          _i(rot.shape[1]), _p(sh), _i(sh.shape[0] if sh is not None else 1), _i(n),
          *_tail(interpolation, oversampling, fourier_radius_cutoff, num_threads), _p(out), c_int(num_threads))
    return out


def project_3d_to_2d_forw(reconstruction, rotations, shifts, output_shape, interpolation, oversampling,
                          fourier_radius_cutoff, num_threads=0):
    rec, rot, sh = _c(reconstruction), _c(rotations), _c(shifts)
    B, D, N, H = rec.shape
    n = int(output_shape[0])
    out = torch.empty(B, rot.shape[1], n, n // 2 + 1, dtype=rec.dtype)
    _call("tpo_project_3d_to_2d_forw", c_int(_dtype(rec)), _p(rec), _i(B), _i(D), _i(N), _i(H), _p(rot),
          _i(rot.shape[0]), _i(rot.shape[1]), _p(sh), _i(sh.shape[0] if sh is not None else 1), _i(n),
          *_tail(interpolation, oversampling, fourier_radius_cutoff, num_threads), _p(out), c_int(num_threads))
    return out


def _grad_outputs(rotations, shifts):
    need_rot = rotations.requires_grad
    need_sh = shifts is not None and shifts.requires_grad
    grot = torch.empty_like(rotations.detach()) if need_rot else torch.empty(0, dtype=rotations.dtype)
    gsh = torch.empty_like(shifts.detach()) if need_sh else torch.empty(0, dtype=rotations.dtype)
    return need_rot, need_sh, grot, gsh


def project_2d_back(grad_projections, reconstruction, rotations, shifts, interpolation, oversampling,
                    fourier_radius_cutoff, num_threads=0):
    g, rec, rot, sh = _c(grad_projections), _c(reconstruction), _c(rotations), _c(shifts)
    B, P, n, hp = g.shape
    _, N, H = rec.shape
    need_rot, need_sh, grot, gsh = _grad_outputs(rotations, shifts)
    grec = torch.empty_like(rec)
    _call("tpo_project_2d_back", c_int(_dtype(rec)), _p(g), _i(B), _i(P), _i(n), _i(hp), _p(rec), _i(N), _i(H),
          _p(rot), _i(rot.shape[0]), _p(sh), _i(sh.shape[0] if sh is not None else 1),
          *_tail(interpolation, oversampling, fourier_radius_cutoff, num_threads), _p(grec),
          _p(grot if need_rot else None), _p(gsh if need_sh else None), c_int(num_threads))
    return grec, grot, gsh


def project_3d_to_2d_back(grad_projections, reconstruction, rotations, shifts, interpolation, oversampling,
                          fourier_radius_cutoff, num_threads=0):
    g, rec, rot, sh = _c(grad_projections), _c(reconstruction), _c(rotations), _c(shifts)
    B, P, n, hp = g.shape
    _, D, N, H = rec.shape
    need_rot, need_sh, grot, gsh = _grad_outputs(rotations, shifts)
    grec = torch.empty_like(rec)
    _call("tpo_project_3d_to_2d_back", c_int(_dtype(rec)), _p(g), _i(B), _i(P), _i(n), _i(hp), _p(rec), _i(D),
          _i(N), _i(H), _p(rot), _i(rot.shape[0]), _p(sh), _i(sh.shape[0] if sh is not None else 1),
          *_tail(interpolation, oversampling, fourier_radius_cutoff, num_threads), _p(grec),
          _p(grot if need_rot else None), _p(gsh if need_sh else None), c_int(num_threads))
    return grec, grot, gsh


def _backproject_forw(fn, dims, projections, weights, rotations, shifts, interpolation, oversampling,
                      fourier_radius_cutoff, num_threads):
    pr, w, rot, sh = _c(projections), _c(weights), _c(rotations), _c(shifts)
    B, P, n, hp = pr.shape
    N = rec_boxsize(n, oversampling)
    shape = (B, N, N // 2 + 1) if dims == 2 else (B, N, N, N // 2 + 1)
    data = torch.empty(shape, dtype=pr.dtype)
    wrec = torch.empty(shape, dtype=w.dtype) if w is not None else torch.empty(0, dtype=rotations.dtype)
    _call(fn, c_int(_dtype(pr)), _p(pr), _i(B), _i(P), _i(n), _i(hp), _p(w), _p(rot), _i(rot.shape[0]), _p(sh),
          _i(sh.shape[0] if sh is not None else 1),
          *_tail(interpolation, oversampling, fourier_radius_cutoff, num_threads), _p(data),
          _p(wrec if w is not None else None), c_int(num_threads))
    return data, wrec


def backproject_2d_forw(projections, weights, rotations, shifts, interpolation, oversampling,
                        fourier_radius_cutoff, num_threads=0):
    return _backproject_forw("tpo_backproject_2d_forw", 2, projections, weights, rotations, shifts, interpolation,
                             oversampling, fourier_radius_cutoff, num_threads)


def backproject_2d_to_3d_forw(projections, weights, rotations, shifts, interpolation, oversampling,
                              fourier_radius_cutoff, num_threads=0):
    return _backproject_forw("tpo_backproject_2d_to_3d_forw", 3, projections, weights, rotations, shifts,
                             interpolation, oversampling, fourier_radius_cutoff, num_threads)


def _backproject_back(fn, grad_data_rec, grad_weight_rec, projections, weights, rotations, shifts, interpolation,
                      oversampling, fourier_radius_cutoff, num_threads):
    gd, gw, pr, w = _c(grad_data_rec), _c(grad_weight_rec), _c(projections), _c(weights)
    rot, sh = _c(rotations), _c(shifts)
    B, P, n, hp = pr.shape
    N, H = gd.shape[-2], gd.shape[-1]
    need_rot, need_sh, grot, gsh = _grad_outputs(rotations, shifts)
    gproj = torch.empty_like(pr)
    gweights = torch.empty_like(w) if w is not None else torch.empty(0, dtype=rotations.dtype)
    _call(fn, c_int(_dtype(pr)), _p(gd), _p(gw), _i(N), _i(H), _p(pr), _i(B), _i(P), _i(n), _i(hp), _p(w),
          _p(rot), _i(rot.shape[0]), _p(sh), _i(sh.shape[0] if sh is not None else 1),
          *_tail(interpolation, oversampling, fourier_radius_cutoff, num_threads), _p(gproj),
          _p(gweights if w is not None else None), _p(grot if need_rot else None), _p(gsh if need_sh else None),
          c_int(num_threads))
    return gproj, gweights, grot, gsh


def backproject_2d_back(grad_data_rec, grad_weight_rec, projections, weights, rotations, shifts, interpolation,
                        oversampling, fourier_radius_cutoff, num_threads=0):
    return _backproject_back("tpo_backproject_2d_back", grad_data_rec, grad_weight_rec, projections, weights,
                             rotations, shifts, interpolation, oversampling, fourier_radius_cutoff, num_threads)


def backproject_2d_to_3d_back(grad_data_rec, grad_weight_rec, projections, weights, rotations, shifts,
                              interpolation, oversampling, fourier_radius_cutoff, num_threads=0):
    return _backproject_back("tpo_backproject_2d_to_3d_back", grad_data_rec, grad_weight_rec, projections, weights,
                             rotations, shifts, interpolation, oversampling, fourier_radius_cutoff, num_threads)


def scatter_wide(op, args, num_threads=0):
    """The scatter volumes of `op` (project_*_back's reconstruction gradient, backproject_*_forw's data and
    weight volumes) for fp32 inputs, summed in double (tpo_*_wide in tp_oracle.cpp): the same fp32 tap
    values as the op, each cell their exact sum.  `args` are the dispatcher op's positional arguments.
    Returns a tuple of complex128 / float64 tensors in the op's output order (volumes only)."""
    if op in ("project_2d_back", "project_3d_to_2d_back"):
        gproj, rec, rot, sh, interp, os_, cut = args
        g, rec, rot, sh = _c(gproj), _c(rec), _c(rot), _c(sh)
        B, P, n, hp = g.shape
        grec = torch.empty(rec.shape, dtype=torch.complex128)
        shape = [_i(x) for x in rec.shape[1:]]
        _call(f"tpo_{op}_wide", _p(g), _i(B), _i(P), _i(n), _i(hp), _p(rec), *shape, _p(rot), _i(rot.shape[0]),
              _p(sh), _i(sh.shape[0] if sh is not None else 1), *_tail(interp, os_, cut, num_threads), _p(grec),
              c_int(num_threads))
        return (grec,)
    if op in ("backproject_2d_forw", "backproject_2d_to_3d_forw"):
        proj, w, rot, sh, interp, os_, cut = args
        pr, w, rot, sh = _c(proj), _c(w), _c(rot), _c(sh)
        B, P, n, hp = pr.shape
        N = rec_boxsize(n, os_)
        shape = (B, N, N // 2 + 1) if op == "backproject_2d_forw" else (B, N, N, N // 2 + 1)
        data = torch.empty(shape, dtype=torch.complex128)
        wrec = torch.empty(shape, dtype=torch.float64) if w is not None else None
        _call(f"tpo_{op}_wide", _p(pr), _i(B), _i(P), _i(n), _i(hp), _p(w), _p(rot), _i(rot.shape[0]), _p(sh),
              _i(sh.shape[0] if sh is not None else 1), *_tail(interp, os_, cut, num_threads), _p(data), _p(wrec),
              c_int(num_threads))
        return (data,) if wrec is None else (data, wrec)
    raise ValueError(f"{op} has no scatter volume")


OPS = ["project_2d_forw", "project_2d_back", "backproject_2d_forw", "backproject_2d_back",
       "project_3d_to_2d_forw", "project_3d_to_2d_back", "backproject_2d_to_3d_forw", "backproject_2d_to_3d_back"]
