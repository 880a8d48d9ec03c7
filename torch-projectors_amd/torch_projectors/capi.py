"""ctypes binding of the C ABI in include/torch_projectors_hip.h.

This is the boundary a non-PyTorch host binds: plain pointers, sizes and a
stream, no torch types.  `lib()` loads libtorch_projectors_hip.so
and declares every entry point; `call(name, *args)` invokes one and raises
RuntimeError with tp_last_error() on a non-zero return.  `EXPORTS` lists the
symbols the header declares.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY_PATH = os.path.join(_HERE, "libtorch_projectors_hip.so")

TP_OK, TP_ERR_INVALID, TP_ERR_HIP = 0, 1, 2
TP_F32, TP_F64, TP_F16S = 0, 1, 2
TP_LINEAR, TP_CUBIC = 0, 1

_P, _I, _L, _D = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_double

# name -> argument types, in header order
SIGNATURES = {
    "tp_project_2d_forw": [_I, _P, _L, _L, _L, _P, _L, _L, _P, _L, _L, _I, _D, _I, _D, _P, _P],
    "tp_project_2d_back": [_I, _P, _L, _L, _L, _L, _P, _L, _L, _P, _L, _P, _L, _I, _D, _I, _D, _P, _P, _P, _P],
    "tp_backproject_2d_forw": [_I, _P, _L, _L, _L, _L, _P, _P, _L, _P, _L, _I, _D, _I, _D, _P, _P, _P],
    "tp_backproject_2d_back": [_I, _P, _P, _L, _L, _P, _L, _L, _L, _L, _P, _P, _L, _P, _L, _I, _D, _I, _D,
                               _P, _P, _P, _P, _P],
    "tp_project_3d_to_2d_forw": [_I, _P, _L, _L, _L, _L, _P, _L, _L, _P, _L, _L, _I, _D, _I, _D, _P, _P],
    "tp_project_3d_to_2d_forw_noalloc": [_I, _P, _L, _L, _L, _L, _P, _L, _L, _P, _L, _L, _I, _D, _I, _D, _P, _P],
    "tp_project_3d_to_2d_back": [_I, _P, _L, _L, _L, _L, _P, _L, _L, _L, _P, _L, _P, _L, _I, _D, _I, _D,
                                 _P, _P, _P, _P],
    "tp_backproject_2d_to_3d_forw": [_I, _P, _L, _L, _L, _L, _P, _P, _L, _P, _L, _I, _D, _I, _D, _P, _P, _P],
    "tp_backproject_2d_to_3d_back": [_I, _P, _P, _L, _L, _P, _L, _L, _L, _L, _P, _P, _L, _P, _L, _I, _D, _I,
                                     _D, _P, _P, _P, _P, _P],
    # reference preparation
    "tp_fftshift_pad": [_I, _P, _L, _I, _L, _L, _L, _P, _P],
    "tp_ifftshift_crop": [_I, _P, _L, _I, _L, _L, _L, _L, _L, _P, _P],
    "tp_rfftn": [_I, _I, _L, _L, _P, _P, _P],
    "tp_irfftn": [_I, _I, _L, _L, _P, _P, _P],
    "tp_normalize_reconstruction": [_I, _P, _P, _L, _D, _P, _P],
}
# helpers returning a size: name -> argument types
SIZE_HELPERS = {
    "tp_backproject_rec_boxsize": [_L, _D],
    "tp_padded_boxsize": [_L, _D],
    "tp_cropped_boxsize": [_L, _D],
}
EXPORTS = ["tp_last_error", "tp_abi_version", *SIZE_HELPERS, *SIGNATURES]

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY_PATH):
            raise ImportError(f"{LIBRARY_PATH} not built; run `python torch-projectors_amd/build.py`")
        L = ctypes.CDLL(LIBRARY_PATH)
        L.tp_last_error.restype = ctypes.c_char_p
        L.tp_last_error.argtypes = []
        L.tp_abi_version.restype = ctypes.c_int
        L.tp_abi_version.argtypes = []
        for name, argtypes in SIZE_HELPERS.items():
            f = getattr(L, name)
            f.restype = ctypes.c_int64
            f.argtypes = argtypes
        for name, argtypes in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = ctypes.c_int
            f.argtypes = argtypes
        _lib = L
    return _lib


def call(name, *args):
    rc = getattr(lib(), name)(*args)
    if rc != TP_OK:
        raise RuntimeError(f"{name} failed ({rc}): {lib().tp_last_error().decode()}")


def rec_boxsize(n, oversampling):
    return int(lib().tp_backproject_rec_boxsize(int(n), float(oversampling)))


def padded_boxsize(n, oversampling):
    return int(lib().tp_padded_boxsize(int(n), float(oversampling)))


def cropped_boxsize(n, oversampling):
    return int(lib().tp_cropped_boxsize(int(n), float(oversampling)))
