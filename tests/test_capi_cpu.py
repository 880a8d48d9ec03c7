"""The C ABI library without a GPU: it loads, exports every symbol that
include/torch_projectors_hip.h declares, and rejects invalid arguments before
anything is enqueued (no compute call needs a device)."""
import ctypes
import glob
import os
import re

import pytest

from torch_projectors import capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = glob.glob(os.path.join(ROOT, "include", "*.h"))
_P = ctypes.c_void_p


def declared_symbols():
    names = set()
    for h in HEADERS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(tp_\w+)\s*\(", text))
    return names


def test_every_declared_symbol_is_exported():
    lib = capi.lib()
    declared = declared_symbols()
    assert declared, "no declarations found"
    assert declared == set(capi.EXPORTS), declared ^ set(capi.EXPORTS)
    for name in declared:
        assert hasattr(lib, name), name


def test_abi_version_and_rec_box():
    assert capi.lib().tp_abi_version() == 1
    from oracle import oracle as O
    for n in (8, 12, 64, 128, 256):
        for os_ in (1.0, 1.5, 2.0, 2.5, 3.0):
            assert capi.rec_boxsize(n, os_) == O.rec_boxsize(n, os_)
    assert capi.rec_boxsize(256, 2.0) == 512
    assert capi.rec_boxsize(15, 1.0) == 16


def _forw3(**kw):
    a = dict(dtype=0, rec=_P(8), B=1, D=16, N=16, H=9, rot=_P(8), B_rot=1, P=2, shifts=_P(None), B_shift=1, n=8,
             interp=0, os=1.0, has_cut=0, cut=0.0, out=_P(8), stream=_P(None))
    a.update(kw)
    return capi.lib().tp_project_3d_to_2d_forw(*a.values())


@pytest.mark.parametrize("kw,msg", [
    (dict(dtype=7), "dtype"),
    (dict(interp=5), "interpolation"),
    (dict(B_rot=3, B=2), "rotations"),
    (dict(shifts=_P(8), B_shift=3, B=2, B_rot=2), "shifts"),
    (dict(D=8), "depth"),
    (dict(H=10), "boxsize/2+1"),
    (dict(n=0), "projection box"),
    (dict(N=1, D=1, H=1), "at least 2"),
    (dict(rec=_P(None)), "reconstruction"),
])
def test_invalid_arguments_rejected(kw, msg):
    rc = _forw3(**kw)
    assert rc == capi.TP_ERR_INVALID
    assert msg in capi.lib().tp_last_error().decode()


def test_backprojection_weights_pairing_rejected():
    lib = capi.lib()
    rc = lib.tp_backproject_2d_to_3d_forw(0, _P(8), 1, 1, 8, 5, _P(8), _P(8), 1, _P(None), 1, 0, 2.0, 0, 0.0,
                                          _P(8), _P(None), _P(None))
    assert rc == capi.TP_ERR_INVALID
    assert "weight_reconstruction" in lib.tp_last_error().decode()


def test_volume_limit_rejected():
    # 2048^2 * 1025 elements per batch item exceeds the 32-bit in-volume offset range
    rc = _forw3(N=2048, D=2048, H=1025)
    assert rc == capi.TP_ERR_INVALID
    assert "too large" in capi.lib().tp_last_error().decode()


@pytest.mark.parametrize("kw,msg", [
    (dict(dtype=capi.TP_F16S, interp=5), "interpolation"),
    (dict(dtype=capi.TP_F16S, D=8), "depth"),
    (dict(dtype=capi.TP_F16S, rec=_P(None)), "reconstruction"),
])
def test_half_volume_forward_checks_arguments(kw, msg):
    rc = _forw3(**kw)
    assert rc == capi.TP_ERR_INVALID
    assert msg in capi.lib().tp_last_error().decode()


def test_half_volume_storage_is_projection_only():
    """TP_F16S (complex-half volume) is accepted by the two forward projections
    and their backward ops only; every other entry point rejects it before
    enqueuing anything."""
    lib = capi.lib()
    assert _forw3(dtype=capi.TP_F16S, P=0) == capi.TP_OK  # nothing to do, valid arguments
    rc = lib.tp_project_2d_forw(capi.TP_F16S, _P(8), 1, 16, 9, _P(8), 1, 0, _P(None), 1, 8, 0, 1.0, 0, 0.0, _P(8),
                                _P(None))
    assert rc == capi.TP_OK
    # the backward's argument checks run for TP_F16S (a depth other than the height is rejected)
    rc = lib.tp_project_3d_to_2d_back(capi.TP_F16S, _P(8), 1, 2, 8, 5, _P(8), 8, 16, 9, _P(8), 1, _P(None), 1, 0,
                                      1.0, 0, 0.0, _P(8), _P(None), _P(None), _P(None))
    assert rc == capi.TP_ERR_INVALID and "depth" in lib.tp_last_error().decode()
    rc = lib.tp_project_3d_to_2d_back(3, _P(8), 1, 2, 8, 5, _P(8), 16, 16, 9, _P(8), 1, _P(None), 1, 0,
                                      1.0, 0, 0.0, _P(8), _P(None), _P(None), _P(None))
    assert rc == capi.TP_ERR_INVALID and "dtype" in lib.tp_last_error().decode()
    rc = lib.tp_backproject_2d_forw(capi.TP_F16S, _P(8), 1, 1, 8, 5, _P(None), _P(8), 1, _P(None), 1, 0, 2.0, 0,
                                    0.0, _P(8), _P(None), _P(None))
    assert rc == capi.TP_ERR_INVALID and "dtype" in lib.tp_last_error().decode()


def test_noalloc_forward_checks_arguments_first():
    """The no-allocation forward rejects invalid arguments with the same messages, before it
    touches a device (nothing here has one)."""
    lib = capi.lib()
    a = dict(dtype=0, rec=_P(8), B=1, D=8, N=16, H=9, rot=_P(8), B_rot=1, P=2, shifts=_P(None), B_shift=1, n=8,
             interp=0, os=1.0, has_cut=0, cut=0.0, out=_P(8), stream=_P(None))
    assert lib.tp_project_3d_to_2d_forw_noalloc(*a.values()) == capi.TP_ERR_INVALID
    assert "depth" in lib.tp_last_error().decode()
    a.update(D=16, P=0)  # valid, nothing to do
    assert lib.tp_project_3d_to_2d_forw_noalloc(*a.values()) == capi.TP_OK
