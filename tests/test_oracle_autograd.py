"""The reference's gradient, batching and oversampling checks
(tests/reference_props.py) on the CPU oracle under torch.autograd
(tests/oracle_autograd.py).

They pin the oracle's backward functions against what the mathematics fixes —
complex128 gradcheck, shift gradients against a phase ramp written in torch
operations, rotation and weight gradients against finite differences — and
show, by planting mistakes in the oracle's backward, that each kind of check
notices the mistake it is there for.  The same bodies run on the HIP
operators in tests/test_gpu_autograd.py.
"""
import pytest
import torch

from tests import reference_props as A
from tests import oracle_autograd as OA

CPU = "cpu"
INTERP = ["linear", "cubic"]
DIMS = [2, 3]


@pytest.mark.parametrize("interp", INTERP)
@pytest.mark.parametrize("dim", DIMS)
def test_gradcheck(dim, interp):
    A.gradcheck_projection(OA, CPU, dim, interp)
    A.gradcheck_backprojection(OA, CPU, dim, interp)
    A.gradcheck_backprojection(OA, CPU, dim, interp, with_weights=True)


@pytest.mark.parametrize("interp", INTERP)
@pytest.mark.parametrize("dim", DIMS)
def test_shift_gradients(dim, interp):
    for shift, B, P in A.SHIFT_CASES:
        A.shift_gradient_projection(OA, CPU, dim, interp, shift, B, P)
        A.shift_gradient_backprojection(OA, CPU, dim, interp, shift, B, P)


@pytest.mark.parametrize("interp", INTERP)
@pytest.mark.parametrize("dim", DIMS)
def test_rotation_gradients(dim, interp):
    A.rotation_fd_projection(OA, CPU, dim, interp)
    A.rotation_fd_backprojection(OA, CPU, dim, interp)
    for bp in (False, True):
        A.rotation_gradient_nonzero(OA, CPU, dim, interp, bp)
        A.rotation_convergence(OA, CPU, dim, interp, bp)


@pytest.mark.parametrize("interp", INTERP)
@pytest.mark.parametrize("dim", DIMS)
def test_weights_steps_and_batching(dim, interp):
    A.weight_fd(OA, CPU, dim, interp)
    for bp in (False, True):
        A.fourier_component_step(OA, CPU, dim, interp, bp)
    A.batching_projection(OA, CPU, dim, interp)
    A.batching_backprojection(OA, CPU, dim, interp)


# ----------------------------------------------------------------------------- planted mistakes
def _on(kind, fix):
    """A plant that edits the gradients of `kind` with fix(list) -> list."""
    def plant(k, grads):
        return tuple(fix(list(grads))) if k == kind else grads
    return plant


def _scale(i, s):
    def fix(g):
        g[i] = g[i] * s
        return g
    return fix


def _conj(i):
    def fix(g):
        g[i] = g[i].conj().resolve_conj()
        return g
    return fix


def _swap_shift(i):
    def fix(g):
        g[i] = g[i].flip(-1).contiguous()
        return g
    return fix


def _transpose_rot(i):
    def fix(g):
        g[i] = g[i].transpose(-1, -2).contiguous()
        return g
    return fix


FAILS = (AssertionError, RuntimeError)

PLANTS = [
    ("projection rec grad x1.03", "project", _scale(0, 1.03),
     lambda: A.gradcheck_projection(OA, CPU, 2, "linear")),
    ("3D projection rec grad conjugated", "project", _conj(0),
     lambda: A.gradcheck_projection(OA, CPU, 3, "cubic")),
    ("backprojection proj grad conjugated", "backproject", _conj(0),
     lambda: A.gradcheck_backprojection(OA, CPU, 2, "cubic")),
    ("backprojection weight grad x0.97", "backproject", _scale(1, 0.97),
     lambda: A.gradcheck_backprojection(OA, CPU, 3, "linear", with_weights=True)),
    ("projection shift grad components swapped", "project", _swap_shift(2),
     lambda: A.shift_gradient_projection(OA, CPU, 2, "linear", (2.0, 1.0), 1, 1)),
    ("backprojection shift grad negated", "backproject", _scale(3, -1.0),
     lambda: A.shift_gradient_backprojection(OA, CPU, 3, "linear", (0.5, 0.3), 1, 1)),
    ("projection rotation grad transposed", "project", _transpose_rot(1),
     lambda: A.rotation_fd_projection(OA, CPU, 2, "cubic")),
    ("3D projection rotation grad x1.01", "project", _scale(1, 1.01),
     lambda: A.rotation_fd_projection(OA, CPU, 3, "linear")),
    ("backprojection rotation grad negated", "backproject", _scale(2, -1.0),
     lambda: A.rotation_fd_backprojection(OA, CPU, 2, "linear")),
    ("backprojection weight grad dropped", "backproject", _scale(1, 0.0),
     lambda: A.weight_fd(OA, CPU, 2, "linear")),
]


@pytest.mark.parametrize("name,kind,fix,check", PLANTS, ids=[p[0] for p in PLANTS])
def test_checks_notice_planted_mistakes(monkeypatch, name, kind, fix, check):
    check()  # passes on the oracle as it is
    monkeypatch.setattr(OA, "plant", _on(kind, fix))
    with pytest.raises(FAILS):
        check()


@pytest.mark.parametrize("interp", INTERP)
@pytest.mark.parametrize("dim", DIMS)
def test_oversampling(dim, interp):
    for os_ in (2.0, 3.0):
        for B in (1, 3):
            A.oversampling_projection(OA, CPU, dim, interp, os_, B)
            A.oversampling_backprojection(OA, CPU, dim, interp, os_, B)
    A.oversampling_weights(OA, CPU, dim)
