"""The public operators on cuda:0 under torch.autograd: the reference's own
gradient and batching checks (tests/autograd_props.py) through the dispatcher
ops and the autograd Functions of torch_projectors.ops.

complex128 gradchecks run the fp64 kernels; the fp32 checks (shift and
rotation gradients, weights, convergence, batching) run the tile-owner
kernels for rotation poses.
"""
import pytest

from tests import autograd_props as A

pytestmark = pytest.mark.gpu

INTERP = ["linear", "cubic"]
DIMS = [2, 3]


@pytest.fixture(scope="module")
def api(gpu):
    import torch_projectors
    return torch_projectors


def _say(*a):
    print("[autograd]", *a, flush=True)


@pytest.mark.parametrize("interp", INTERP)
@pytest.mark.parametrize("dim", DIMS)
def test_gradcheck_projection(api, gpu, dim, interp):
    _say("gradcheck projection", dim, interp)
    A.gradcheck_projection(api, gpu, dim, interp)


@pytest.mark.parametrize("weights", [False, True])
@pytest.mark.parametrize("interp", INTERP)
@pytest.mark.parametrize("dim", DIMS)
def test_gradcheck_backprojection(api, gpu, dim, interp, weights):
    _say("gradcheck backprojection", dim, interp, weights)
    A.gradcheck_backprojection(api, gpu, dim, interp, with_weights=weights)


@pytest.mark.parametrize("shift,B,P", A.SHIFT_CASES, ids=[f"{s}-B{b}P{p}" for s, b, p in A.SHIFT_CASES])
@pytest.mark.parametrize("interp", INTERP)
@pytest.mark.parametrize("dim", DIMS)
def test_shift_gradient_projection(api, gpu, dim, interp, shift, B, P):
    _say("shift grad projection", dim, interp, shift, B, P)
    A.shift_gradient_projection(api, gpu, dim, interp, shift, B, P)


@pytest.mark.parametrize("shift,B,P", A.SHIFT_CASES, ids=[f"{s}-B{b}P{p}" for s, b, p in A.SHIFT_CASES])
@pytest.mark.parametrize("interp", INTERP)
@pytest.mark.parametrize("dim", DIMS)
def test_shift_gradient_backprojection(api, gpu, dim, interp, shift, B, P):
    _say("shift grad backprojection", dim, interp, shift, B, P)
    A.shift_gradient_backprojection(api, gpu, dim, interp, shift, B, P)


@pytest.mark.parametrize("backprojection", [False, True])
@pytest.mark.parametrize("interp", INTERP)
@pytest.mark.parametrize("dim", DIMS)
def test_rotation_gradients(api, gpu, dim, interp, backprojection):
    _say("rotation grads", dim, interp, backprojection)
    if backprojection:
        A.rotation_fd_backprojection(api, gpu, dim, interp)
    else:
        A.rotation_fd_projection(api, gpu, dim, interp)
    A.rotation_gradient_nonzero(api, gpu, dim, interp, backprojection)
    A.rotation_convergence(api, gpu, dim, interp, backprojection)


@pytest.mark.parametrize("interp", INTERP)
@pytest.mark.parametrize("dim", DIMS)
def test_weight_gradients(api, gpu, dim, interp):
    _say("weight grads", dim, interp)
    A.weight_fd(api, gpu, dim, interp)


@pytest.mark.parametrize("backprojection", [False, True])
@pytest.mark.parametrize("interp", INTERP)
@pytest.mark.parametrize("dim", DIMS)
def test_fourier_component_step(api, gpu, dim, interp, backprojection):
    _say("fourier component step", dim, interp, backprojection)
    A.fourier_component_step(api, gpu, dim, interp, backprojection)


@pytest.mark.parametrize("interp", INTERP)
@pytest.mark.parametrize("dim", DIMS)
def test_batching(api, gpu, dim, interp):
    _say("batching", dim, interp)
    A.batching_projection(api, gpu, dim, interp)
    A.batching_backprojection(api, gpu, dim, interp)
