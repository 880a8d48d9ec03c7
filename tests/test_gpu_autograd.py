"""The public operators on cuda:0 under torch.autograd: the reference's own
gradient, batching and oversampling checks (tests/reference_props.py)
through the dispatcher ops, the autograd Functions of torch_projectors.ops
and the preparation helpers of torch_projectors.fourier.

complex128 gradchecks run the fp64 kernels; the fp32 checks (shift and
rotation gradients, weights, convergence, batching) run the tile-owner
kernels for rotation poses.
"""
import pytest

from tests import reference_props as A

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


@pytest.mark.parametrize("B", [1, 3])
@pytest.mark.parametrize("os_", [2.0, 3.0])
@pytest.mark.parametrize("interp", INTERP)
@pytest.mark.parametrize("dim", DIMS)
def test_oversampling_equivalence(api, gpu, dim, interp, os_, B):
    from torch_projectors import fourier
    _say("oversampling", dim, interp, os_, B)
    both = _With(api, fourier)
    A.oversampling_projection(both, gpu, dim, interp, os_, B)
    A.oversampling_backprojection(both, gpu, dim, interp, os_, B)


@pytest.mark.parametrize("dim", DIMS)
def test_oversampling_weights(api, gpu, dim):
    from torch_projectors import fourier
    _say("oversampling weights", dim)
    A.oversampling_weights(_With(api, fourier), gpu, dim)


class _With:
    """The operators of `ops` with the preparation helpers of `prep`."""

    def __init__(self, ops, prep):
        self._ops, self.pad_and_fftshift, self.ifftshift_and_crop = ops, prep.pad_and_fftshift, \
            prep.ifftshift_and_crop

    def __getattr__(self, name):
        return getattr(self._ops, name)
