"""Max-pool parity on the GPU: values, int32 argmax and input gradients bit-exact against the native
semantics restated in the oracle (first maximum wins ties, NaN takes over, windows may overlap, -inf
padding), and against the FP64 loops of the reference's tests."""

import numpy as np
import pytest
import torch

import myflows_amd as mf
from myflows_amd import native
from oracle import naive, reference_path as rp
from tests.fixtures import POOL_CASES

pytestmark = pytest.mark.gpu


def gpu(a):
    return torch.as_tensor(np.ascontiguousarray(a), device="cuda")


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("shape,kernel,stride,padding", POOL_CASES + (
    ((4, 8, 60, 80), (3, 3), (2, 2), (0, 0)), ((2, 4, 30, 40), (2, 2), (2, 2), (0, 0)),
    ((2, 3, 9, 9), (3, 3), (1, 1), (1, 1)),
    ((3, 5, 13, 16), (3, 3), (2, 2), (0, 0))))  # two-row backward blocks: odd H, nine planes per workgroup
def test_pool_bit_exact_with_ties_padding_and_overlap(shape, kernel, stride, padding):
    print("pool", shape, kernel, stride, padding, flush=True)
    rng = np.random.default_rng(7)
    x = rng.integers(-3, 4, size=shape).astype(np.float32)  # small integers: many ties
    ph, pw = padding
    padded = np.pad(x, ((0, 0), (0, 0), (ph, ph), (pw, pw)), constant_values=-np.inf)
    y_ref, argmax_ref = rp.maxpool2d_native_forward(padded, kernel, stride)
    dy = rng.standard_normal(y_ref.shape).astype(np.float32)
    dx_ref = rp.maxpool2d_native_backward(dy, argmax_ref, padded.shape)[:, :, ph:ph + shape[2], pw:pw + shape[3]]
    node = mf.Variable(gpu(x))
    pool = mf.MaxPool2d_Op(node, kernel, stride, padding=padding, backend="hip_native")
    pool.forward(node.value)
    pool.grad = gpu(dy)
    pool.backward()
    np.testing.assert_array_equal(host(pool.value), y_ref)
    np.testing.assert_array_equal(host(pool._context.argmax), argmax_ref)
    np.testing.assert_array_equal(host(node.grad), dx_ref)
    np.testing.assert_array_equal(host(pool.value), naive.maxpool_forward(padded.astype(np.float64), kernel, stride))


def test_tie_nan_and_signed_zero():
    y, ctx = native.maxpool2d_forward(gpu(np.array([[[[1.0, 1.0], [0.0, 0.5]]]], np.float32)))
    dx = native.maxpool2d_backward(torch.ones_like(y), ctx)
    np.testing.assert_array_equal(host(dx), [[[[1.0, 0.0], [0.0, 0.0]]]])  # the first maximum gets it
    for position in range(4):
        z = np.arange(1, 5, dtype=np.float32).reshape(1, 1, 2, 2)
        z.reshape(-1)[position] = np.nan
        assert np.isnan(host(native.maxpool2d_forward(gpu(z))[0])).all()
    yz, cz = native.maxpool2d_forward(gpu(np.array([[[[-0.0, 0.0], [0.0, -0.0]]]], np.float32)))
    assert host(cz.argmax).item() == 0 and np.signbit(host(yz).item())


def test_pool_rejects_bad_calls():
    x = gpu(np.zeros((1, 1, 4, 4), np.float32))
    with pytest.raises(ValueError):
        native.maxpool2d_forward(x, kernel_size=(5, 5))
    y, ctx = native.maxpool2d_forward(x)
    with pytest.raises(ValueError):
        native.maxpool2d_backward(torch.zeros((1, 1, 3, 3), device="cuda"), ctx)
    with pytest.raises(ValueError):
        native.maxpool2d_backward(y, object())
