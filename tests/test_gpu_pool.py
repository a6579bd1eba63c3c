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
    ((3, 5, 13, 16), (3, 3), (2, 2), (0, 0)),  # two-row backward blocks: odd H, nine planes per workgroup
    # 2x2 windows that tile the planes (the direct kernels), and beside them an odd H and a W that is
    # not a multiple of four (the staged kernels)
    ((3, 5, 14, 24), (2, 2), (2, 2), (0, 0)), ((1, 2, 2, 4), (2, 2), (2, 2), (0, 0)),
    ((3, 5, 13, 24), (2, 2), (2, 2), (0, 0)), ((3, 5, 14, 22), (2, 2), (2, 2), (0, 0))))
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


def test_tiling_2x2_pool_nan_signed_zero_and_without_indices():
    """The direct 2x2 kernels (windows tiling the planes) on NaNs at every window position, signed zeros
    and ties, a -0 gradient (0 + -0 is +0, as the staged kernels' sums give), and a pass without
    indices: bit-exact with the native semantics."""
    rng = np.random.default_rng(5)
    x = rng.integers(-1, 2, size=(2, 3, 8, 16)).astype(np.float32)
    x[0, 0, 0, :8] = [np.nan, 1, 2, np.nan, 0, 0, 3, 3]
    x[0, 0, 1, :8] = [0, np.nan, np.nan, 5, np.nan, 1, 3, np.nan]
    x[1, 2, 2:4, 4:8] = [[-0.0, 0.0, 0.0, -0.0], [0.0, -0.0, -0.0, -0.0]]
    y_ref, argmax_ref = rp.maxpool2d_native_forward(x, (2, 2), (2, 2))
    dy = rng.standard_normal(y_ref.shape).astype(np.float32)
    dy[0, 0, 0, :2] = -0.0
    dx_ref = rp.maxpool2d_native_backward(dy, argmax_ref, x.shape)
    y, ctx = native.maxpool2d_forward(gpu(x))
    np.testing.assert_array_equal(host(y), y_ref)
    np.testing.assert_array_equal(np.signbit(host(y)), np.signbit(y_ref))
    np.testing.assert_array_equal(host(ctx.argmax), argmax_ref)
    dx = host(native.maxpool2d_backward(gpu(dy), ctx))
    np.testing.assert_array_equal(dx, dx_ref)
    np.testing.assert_array_equal(np.signbit(dx), np.signbit(dx_ref))
    y_plain, ctx_plain = native.maxpool2d_forward(gpu(x), with_argmax=False)
    np.testing.assert_array_equal(host(y_plain), y_ref)
    assert ctx_plain.argmax is None


def test_pool_rejects_bad_calls():
    x = gpu(np.zeros((1, 1, 4, 4), np.float32))
    with pytest.raises(ValueError):
        native.maxpool2d_forward(x, kernel_size=(5, 5))
    y, ctx = native.maxpool2d_forward(x)
    with pytest.raises(ValueError):
        native.maxpool2d_backward(torch.zeros((1, 1, 3, 3), device="cuda"), ctx)
    with pytest.raises(ValueError):
        native.maxpool2d_backward(y, object())


@pytest.mark.parametrize("shape,kernel,stride", (((4, 8, 60, 80), (3, 3), (2, 2)), ((3, 5, 13, 16), (2, 2), (2, 2)),
                                                 ((2, 3, 9, 9), (3, 3), (1, 1))), ids=str)
def test_pool_forward_without_indices_gives_the_same_values_and_no_backward(shape, kernel, stride):
    """A pass no backward follows (with_argmax=False: the inference graph's max-pools) writes the same
    window maxima and no indices; its context refuses a backward."""
    print("pool without indices", shape, kernel, stride, flush=True)
    x = gpu(np.random.default_rng(9).integers(-3, 4, size=shape).astype(np.float32))
    y, ctx = native.maxpool2d_forward(x, kernel_size=kernel, stride=stride)
    y_plain, ctx_plain = native.maxpool2d_forward(x, kernel_size=kernel, stride=stride, with_argmax=False)
    assert ctx_plain.argmax is None and ctx.argmax is not None
    np.testing.assert_array_equal(host(y_plain), host(y))
    with pytest.raises(ValueError):
        native.maxpool2d_backward(torch.ones_like(y_plain), ctx_plain)


def test_inference_graph_pools_keep_no_indices():
    """apply_graph_optimizations(mode="inference") marks the max-pools: they store no window indices
    and refuse a backward, while the pooled values are the training graph's."""
    print("inference graph pool", flush=True)
    x = mf.Variable(gpu(np.random.default_rng(11).standard_normal((2, 3, 16, 16)).astype(np.float32)),
                    requires_grad=False)
    conv = mf.Conv2D(3, 4, 3, padding=1, fuse_activation=False, backend="hip_native")
    bn = mf.BatchNorm2d(4)
    bn.eval()
    out = mf.MaxPool2d(3, 2, backend="hip_native")(mf.ReLU(bn(conv(x))))
    plain = mf.Graph(out)
    plain.forward()
    expected = host(out.value)
    root, stats = mf.apply_graph_optimizations(out, mode="inference", fold_constants=False)
    assert stats["bn_folds"] == 1
    pool = root if isinstance(root, mf.MaxPool2d_Op) else next(
        n for n in mf.Graph(root).nodes if isinstance(n, mf.MaxPool2d_Op))
    assert pool.inference
    mf.Graph(root, optimize=True).forward()
    assert pool._context is None
    np.testing.assert_allclose(host(pool.value), expected, rtol=1e-5, atol=1e-5)
    pool.grad = torch.ones_like(pool.value)
    with pytest.raises(RuntimeError):
        pool.backward()
