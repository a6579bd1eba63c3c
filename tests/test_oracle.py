"""Pins the CPU oracle before it is trusted as the checker of the HIP kernels.

Each check is chosen so that a plausible mistake in the oracle (a wrong index, a transposed operand,
a dropped term, a wrong tie rule) fails: FP64 window loops (the reference's own test oracles,
restated in oracle/naive.py), scipy.signal.correlate, the adjoint identities of convolution,
torch's CPU float64 routines, closed forms and the reference tests' known answers.
"""

import numpy as np
import pytest
import scipy.signal
import torch

from oracle import naive, reference_path as rp
from oracle import resnet as oracle_resnet
from tests.fixtures import CONV_CASES, PERFORMANCE_CASES, POOL_CASES, conv_fixture

F64 = np.float64


def test_fastdiv_formula_is_exact():
    """The magic-number division used by the HIP kernels (csrc/fastdiv.h), checked on the CPU."""
    rng = np.random.default_rng(5)
    divisors = np.concatenate([np.arange(1, 300), rng.integers(1, 2**31 - 1, 2000), [2**31 - 1, 2**30, 65535]])
    n = np.concatenate([rng.integers(0, 2**31, 4000), [0, 1, 2**31 - 1, 2**31 - 2]]).astype(np.uint64)
    for d in divisors.astype(np.uint64):
        shift = int(np.ceil(np.log2(int(d)))) if d > 1 else 0
        while (1 << shift) < int(d):
            shift += 1
        magic = ((1 << 32) * ((1 << shift) - int(d))) // int(d) + 1
        q = (((n * np.uint64(magic)) >> np.uint64(32)) + n) >> np.uint64(shift)
        assert np.array_equal(q, n // d), int(d)


@pytest.mark.parametrize("shape,kernel,stride,padding", [
    ((2, 3, 4, 5), (2, 3), (1, 2), (1, 0)), ((1, 2, 7, 9), (3, 3), (2, 2), (1, 1)), ((2, 1, 6, 5), (1, 1), (1, 1), (0, 0)),
    ((1, 3, 16, 16), (7, 7), (2, 2), (3, 3))])
def test_im2col_col2im_match_fp64_loops(shape, kernel, stride, padding):
    rng = np.random.default_rng(7)
    x = rng.normal(size=shape)
    cols = rp.im2col(x, kernel, stride, padding)
    assert np.array_equal(cols, naive.im2col(x, kernel, stride, padding))  # pure copy: exact
    rows = rng.normal(size=cols.shape)
    ref = naive.col2im(rows, shape, kernel, stride, padding)
    np.testing.assert_allclose(rp.col2im(rows, shape, kernel, stride, padding), ref, atol=1e-10)
    np.testing.assert_allclose(rp.col2im_native(rows.astype(np.float32), shape, kernel, stride, padding), ref,
                               atol=1e-5)
    # <im2col(x), r> = <x, col2im(r)>: col2im is the adjoint of im2col.
    assert np.isclose(np.vdot(cols, rows), np.vdot(x, ref), rtol=1e-12)


def test_conv_known_answer_t0():
    """arange(25) * ones(3x3), stride 1, no padding: each output is the sum of its 3x3 window."""
    x, w, b, _ = conv_fixture(CONV_CASES[0])
    y, _ = rp.conv2d_forward(x, w, b, (1, 1), (0, 0))
    grid = np.arange(25).reshape(5, 5)
    expected = np.array([[grid[i:i + 3, j:j + 3].sum() for j in range(3)] for i in range(3)], dtype=np.float32)
    assert np.array_equal(y[0, 0], expected)
    assert expected[0, 0] == 54 and expected[2, 2] == 162


@pytest.mark.parametrize("case", CONV_CASES + PERFORMANCE_CASES[:1] + PERFORMANCE_CASES[2:], ids=lambda c: c[0])
def test_conv_forward_backward_match_fp64_loops(case):
    x, w, b, dy = conv_fixture(case)
    stride, padding = case[3], case[4]
    y, cols = rp.conv2d_forward(x, w, b, stride, padding)
    x64, w64, dy64 = x.astype(F64), w.astype(F64), dy.astype(F64)
    pre = naive.conv_forward(x64, w64, stride, padding) + b.astype(F64)[None, :, None, None]
    scale = np.abs(pre).max()
    assert np.abs(y - pre).max() <= 1e-5 * scale
    dx, dw, db = rp.conv2d_backward(x, w, dy, cols, stride, padding)
    ref_dx, ref_dw = naive.conv_backward(x64, w64, dy64, stride, padding)
    assert np.abs(dx - ref_dx).max() <= 1e-5 * np.abs(ref_dx).max()
    assert np.abs(dw - ref_dw).max() <= 1e-5 * np.abs(ref_dw).max()
    ref_db = dy64.sum(axis=(0, 2, 3))
    assert np.all(np.abs(db - ref_db) <= np.spacing(np.abs(ref_db).astype(np.float32)))


def test_conv_forward_matches_scipy_correlate():
    rng = np.random.default_rng(3)
    x = rng.normal(size=(2, 3, 9, 11))
    w = rng.normal(size=(4, 3, 3, 3))
    y, _ = rp.conv2d_forward(x, w, None, (1, 1), (0, 0))
    for n in range(2):
        for co in range(4):
            ref = sum(scipy.signal.correlate(x[n, ci], w[co, ci], mode="valid") for ci in range(3))
            np.testing.assert_allclose(y[n, co], ref, atol=1e-10)


def test_conv_backward_is_the_adjoint_of_forward():
    """<conv(x, W), g> = <x, dX(g)> = <W, dW(g)> in FP64 for a strided, padded, non-square case."""
    rng = np.random.default_rng(11)
    x = rng.normal(size=(2, 3, 8, 9))
    w = rng.normal(size=(5, 3, 3, 2))
    y, cols = rp.conv2d_forward(x, w, None, (2, 1), (1, 1))
    g = rng.normal(size=y.shape)
    dx, dw, _ = rp.conv2d_backward(x, w, g, cols, (2, 1), (1, 1))
    inner = np.vdot(y.astype(F64), g)
    assert np.isclose(inner, np.vdot(x, dx), rtol=1e-6)
    assert np.isclose(inner, np.vdot(w, dw), rtol=1e-6)


@pytest.mark.parametrize("shape,kernel,stride,padding", POOL_CASES)
def test_pool_paths_match_fp64_loops_with_ties(shape, kernel, stride, padding):
    rng = np.random.default_rng(7)
    x = rng.integers(-3, 4, size=shape).astype(np.float32)
    ph, pw = padding
    padded = np.pad(x.astype(F64), ((0, 0), (0, 0), (ph, ph), (pw, pw)), constant_values=-np.inf)
    expected = naive.maxpool_forward(padded, kernel, stride)
    dy = rng.standard_normal(expected.shape).astype(np.float32)
    expected_dx = naive.maxpool_backward(padded, dy.astype(F64), kernel, stride)[:, :, ph:ph + shape[2], pw:pw + shape[3]]
    y, mask, pshape = rp.maxpool2d_forward(x, kernel, stride, padding)
    assert np.array_equal(y, expected)
    np.testing.assert_allclose(rp.maxpool2d_backward(dy, mask, pshape, kernel, stride, padding), expected_dx, atol=1e-6)
    yn, argmax = rp.maxpool2d_native_forward(padded.astype(np.float32), kernel, stride)
    assert np.array_equal(yn, expected)
    assert np.array_equal(yn.reshape(-1), padded.astype(np.float32).reshape(-1)[argmax.reshape(-1)])
    dxn = rp.maxpool2d_native_backward(dy, argmax, padded.shape)[:, :, ph:ph + shape[2], pw:pw + shape[3]]
    np.testing.assert_allclose(dxn, expected_dx, atol=1e-6)


def test_pool_tie_goes_to_first_index_and_nan_propagates():
    x = np.array([[[[1.0, 1.0], [0.0, 0.5]]]], dtype=np.float32)
    y, argmax = rp.maxpool2d_native_forward(x, (2, 2), (2, 2))
    assert argmax.item() == 0 and y.item() == 1.0
    np.testing.assert_array_equal(rp.maxpool2d_native_backward(np.ones_like(y), argmax, x.shape),
                                  [[[[1.0, 0.0], [0.0, 0.0]]]])
    for position in range(4):
        z = np.arange(1, 5, dtype=np.float32).reshape(1, 1, 2, 2)
        z.reshape(-1)[position] = np.nan
        assert np.isnan(rp.maxpool2d_native_forward(z, (2, 2), (2, 2))[0]).all()
    # signed zeros tie: the first element is returned bit for bit
    z = np.array([[[[-0.0, 0.0], [0.0, -0.0]]]], dtype=np.float32)
    yz, az = rp.maxpool2d_native_forward(z, (2, 2), (2, 2))
    assert az.item() == 0 and np.signbit(yz.item())


def test_batchnorm_matches_torch_float64():
    rng = np.random.default_rng(4)
    x = rng.normal(1.0, 2.0, size=(4, 3, 5, 6)).astype(np.float32)
    gamma = rng.uniform(0.5, 1.5, 3).astype(np.float32)
    beta = rng.normal(size=3).astype(np.float32)
    rm, rv = np.zeros(3, np.float32), np.ones(3, np.float32)
    y, mean, inv_std = rp.batchnorm2d_forward(x, gamma, beta, rm, rv, training=True)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    gt = torch.tensor(gamma, dtype=torch.float64, requires_grad=True)
    bt = torch.tensor(beta, dtype=torch.float64, requires_grad=True)
    rmt, rvt = torch.zeros(3, dtype=torch.float64), torch.ones(3, dtype=torch.float64)
    yt = torch.nn.functional.batch_norm(xt, rmt, rvt, gt, bt, training=True, momentum=0.1, eps=1e-5)
    np.testing.assert_allclose(y, yt.detach().numpy(), rtol=0, atol=2e-6)
    np.testing.assert_allclose(rm, rmt.numpy(), atol=1e-7)
    # torch tracks the unbiased variance; the reference's default tracks the biased one.
    count = 4 * 5 * 6
    np.testing.assert_allclose((rv - 0.9) / 0.1 * count / (count - 1), (rvt.numpy() - 0.9) / 0.1, rtol=1e-5)
    dy = rng.normal(size=x.shape).astype(np.float32)
    yt.backward(torch.tensor(dy, dtype=torch.float64))
    dx, dgamma, dbeta = rp.batchnorm2d_backward(x, dy, gamma, mean, inv_std, training=True)
    np.testing.assert_allclose(dx, xt.grad.numpy(), atol=2e-5)
    np.testing.assert_allclose(dgamma, gt.grad.numpy(), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(dbeta, bt.grad.numpy(), rtol=1e-6)


def test_adam_first_step_closed_form():
    """With zero moments the first bias-corrected step is lr * g / (|g| + eps)."""
    rng = np.random.default_rng(2)
    g = rng.normal(size=100).astype(np.float32)
    p = rng.normal(size=100).astype(np.float32)
    p0 = p.copy()
    m, v = np.zeros_like(p), np.zeros_like(p)
    rp.adam_update(p, g, m, v, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, step=1)
    np.testing.assert_allclose(p, p0 - 1e-3 * g / (np.abs(g) + 1e-8), rtol=0, atol=2e-9)
    np.testing.assert_allclose(m, 0.1 * g, rtol=1e-6)
    np.testing.assert_allclose(v, 0.001 * g * g, rtol=1e-5)


def test_adam_recurrence_over_four_steps_matches_the_textbook_and_torch():
    """The moment recurrences from step 2 on (tests/test_fused_ops.py:162-177 of the reference): four
    steps of the oracle's float32 Adam against the FP64 textbook recurrence within 4 eps32
    (normwise), and against torch.optim.Adam (float64) with the same gradients. A dropped (1 - beta)
    factor, a moment not carried over or a bias correction of the wrong step fails one of them."""
    rng = np.random.default_rng(3)
    grads = [rng.standard_normal((5, 7)).astype(np.float32) for _ in range(4)]
    start = np.linspace(-1, 1, 35, dtype=np.float32).reshape(5, 7)
    p, m, v = start.copy(), np.zeros((5, 7), np.float32), np.zeros((5, 7), np.float32)
    theta, m64, v64 = start.astype(np.float64), np.zeros((5, 7)), np.zeros((5, 7))
    t_param = torch.tensor(start.astype(np.float64), requires_grad=True)
    t_opt = torch.optim.Adam([t_param], lr=1e-3, betas=(0.9, 0.999), eps=1e-8)
    eps32 = np.finfo(np.float32).eps
    for step, g in enumerate(grads, 1):
        rp.adam_update(p, g, m, v, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, step=step)
        g64 = g.astype(np.float64)
        m64 = 0.9 * m64 + 0.1 * g64
        v64 = 0.999 * v64 + 0.001 * g64 * g64
        theta = theta - 1e-3 * (m64 / (1 - 0.9 ** step)) / (np.sqrt(v64 / (1 - 0.999 ** step)) + 1e-8)
        t_param.grad = torch.tensor(g64)
        t_opt.step()
        assert np.abs(p - theta).max() <= 4 * eps32 * np.abs(theta).max(), step
        np.testing.assert_allclose(p, t_param.detach().numpy(), rtol=0, atol=4 * eps32)
        np.testing.assert_allclose(m, m64, rtol=1e-6, atol=1e-7)
        np.testing.assert_allclose(v, v64, rtol=1e-5, atol=1e-9)


def test_linear_and_mse_match_torch():
    rng = np.random.default_rng(1)
    x = rng.normal(size=(7, 5)).astype(np.float32)
    w = rng.normal(size=(5, 3)).astype(np.float32)
    b = rng.normal(size=(3,)).astype(np.float32)
    t = rng.normal(size=(7, 3)).astype(np.float32)
    out = rp.linear_forward(x, w, b)
    loss = rp.mse_forward(out, t)
    xt, wt, bt = (torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (x, w, b))
    lt = torch.nn.functional.mse_loss(xt @ wt + bt, torch.tensor(t, dtype=torch.float64))
    lt.backward()
    assert np.isclose(loss, lt.item(), rtol=1e-6)
    dx, dw, db = rp.linear_backward(x, w, b.shape, rp.mse_backward(out, t))
    np.testing.assert_allclose(dx, xt.grad.numpy(), rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(dw, wt.grad.numpy(), rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(db, bt.grad.numpy(), rtol=1e-5, atol=1e-7)


def _torch_resnet_loss(params, x, target):
    """ResNet18 (myflows compat) written with torch CPU float64 functional ops from the same params."""
    F = torch.nn.functional
    P = {k: torch.tensor(v, dtype=torch.float64, requires_grad=True) for k, v in params.items()}

    def conv(h, name, stride, pad):
        return F.conv2d(h, P[f"{name}.weight"], P[f"{name}.bias"], stride=stride, padding=pad)

    def bn(h, name):
        return F.batch_norm(h, None, None, P[f"{name}.gamma"], P[f"{name}.beta"], training=True, eps=1e-5)

    h = F.relu(bn(conv(torch.tensor(x, dtype=torch.float64), "stem", 2, 3), "stem_bn"))
    h = F.max_pool2d(h, 3, 2)
    for name, ci, co, stride in oracle_resnet.block_specs(params["stem.weight"].shape[0]):
        a = F.relu(bn(conv(h, f"{name}.conv1", stride, 1), f"{name}.bn1"))
        b = bn(conv(a, f"{name}.conv2", 1, 1), f"{name}.bn2")
        s = bn(conv(h, f"{name}.down", stride, 0), f"{name}.down_bn") if f"{name}.down.weight" in P else h
        h = F.relu(b + s)
    out = h.mean(dim=(2, 3)) @ P["fc.W"] + P["fc.b"]
    loss = F.mse_loss(out, torch.tensor(target, dtype=torch.float64))
    loss.backward()
    return loss.item(), {k: v.grad.numpy() for k, v in P.items()}


def test_resnet_oracle_matches_torch_float64_autograd():
    """The straight-line NumPy ResNet18 step (graph order, BN statistics, residual gradients, pooling,
    GAP, fc, MSE) against torch autograd on the same weights (small width and image)."""
    params, running = oracle_resnet.init_params(base_width=8, seed=0)
    x, target = oracle_resnet.synthetic_batch(2, 48, 64, seed=0)
    loss, grads, _ = oracle_resnet.forward_backward(params, running, x, target)
    ref_loss, ref_grads = _torch_resnet_loss(params, x, target)
    assert np.isclose(loss, ref_loss, rtol=1e-5)
    # Conv biases in front of a BN have an exactly zero gradient (BN removes the mean); the floor
    # relative to the largest gradient absorbs their float32 rounding noise.
    floor = 1e-5 * max(np.abs(g).max() for g in ref_grads.values())
    for name, ref in ref_grads.items():
        scale = np.abs(ref).max()
        err = np.abs(grads[name] - ref).max()
        assert err <= 2e-3 * scale + floor, (name, err, scale)


def test_resnet_param_order_and_count():
    params, _ = oracle_resnet.init_params()
    assert sum(p.size for p in params.values()) == 11_182_338  # myflows compat: convs carry a bias
    names = list(params)
    assert names[0] == "stem.weight" and names[-2:] == ["fc.W", "fc.b"]
    assert names.index("layer2.0.down.weight") > names.index("layer2.0.conv2.weight")


def test_resnet_oracle_follows_imposed_decisions():
    """The decisions a pass records, imposed on the same pass, reproduce it bit for bit; flipping one
    ReLU mask entry changes the gradient only through that entry's term."""
    params, running = oracle_resnet.init_params(base_width=8, seed=1)
    x, t = oracle_resnet.synthetic_batch(2, 32, 40, seed=1)
    record = {}
    loss, grads, out = oracle_resnet.forward_backward(params, {k: (m.copy(), v.copy()) for k, (m, v) in running.items()},
                                               x, t, record=record)
    decisions = {k: v for k, v in record.items() if not k.endswith("/input")}
    loss2, grads2, out2 = oracle_resnet.forward_backward(params, {k: (m.copy(), v.copy()) for k, (m, v) in running.items()},
                                                  x, t, decisions=decisions)
    assert loss2 == loss and np.array_equal(out2, out)
    for name in grads:
        np.testing.assert_array_equal(grads2[name], grads[name], err_msg=name)
    flipped = dict(decisions)
    mask = flipped["layer4.1.out"].copy()
    mask.flat[0] = not mask.flat[0]
    flipped["layer4.1.out"] = mask
    _, grads3, _ = oracle_resnet.forward_backward(params, {k: (m.copy(), v.copy()) for k, (m, v) in running.items()},
                                           x, t, decisions=flipped)
    assert not np.array_equal(grads3["fc.W"], grads["fc.W"])

