"""Batch norm (+ residual + ReLU), ReLU and Adam kernels on the GPU against the oracle.

* Adam: bit-exact against the oracle's float32 NumPy step (IEEE division and square root, the same
  rounding order), single and multi-tensor, with a gradient scale and weight decay.
* ReLU: bit-exact (a selection and, when accumulating, one float32 addition).
* Head: the global average pool, the MSE loss and a Linear bias gradient sum in FP64 and round
  once, their gradients are float32 divisions and products in the operator's order: bit-exact
  where the FP64 sums are exact (the network's shapes), within one ulp on long sums.
* Batch norm: the GPU forms its FP64 statistics in one shifted pass, the oracle in two passes; the
  float32 results agree to within 4 ulp of the largest output (written in each test); the running
  statistics, dgamma and dbeta within 2e-6 relative.
"""

import numpy as np
import pytest
import torch

from myflows_amd import fused, native
from oracle import reference_path as rp
from tests.fixtures import assert_near

pytestmark = pytest.mark.gpu


def gpu(a):
    return torch.as_tensor(np.ascontiguousarray(a), device="cuda")


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def ulps_of_max(got, expected, ulps):
    scale = np.spacing(np.float32(np.abs(expected).max()))
    worst = float(np.abs(got.astype(np.float64) - expected).max())
    assert worst <= ulps * scale, f"max error {worst:.3e} > {ulps} ulp(max|ref|) = {ulps * scale:.3e}"


def bn_inputs(shape, seed):
    rng = np.random.default_rng(seed)
    c = shape[1]
    x = rng.normal(0.7, 2.0, size=shape).astype(np.float32)
    gamma = rng.uniform(0.5, 1.5, c).astype(np.float32)
    beta = rng.normal(size=c).astype(np.float32)
    rm = rng.normal(0, 0.1, c).astype(np.float32)
    rv = rng.uniform(0.5, 1.5, c).astype(np.float32)
    return x, gamma, beta, rm, rv, rng


SHAPES = ((2, 3, 5, 7), (4, 16, 30, 40), (64, 64, 29, 39), (3, 512, 4, 5))


@pytest.mark.parametrize("shape", SHAPES, ids=str)
@pytest.mark.parametrize("relu,residual", ((False, False), (True, False), (True, True)))
def test_batchnorm_forward_training(shape, relu, residual):
    print("bn forward", shape, relu, residual, flush=True)
    x, gamma, beta, rm, rv, rng = bn_inputs(shape, 11)
    res = rng.normal(size=shape).astype(np.float32) if residual else None
    rm_ref, rv_ref = rm.copy(), rv.copy()
    y_ref, mean_ref, inv_ref = rp.batchnorm2d_forward(x, gamma, beta, rm_ref, rv_ref, momentum=0.1, eps=1e-5,
                                                      relu=relu, residual=res)
    rm_gpu, rv_gpu = gpu(rm), gpu(rv)
    y, mean, inv_std = fused.batchnorm2d_forward(gpu(x), gpu(gamma), gpu(beta), rm_gpu, rv_gpu, momentum=0.1,
                                                 eps=1e-5, training=True, relu=relu,
                                                 residual=None if res is None else gpu(res))
    ulps_of_max(host(y), y_ref, 4)
    np.testing.assert_allclose(host(mean).astype(np.float64).sum(0), mean_ref.astype(np.float64).sum(0),
                               rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(host(inv_std), inv_ref, rtol=2e-7)
    np.testing.assert_allclose(host(rm_gpu), rm_ref, rtol=2e-6, atol=1e-7)
    np.testing.assert_allclose(host(rv_gpu), rv_ref, rtol=2e-6)
    if relu:
        assert (host(y) >= 0).all()


def test_batchnorm_forward_eval_and_unbiased_running_variance():
    x, gamma, beta, rm, rv, _ = bn_inputs((4, 8, 6, 6), 12)
    y_ref, _, _ = rp.batchnorm2d_forward(x, gamma, beta, rm.copy(), rv.copy(), training=False)
    rm_gpu, rv_gpu = gpu(rm), gpu(rv)
    y, mean, _ = fused.batchnorm2d_forward(gpu(x), gpu(gamma), gpu(beta), rm_gpu, rv_gpu, momentum=0.1, eps=1e-5,
                                           training=False)
    ulps_of_max(host(y), y_ref, 2)
    np.testing.assert_array_equal(host(rm_gpu), rm)  # eval leaves the running statistics alone
    np.testing.assert_array_equal(host(mean)[0], rm)
    # training with the torch convention: the running variance tracks the unbiased batch variance
    rv_gpu = gpu(rv)
    fused.batchnorm2d_forward(gpu(x), gpu(gamma), gpu(beta), gpu(rm), rv_gpu, momentum=0.1, eps=1e-5, training=True,
                              unbiased_running_var=True)
    count = 4 * 36
    batch_var = x.astype(np.float64).var(axis=(0, 2, 3))
    np.testing.assert_allclose(host(rv_gpu), 0.9 * rv + 0.1 * batch_var * count / (count - 1), rtol=2e-6)


@pytest.mark.parametrize("shape", SHAPES, ids=str)
@pytest.mark.parametrize("training", (True, False))
def test_batchnorm_backward(shape, training):
    print("bn backward", shape, training, flush=True)
    x, gamma, beta, rm, rv, rng = bn_inputs(shape, 13)
    dy = rng.normal(size=shape).astype(np.float32)
    _, mean_ref, inv_ref = rp.batchnorm2d_forward(x, gamma, beta, rm.copy(), rv.copy(), training=training)
    dx_ref, dgamma_ref, dbeta_ref = rp.batchnorm2d_backward(x, dy, gamma, mean_ref, inv_ref, training=training)
    x_grad = torch.full(shape, 0.25, device="cuda")  # accumulate into an existing gradient
    gamma_grad, beta_grad = torch.empty(shape[1], device="cuda"), torch.empty(shape[1], device="cuda")
    fused.batchnorm2d_backward(gpu(x), gpu(dy), gpu(gamma), gpu(mean_ref), gpu(inv_ref), training=training,
                               x_grad=x_grad, gamma_grad=gamma_grad, beta_grad=beta_grad,
                               accumulate=(True, False, False))
    assert_near(host(x_grad) - np.float32(0.25), dx_ref, 1e-5, "dx")
    np.testing.assert_allclose(host(gamma_grad), dgamma_ref, rtol=2e-6, atol=1e-6 * np.abs(dgamma_ref).max())
    np.testing.assert_allclose(host(beta_grad), dbeta_ref, rtol=2e-6, atol=1e-6 * np.abs(dbeta_ref).max())


def test_batchnorm_backward_through_fused_relu_and_residual():
    """g = dy where the ReLU output > 0: the residual branch receives g, BN's gradients use g."""
    shape = (8, 32, 15, 20)
    x, gamma, beta, rm, rv, rng = bn_inputs(shape, 14)
    res = rng.normal(size=shape).astype(np.float32)
    dy = rng.normal(size=shape).astype(np.float32)
    y_ref, mean_ref, inv_ref = rp.batchnorm2d_forward(x, gamma, beta, rm.copy(), rv.copy(), relu=True, residual=res)
    g = np.where(y_ref > 0, dy, np.float32(0))
    dx_ref, dgamma_ref, dbeta_ref = rp.batchnorm2d_backward(x, g, gamma, mean_ref, inv_ref)
    x_grad = torch.empty(shape, device="cuda")
    gamma_grad, beta_grad = torch.zeros(shape[1], device="cuda"), torch.zeros(shape[1], device="cuda")
    residual_grad = torch.empty(shape, device="cuda")
    fused.batchnorm2d_backward(gpu(x), gpu(dy), gpu(gamma), gpu(mean_ref), gpu(inv_ref), training=True,
                               x_grad=x_grad, gamma_grad=gamma_grad, beta_grad=beta_grad,
                               accumulate=(False, True, True), gate=gpu(y_ref), residual_grad=residual_grad)
    np.testing.assert_array_equal(host(residual_grad), g)
    assert_near(host(x_grad), dx_ref, 1e-5, "dx")
    np.testing.assert_allclose(host(gamma_grad), dgamma_ref, rtol=2e-6, atol=1e-6 * np.abs(dgamma_ref).max())
    np.testing.assert_allclose(host(beta_grad), dbeta_ref, rtol=2e-6, atol=1e-6 * np.abs(dbeta_ref).max())


def test_batchnorm_is_bitwise_reproducible():
    x, gamma, beta, rm, rv, rng = bn_inputs((16, 64, 30, 40), 15)
    dy = gpu(rng.normal(size=x.shape).astype(np.float32))
    runs = []
    for _ in range(2):
        y, mean, inv = fused.batchnorm2d_forward(gpu(x), gpu(gamma), gpu(beta), gpu(rm), gpu(rv), momentum=0.1,
                                                 eps=1e-5, training=True)
        grads = [torch.empty_like(y), torch.empty(64, device="cuda"), torch.empty(64, device="cuda")]
        fused.batchnorm2d_backward(gpu(x), dy, gpu(gamma), mean, inv, training=True, x_grad=grads[0],
                                   gamma_grad=grads[1], beta_grad=grads[2], accumulate=(False, False, False))
        runs.append([host(t) for t in (y, mean, inv, *grads)])
    for a, b in zip(*runs):
        np.testing.assert_array_equal(a, b)


def test_relu_forward_and_backward_are_exact():
    rng = np.random.default_rng(16)
    x = rng.normal(size=(3, 5, 7, 11)).astype(np.float32)
    x.reshape(-1)[:4] = [0.0, -0.0, np.nan, -np.inf]
    g = rng.normal(size=x.shape).astype(np.float32)
    y = host(fused.relu_forward(gpu(x)))
    np.testing.assert_array_equal(np.isnan(y), np.isnan(x))
    finite = ~np.isnan(x)
    np.testing.assert_array_equal(y[finite], np.maximum(x, 0)[finite])
    np.testing.assert_array_equal(host(fused.relu_backward_accumulate(gpu(x), gpu(g), None)), rp.relu_backward(x, g))
    out = gpu(g)
    fused.relu_backward_accumulate(gpu(x), gpu(g), out)
    np.testing.assert_array_equal(host(out), g + rp.relu_backward(x, g))
    leaky = host(fused.leaky_relu_backward_accumulate(gpu(x), gpu(g), None, 0.2))
    np.testing.assert_array_equal(leaky, np.where(x > 0, g, np.float32(0.2) * g))


def test_global_avg_pool_forward_and_backward_match_the_oracle():
    print("global average pool", flush=True)
    rng = np.random.default_rng(31)
    x = rng.normal(size=(64, 512, 4, 5)).astype(np.float32)
    np.testing.assert_array_equal(host(fused.global_avg_pool_forward(gpu(x))), rp.gap_forward(x))
    wide = rng.normal(size=(3, 7, 60, 80)).astype(np.float32)
    got, ref = host(fused.global_avg_pool_forward(gpu(wide))), rp.gap_forward(wide)
    assert np.all(np.abs(got - ref) <= np.spacing(np.abs(ref))), "long plane sums within one ulp"
    g = rng.normal(size=(64, 512)).astype(np.float32)
    expected = rp.gap_backward(g, x.shape)
    np.testing.assert_array_equal(host(fused.global_avg_pool_backward(gpu(g), x.shape)), expected)
    base = rng.normal(size=x.shape).astype(np.float32)
    out = gpu(base)
    fused.global_avg_pool_backward(gpu(g), x.shape, out, add=True)
    np.testing.assert_array_equal(host(out), base + expected)
    with pytest.raises(ValueError):
        fused.global_avg_pool_backward(gpu(g), x.shape, None, add=True)


@pytest.mark.parametrize("shape", ((64, 2), (3, 1000, 37)))
def test_mse_loss_and_gradient_match_the_oracle(shape):
    print("mse", shape, flush=True)
    rng = np.random.default_rng(32)
    pred = rng.normal(size=shape).astype(np.float32)
    target = rng.uniform(-1, 1, size=shape).astype(np.float32)
    loss, ref = host(fused.mse_loss_forward(gpu(pred), gpu(target))), rp.mse_forward(pred, target)
    assert loss.shape == () and abs(float(loss) - float(ref)) <= np.spacing(np.float32(ref)), (loss, ref)
    if pred.size <= 1024:
        np.testing.assert_array_equal(loss, ref)
    for seed in (np.float32(1.0), np.float32(0.37)):
        expected = rp.mse_backward(pred, target, seed)
        got = host(fused.mse_loss_backward(gpu(pred), gpu(target), gpu(np.array(seed))))
        np.testing.assert_array_equal(got, expected)
    base = rng.normal(size=shape).astype(np.float32)
    out = gpu(base)
    fused.mse_loss_backward(gpu(pred), gpu(target), gpu(np.array(np.float32(1.0))), out, add=True)
    np.testing.assert_array_equal(host(out), base + rp.mse_backward(pred, target))


def test_mse_of_no_elements_is_nan_like_the_oracle():
    empty = np.zeros((0, 2), dtype=np.float32)
    with np.errstate(invalid="ignore", divide="ignore"), pytest.warns(RuntimeWarning):
        ref = rp.mse_forward(empty, empty)
    assert np.isnan(ref) and np.isnan(host(fused.mse_loss_forward(gpu(empty), gpu(empty))))


def test_linear_bias_gradient_column_sums():
    rng = np.random.default_rng(33)
    g = rng.normal(size=(64, 2)).astype(np.float32)
    np.testing.assert_array_equal(host(fused.column_sums(gpu(g))), rp.reduce_to(g, (2,)))
    tall = rng.normal(size=(5000, 300)).astype(np.float32)
    got, ref = host(fused.column_sums(gpu(tall))), rp.reduce_to(tall, (300,))
    assert np.all(np.abs(got - ref) <= np.spacing(np.abs(ref))), "long column sums within one ulp"


@pytest.mark.parametrize("scale,decay", ((1.0, 0.0), (0.5, 0.0), (0.25, 1e-2)))
def test_adam_matches_the_oracle_bit_for_bit(scale, decay):
    rng = np.random.default_rng(17)
    sizes = (1, 7, 256, 257, 4096, 100003)
    params = [rng.normal(size=s).astype(np.float32) for s in sizes]
    state = [(np.zeros(s, np.float32), np.zeros(s, np.float32)) for s in sizes]
    dev_params = [gpu(p) for p in params]
    dev_state = [(gpu(m), gpu(v)) for m, v in state]
    for step in (1, 2, 3):
        grads = [rng.normal(size=s).astype(np.float32) for s in sizes]
        for p, g, (m, v) in zip(params, grads, state):
            rp.adam_update(p, g, m, v, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, step=step, grad_scale=scale,
                           weight_decay=decay)
        updates = [(p, gpu(g), m, v, 1e-3, decay, step) for p, g, (m, v) in zip(dev_params, grads, dev_state)]
        fused.adam_update_many(updates, beta1=0.9, beta2=0.999, eps=1e-8, grad_scale=scale)
        for p, p_ref, (m, v), (m_ref, v_ref) in zip(dev_params, params, dev_state, state):
            np.testing.assert_array_equal(host(p), p_ref)
            np.testing.assert_array_equal(host(m), m_ref)
            np.testing.assert_array_equal(host(v), v_ref)
    single = gpu(params[3])
    m, v = gpu(state[3][0]), gpu(state[3][1])
    g = rng.normal(size=sizes[3]).astype(np.float32)
    fused.adam_update(single, gpu(g), m, v, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, step=4, grad_scale=scale,
                      weight_decay=decay)
    rp.adam_update(params[3], g, *state[3], lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, step=4, grad_scale=scale,
                   weight_decay=decay)
    np.testing.assert_array_equal(host(single), params[3])


def test_adam_over_more_tensors_than_one_launch_takes():
    """ResNet18 has 62 parameter tensors: one step spans two launches, with 4-element (size a
    multiple of 4) and 1-element tensors mixed in each; every element matches the oracle's step."""
    rng = np.random.default_rng(23)
    sizes = [64 * (i % 5 + 1) + (3 if i % 7 == 0 else 0) for i in range(62)]
    params = [rng.normal(size=s).astype(np.float32) for s in sizes]
    grads = [rng.normal(size=s).astype(np.float32) for s in sizes]
    state = [(np.zeros(s, np.float32), np.zeros(s, np.float32)) for s in sizes]
    dev = [(gpu(p), gpu(g), gpu(m), gpu(v)) for p, g, (m, v) in zip(params, grads, state)]
    fused.adam_update_many([(p, g, m, v, 1e-3, 0.0, 1) for p, g, m, v in dev], beta1=0.9, beta2=0.999, eps=1e-8,
                           grad_scale=1.0)
    for p, g, (m, v), (dp, _, dm, dv) in zip(params, grads, state, dev):
        rp.adam_update(p, g, m, v, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, step=1)
        np.testing.assert_array_equal(host(dp), p)
        np.testing.assert_array_equal(host(dm), m)
        np.testing.assert_array_equal(host(dv), v)


def test_adam_falls_back_to_one_tensor_at_a_time_for_overlapping_or_strided_tensors():
    """tests/test_multi_adam.py:45-51: parameters that overlap another update's, and a strided
    gradient, cannot share one multi-tensor launch; the updates then run one tensor after another
    in the order given, which the oracle repeats on NumPy views of the same arrays."""
    arr = np.arange(20, dtype=np.float32) / 7
    dev = gpu(arr)

    def update(p, g):
        return p, g, torch.zeros_like(p), torch.zeros_like(p), 0.01, 0.0, 1

    overlapping = [update(dev[:10], dev[10:]), update(dev[5:15], gpu(arr[:10] + 1))]
    strided = [update(gpu(arr[:10]), gpu(arr)[::2])]
    assert not fused._multi_adam_fits(overlapping)
    for updates in (overlapping, strided):
        calls = []
        call = native._call
        native._call = lambda name, *args: (calls.append(name), call(name, *args))[1]
        try:
            fused.adam_update_many(updates, beta1=0.9, beta2=0.999, eps=1e-8, grad_scale=1.0)
        finally:
            native._call = call
        assert calls == ["mfh_adam_step"] * len(updates)
    ref = arr.copy()
    for p, g in ((ref[:10], ref[10:].copy()), (ref[5:15], arr[:10] + 1)):
        rp.adam_update(p, g, np.zeros(10, np.float32), np.zeros(10, np.float32), lr=0.01, beta1=0.9, beta2=0.999,
                       eps=1e-8, step=1)
    np.testing.assert_array_equal(host(dev), ref)
    p_ref = arr[:10].copy()
    rp.adam_update(p_ref, arr[::2].copy(), np.zeros(10, np.float32), np.zeros(10, np.float32), lr=0.01, beta1=0.9,
                   beta2=0.999, eps=1e-8, step=1)
    np.testing.assert_array_equal(host(strided[0][0]), p_ref)


def test_adam_groups_partial_steps_and_accumulation_are_bitwise_equal_in_one_launch():
    """tests/test_multi_adam.py:19-43: parameter groups (a rate multiplier; an absolute rate with
    weight decay), a parameter frozen for the first two updates, a parameter without a gradient at
    each update and accumulation counts 1-3: the multi-tensor optimiser (one launch per update) and
    the per-tensor one give the same parameters, moments and per-parameter steps bit for bit."""
    import myflows_amd as mf

    def trajectory(multi):
        rng = np.random.default_rng(7)
        nodes = [mf.Variable(gpu(rng.normal(size=n).astype(np.float32)), trainable=True)
                 for n in (1, 255, 256, 257, 8195)]
        groups = [{"name": "head", "params": nodes[:2], "lr_mult": .3},
                  {"name": "trunk", "params": nodes[2:], "lr": .002, "weight_decay": .001}]

        class Nodes:
            pass
        graph = Nodes()
        graph.nodes = nodes
        opt = mf.Adam(graph, learning_rate=.001, param_groups=groups, multi_tensor=multi)
        assert opt.group_learning_rates() == {"head": .001 * .3, "trunk": .002}
        for step in range(7):
            nodes[2].trainable = step >= 2
            opt.acc_no = 1 + step % 3
            for i, node in enumerate(nodes):
                g = rng.normal(size=node.value.shape).astype(np.float32)
                if i != step % 5:
                    opt.acc_gradient[node] = gpu(g)
            opt.update()
        return [(host(n.value), host(opt.v[n]), host(opt.s[n]), opt.parameter_steps[n]) for n in nodes]

    calls = []
    call = native._call
    native._call = lambda name, *args: (calls.append(name), call(name, *args))[1]
    try:
        batched = trajectory(True)
    finally:
        native._call = call
    assert calls.count("mfh_adam_step") == 7
    expected = trajectory(False)
    for left, right in zip(expected, batched):
        assert left[-1] == right[-1]
        for a, b in zip(left[:3], right[:3]):
            np.testing.assert_array_equal(a, b)
    assert [s for *_, s in batched] == [5, 5, 4, 6, 6]


# --- the reference's own edge cases (tests/test_fused_ops.py) --------------------------------------
def _adam_history(grads, lr=1e-3):
    """theta after each of the steps of mf.Adam fed `grads` one update at a time (acc_no = 1)."""
    import myflows_amd as mf

    node = mf.Variable(gpu(np.linspace(-1, 1, grads[0].size, dtype=np.float32).reshape(grads[0].shape)),
                       trainable=True)

    class OneParameter:
        nodes = (node,)

    opt = mf.Adam(OneParameter(), learning_rate=lr)
    history = []
    for g in grads:
        opt.acc_gradient = {node: gpu(g)}
        opt.acc_no = 1
        opt._update()
        history.append(host(node.value).copy())
    return history


def test_adam_follows_the_textbook_recurrence_over_four_steps():
    """tests/test_fused_ops.py:162-177: four steps against the FP64 textbook Adam, within 4 eps32
    (normwise), and the first step moves every coordinate by lr."""
    rng = np.random.default_rng(3)
    grads = [rng.standard_normal((5, 7)).astype(np.float32) for _ in range(4)]
    history = _adam_history(grads)
    start = np.linspace(-1, 1, 35, dtype=np.float32).reshape(5, 7)
    theta, m, v = start.astype(np.float64), np.zeros((5, 7)), np.zeros((5, 7))
    for t, g in enumerate(grads, 1):
        g = g.astype(np.float64)
        m = 0.9 * m + 0.1 * g
        v = 0.999 * v + 0.001 * g * g
        theta = theta - 1e-3 * (m / (1 - 0.9 ** t)) / (np.sqrt(v / (1 - 0.999 ** t)) + 1e-8)
        assert_near(history[t - 1], theta, 4 * np.finfo(np.float32).eps, f"step {t}")
    np.testing.assert_allclose(np.abs(history[0] - start), 1e-3, rtol=1e-3)


def test_adam_averages_the_gradient_over_the_accumulation_count():
    """tests/test_fused_ops.py:187-205: a gradient summed over acc_no = 2 steps gives exactly the
    update of its average taken as one step."""
    import myflows_amd as mf

    node = mf.Variable(torch.zeros(3, device="cuda"), trainable=True)

    class OneParameter:
        nodes = (node,)

    averaged, summed = mf.Adam(OneParameter(), learning_rate=0.1), mf.Adam(OneParameter(), learning_rate=0.1)
    averaged.acc_gradient, averaged.acc_no = {node: gpu(np.array([2.0, -4.0, 6.0], np.float32))}, 2
    averaged._update()
    first = host(node.value).copy()
    node.value = torch.zeros(3, device="cuda")
    summed.acc_gradient, summed.acc_no = {node: gpu(np.array([1.0, -2.0, 3.0], np.float32))}, 1
    summed._update()
    np.testing.assert_array_equal(first, host(node.value))
    assert np.all(first != 0)


def _bn_fp64(x, dy, gamma, beta, eps, training, rm, rv):
    x, dy, gamma, beta = (a.astype(np.float64) for a in (x, dy, gamma, beta))
    axes = (0, 2, 3)
    mean = x.mean(axis=axes) if training else rm.astype(np.float64)
    var = x.var(axis=axes) if training else rv.astype(np.float64)
    inv = 1.0 / np.sqrt(var + eps)
    ch = lambda a: a.reshape(1, -1, 1, 1)
    xhat = (x - ch(mean)) * ch(inv)
    dbeta, dgamma = dy.sum(axis=axes), (dy * xhat).sum(axis=axes)
    m = x.shape[0] * x.shape[2] * x.shape[3]
    dx = ch(gamma * inv) * (dy - ch(dbeta / m) - xhat * ch(dgamma / m)) if training else dy * ch(gamma * inv)
    return xhat * ch(gamma) + ch(beta), dx, dgamma, dbeta, mean, var


@pytest.mark.parametrize("shape,offset,scale", [((4, 3, 5, 7), 0.0, 1.0), ((2, 40, 9, 11), 0.0, 1.0),
                                                ((1, 2, 1, 1), 0.0, 1.0), ((8, 4, 6, 6), 1000.0, 0.01),
                                                ((64, 64, 29, 39), 1000.0, 0.01)], ids=str)
def test_batchnorm_operator_against_fp64_including_a_large_mean(shape, offset, scale):
    """tests/test_fused_ops.py:51-101 on the operator: y within 8 eps32, dx 64, dgamma 4, dbeta 2
    (normwise) of the FP64 batch norm, running statistics within 4 eps32, in training and eval mode;
    with mean 1e3 and std 1e-2 a float32 one-pass variance would lose every digit (the last case is
    the bs64 layer1 shape, which takes the two-launch path with several slices per channel)."""
    import myflows_amd as mf

    eps32 = np.finfo(np.float32).eps
    rng = np.random.default_rng(1)
    x = (offset + scale * rng.standard_normal(shape)).astype(np.float32)
    dy = rng.standard_normal(shape).astype(np.float32)
    c = shape[1]
    gamma = rng.uniform(0.5, 1.5, c).astype(np.float32)
    beta = rng.standard_normal(c).astype(np.float32)
    for training in (True, False):
        rm = (offset + 0.1 * rng.standard_normal(c)).astype(np.float32)
        rv = rng.uniform(0.5, 2.0, c).astype(np.float32) * np.float32(scale ** 2)
        running_mean, running_var = gpu(rm.copy()), gpu(rv.copy())
        nodes = [mf.Variable(gpu(a), trainable=True) for a in (x, gamma, beta)]
        op = mf.BatchNorm2d_Op(*nodes, running_mean, running_var, momentum=0.1, eps=1e-5, training=training)
        op.forward(*(n.value for n in nodes))
        op.grad = gpu(dy)
        op.backward()
        y, dx, dgamma, dbeta, mean, var = _bn_fp64(x, dy, gamma, beta, 1e-5, training, rm, rv)
        label = f"training={training}"
        assert op.value.dtype == torch.float32
        assert_near(host(op.value), y, 8 * eps32, f"y {label}")
        assert_near(host(nodes[0].grad), dx, 64 * eps32, f"dx {label}")
        assert_near(host(nodes[1].grad), dgamma, 4 * eps32, f"dgamma {label}")
        assert_near(host(nodes[2].grad), dbeta, 2 * eps32, f"dbeta {label}")
        if training:
            assert_near(host(running_mean), 0.9 * rm.astype(np.float64) + 0.1 * mean, 4 * eps32, "running_mean")
            assert_near(host(running_var), 0.9 * rv.astype(np.float64) + 0.1 * var, 4 * eps32, "running_var")
        else:
            np.testing.assert_array_equal(host(running_mean), rm)


# ---- batch norm + ReLU + max-pool as one unit --------------------------------------------------
POOL_UNIT_CASES = (
    ((64, 8, 60, 80), (3, 3), (2, 2)),   # the ResNet18 stem's shape at a quarter of its channels; float4 paths
    ((3, 5, 9, 11), (2, 2), (2, 2)),     # odd planes: scalar paths, one slice per channel
    ((24, 4, 31, 33), (3, 3), (1, 1)),   # overlapping windows, several slices that cut planes
    ((2, 3, 7, 8), (7, 8), (1, 1)),      # one window per plane
)


def _separate_bn_relu_pool(x, gamma, beta, rm, rv, kernel, stride, training):
    y, mean, inv_std = fused.batchnorm2d_forward(x, gamma, beta, rm, rv, momentum=0.1, eps=1e-5,
                                                 training=training, relu=True)
    pooled, context = native.maxpool2d_forward(y, kernel_size=kernel, stride=stride)
    return y, pooled, context, mean, inv_std


@pytest.mark.parametrize("shape,kernel,stride", POOL_UNIT_CASES, ids=str)
@pytest.mark.parametrize("training", (True, False))
@pytest.mark.parametrize("integer", (False, True), ids=("normal", "ties"))
def test_batchnorm_relu_pool_unit_equals_the_separate_passes(shape, kernel, stride, training, integer):
    """batchnorm2d_relu_pool_forward / _backward against batchnorm2d_forward(relu) + max-pool forward
    and max-pool backward + batchnorm2d_backward(gate=y): pooled values, argmax, statistics, running
    statistics and every gradient equal bit for bit (integer-valued inputs make ties and zero ReLU
    outputs common; the gradients are added into existing ones on a second call)."""
    x, gamma, beta, rm, rv, rng = bn_inputs(shape, 21)
    if integer:
        x = rng.integers(-3, 4, size=shape).astype(np.float32)
    xg, gg, bg = gpu(x), gpu(gamma), gpu(beta)
    rm1, rv1, rm2, rv2 = gpu(rm), gpu(rv), gpu(rm), gpu(rv)
    y, pooled, context, mean, inv_std = _separate_bn_relu_pool(xg, gg, bg, rm1, rv1, kernel, stride, training)
    pooled_u, argmax_u, mean_u, inv_std_u = fused.batchnorm2d_relu_pool_forward(
        xg, gg, bg, rm2, rv2, momentum=0.1, eps=1e-5, training=training, kernel_size=kernel, stride=stride)
    for a, b in ((pooled, pooled_u), (context.argmax, argmax_u), (mean, mean_u), (inv_std, inv_std_u),
                 (rm1, rm2), (rv1, rv2)):
        assert torch.equal(a, b)
    dp = gpu(rng.standard_normal(tuple(pooled.shape)).astype(np.float32))
    dy = native.maxpool2d_backward(dp, context)
    outs = []
    for unit in (False, True):
        grads = [torch.zeros_like(xg), torch.zeros_like(gg), torch.zeros_like(gg)]
        for _ in range(2):  # the second call adds into the first's gradients
            if unit:
                fused.batchnorm2d_relu_pool_backward(
                    xg, dp, argmax_u, gg, bg, mean_u, inv_std_u, training=training, kernel_size=kernel,
                    stride=stride, x_grad=grads[0], gamma_grad=grads[1], beta_grad=grads[2])
            else:
                fused.batchnorm2d_backward(xg, dy, gg, mean, inv_std, training=training, x_grad=grads[0],
                                           gamma_grad=grads[1], beta_grad=grads[2], gate=y)
        outs.append([host(g) for g in grads])
    for a, b in zip(*outs):
        np.testing.assert_array_equal(a, b)


def test_batchnorm_relu_pool_unit_with_nan_inputs():
    """A NaN in x propagates through BN and ReLU (NaN stays NaN) and wins its pooling windows, in
    the unit as in the separate passes; its gradient gate is closed (NaN > 0 is false)."""
    x, gamma, beta, rm, rv, rng = bn_inputs((2, 3, 9, 12), 5)
    x[0, 1, 4, 5] = np.nan
    xg, gg, bg = gpu(x), gpu(gamma), gpu(beta)
    _, pooled, context, _, _ = _separate_bn_relu_pool(xg, gg, bg, gpu(rm), gpu(rv), (3, 3), (2, 2), False)
    pooled_u, argmax_u, _, _ = fused.batchnorm2d_relu_pool_forward(
        xg, gg, bg, gpu(rm), gpu(rv), momentum=0.1, eps=1e-5, training=False, kernel_size=(3, 3), stride=(2, 2))
    assert torch.isnan(pooled_u).any()
    np.testing.assert_array_equal(host(pooled), host(pooled_u))
    assert torch.equal(context.argmax, argmax_u)


def test_batchnorm_relu_pool_unit_rejects_planes_beyond_its_lds():
    """A plane too large for the fused kernels' LDS staging is refused by the support query (the
    Graph unit then runs the separate nodes)."""
    assert fused.batchnorm_relu_pool_supported((2, 4, 60, 80), (3, 3), (2, 2))
    assert not fused.batchnorm_relu_pool_supported((1, 1, 200, 200), (3, 3), (2, 2))


@pytest.mark.parametrize("x_shape,w_shape,stride,residual", [
    ((64, 256, 8, 10), (512, 256, 3, 3), 2, False),   # layer4.0 conv1 at batch 64: 6 slices
    ((64, 512, 4, 5), (512, 512, 3, 3), 1, True),     # layer4 3x3, the BN with a residual: 6 slices
    ((64, 128, 15, 20), (256, 128, 3, 3), 2, False),  # layer3.0 conv1: 3 slices, 1024 threads per channel
], ids=("layer4-down", "layer4-residual", "layer3-down"))
def test_batch_norm_forms_a_deferred_convolution_output_bit_for_bit(x_shape, w_shape, stride, residual):
    """A split convolution product whose output the training batch norm forms (FP64 slice sums,
    the bias, then the statistics and y in one launch) against the product's own slice reduction
    followed by the batch norm: x, y, the statistics and the running statistics bit for bit."""
    print("deferred", x_shape, w_shape, flush=True)
    rng = np.random.default_rng(23)
    x = gpu(rng.standard_normal(x_shape).astype(np.float32))
    w = gpu((rng.standard_normal(w_shape) * (2.0 / np.prod(w_shape[1:])) ** 0.5).astype(np.float32))
    b = gpu(rng.standard_normal(w_shape[0]).astype(np.float32))
    c = w_shape[0]
    gamma, beta = gpu(rng.uniform(0.5, 1.5, c).astype(np.float32)), gpu(rng.standard_normal(c).astype(np.float32))
    conv = dict(stride=(stride, stride), padding=(1, 1))
    ref_x, _ = native.conv2d_forward(x, w, b, **conv)
    r = gpu(rng.standard_normal(tuple(ref_x.shape)).astype(np.float32)) if residual else None
    stats = [(torch.zeros(c, device="cuda"), torch.ones(c, device="cuda")) for _ in range(2)]
    bn = dict(momentum=0.1, eps=1e-5, training=True, relu=True, residual=r)
    ref = fused.batchnorm2d_forward(ref_x, gamma, beta, *stats[0], **bn)
    formed = native.conv2d_forward_deferred(x, w, b, max_positions=fused.SPLIT_FORM_MAX_POSITIONS, **conv)
    assert id(formed) in native._PENDING_SPLITS  # the plan splits K: the batch norm forms the output
    out = fused.batchnorm2d_forward(formed, gamma, beta, *stats[1], **bn)
    assert id(formed) not in native._PENDING_SPLITS
    for name, a, e in [("x", formed, ref_x), ("y", out[0], ref[0]), ("mean", out[1], ref[1]),
                       ("inv_std", out[2], ref[2]), ("running_mean", stats[1][0], stats[0][0]),
                       ("running_var", stats[1][1], stats[0][1])]:
        np.testing.assert_array_equal(host(a), host(e), err_msg=name)


def test_resnet_step_with_deferred_split_outputs_matches_the_plain_step():
    """ResNet18 at batch 64, 3x120x160 (the bench step): the Graph lets the training batch norms
    of layer3 and layer4 form their split convolutions' outputs; one forward and backward with and
    without that give the same loss, output and gradients bit for bit."""
    import myflows_amd as mf
    from myflows_amd import ops_conv
    from tests.test_gpu_model import build_resnet
    print("deferred step", flush=True)
    formed = []
    take = native.take_pending_split

    def counting(y):
        entry = take(y)
        formed.append(entry is not None)
        return entry

    runs = []
    for defer in (True, False):
        model, graph, out, loss, _, _ = build_resnet(64, 120, 160, optimize=True)
        graph.forward()  # installs the plan (and its Conv + BN pairs)
        convs = [n for n in graph.nodes if type(n) is ops_conv.Conv2D_Op]
        assert sum(n._defer_bn is not None for n in convs) == 19
        if not defer:
            for n in convs:
                n._defer_bn = None
        native.take_pending_split = counting
        try:
            graph.forward()
        finally:
            native.take_pending_split = take
        graph.backward()
        runs.append([host(loss.value), host(out.value)] + [host(p.grad) for p in model.params])
        if defer:
            assert sum(formed) == 8  # layer3's and layer4's split 3x3 products
        formed.clear()
    for a, b in zip(*runs):
        np.testing.assert_array_equal(a, b)


def test_a_product_between_a_deferred_output_and_its_batch_norm_leaves_the_slices_alone():
    """A deferred product's slices wait in its stream's convolution workspace: another split product
    issued on that stream before the batch norm takes a fresh workspace block (the pending one is
    never handed out), so the batch norm still forms the first output with the plain path's bits."""
    print("deferred then another split product", flush=True)
    rng = np.random.default_rng(29)
    x = gpu(rng.standard_normal((64, 512, 4, 5)).astype(np.float32))
    w = gpu((rng.standard_normal((512, 512, 3, 3)) * 0.02).astype(np.float32))
    b = gpu(rng.standard_normal(512).astype(np.float32))
    x2 = gpu(rng.standard_normal((64, 256, 8, 10)).astype(np.float32))
    w2 = gpu((rng.standard_normal((512, 256, 3, 3)) * 0.03).astype(np.float32))
    gamma, beta = gpu(rng.uniform(0.5, 1.5, 512).astype(np.float32)), gpu(rng.standard_normal(512).astype(np.float32))
    conv = dict(stride=(1, 1), padding=(1, 1))
    ref_x, _ = native.conv2d_forward(x, w, b, **conv)
    ref_x2, _ = native.conv2d_forward(x2, w2, None, stride=(2, 2), padding=(1, 1))
    stats = [(torch.zeros(512, device="cuda"), torch.ones(512, device="cuda")) for _ in range(2)]
    bn = dict(momentum=0.1, eps=1e-5, training=True, relu=True)
    ref = fused.batchnorm2d_forward(ref_x, gamma, beta, *stats[0], **bn)
    formed = native.conv2d_forward_deferred(x, w, b, max_positions=fused.SPLIT_FORM_MAX_POSITIONS, **conv)
    assert id(formed) in native._PENDING_SPLITS
    between, _ = native.conv2d_forward(x2, w2, None, stride=(2, 2), padding=(1, 1))  # splits K too
    out = fused.batchnorm2d_forward(formed, gamma, beta, *stats[1], **bn)
    np.testing.assert_array_equal(host(between), host(ref_x2))
    for name, a, e in [("x", formed, ref_x), ("y", out[0], ref[0]), ("mean", out[1], ref[1])]:
        np.testing.assert_array_equal(host(a), host(e), err_msg=name)


def test_single_stream_step_with_deferred_outputs_matches_the_plain_step_where_the_downsample_splits():
    """ResNet18 at batch 16, 3x120x160, on one stream (overlap_branches=False: the order a profiler
    or the single-stream bench runs): the downsample products of layer3/layer4 split K and run
    between a block's second convolution and its batch norm, so the Graph pairs only convolutions
    whose batch norm is the next unit on their stream. Loss, output and every gradient equal the
    step without deferred outputs bit for bit, and so does the two-stream step."""
    from myflows_amd import ops_conv
    from tests.test_gpu_model import build_resnet
    print("single-stream deferred step bs16", flush=True)
    runs = []
    for overlap, defer in ((False, True), (False, False), (True, True)):
        model, graph, out, loss, _, _ = build_resnet(16, 120, 160, optimize=True)
        graph.overlap_branches = overlap
        graph.forward()  # installs the plan and its pairs for this order
        convs = [n for n in graph.nodes if type(n) is ops_conv.Conv2D_Op]
        assert sum(n._defer_bn is not None for n in convs) == (19 if overlap else 16)
        if not defer:
            for n in convs:
                n._defer_bn = None
        graph.forward()
        graph.backward()
        assert not native._PENDING_SPLITS
        runs.append([host(loss.value), host(out.value)] + [host(p.grad) for p in model.params])
    for other in runs[1:]:
        for a, b in zip(runs[0], other):
            np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("x_shape,two_streams", [
    ((64, 256, 8, 10), True),    # layer3 3x3 at batch 64, dW on the weight-gradient stream
    ((64, 512, 4, 5), True),     # layer4 3x3
    ((64, 512, 4, 5), False),    # layer4 3x3, one stream (dW and dX parts of one stream workspace)
], ids=("layer3-streams", "layer4-streams", "layer4-one-stream"))
def test_batch_norm_backward_forms_a_deferred_input_gradient_bit_for_bit(x_shape, two_streams):
    """A stride-1 convolution backward whose dX product splits K leaves dx in slices; the next
    batch-norm backward (BN+ReLU, training) forms dx (FP64 slice sums rounded once) and then its
    gradients in one launch. dx, x_grad, dgamma, dbeta and the convolution's dW and db equal the
    plain path's (the product's own slice reduction, then the batch-norm backward) bit for bit."""
    from myflows_amd import streams
    print("deferred dx", x_shape, "two streams" if two_streams else "one stream", flush=True)
    rng = np.random.default_rng(31)
    n, c, h, w = x_shape
    # The batch norm's input and output (the convolution's input), and the convolution's kernel.
    bn_x = gpu(rng.standard_normal(x_shape).astype(np.float32))
    gamma, beta = gpu(rng.uniform(0.5, 1.5, c).astype(np.float32)), gpu(rng.standard_normal(c).astype(np.float32))
    stats = (torch.zeros(c, device="cuda"), torch.ones(c, device="cuda"))
    y, mean, inv_std = fused.batchnorm2d_forward(bn_x, gamma, beta, *stats, momentum=0.1, eps=1e-5, training=True,
                                                 relu=True)
    kernel = gpu((rng.standard_normal((c, c, 3, 3)) * (2.0 / (9 * c)) ** 0.5).astype(np.float32))
    dy = gpu(rng.standard_normal(x_shape).astype(np.float32))
    conv = dict(stride=(1, 1), padding=(1, 1), algorithm="implicit")
    results = []
    for defer in (False, True):
        hold = [] if two_streams else None
        side = streams.side_stream(0).cuda_stream if two_streams else None
        dx, dw, db = native.conv2d_backward(y, kernel, dy, None, dw_stream=side, hold=hold,
                                            defer_dx_positions=fused.SPLIT_FORM_MAX_POSITIONS if defer else 0, **conv)
        if defer:
            assert id(dx) in native._PENDING_SPLITS  # the dX plan splits K: the batch norm forms dx
        grads = [torch.empty_like(bn_x), torch.empty_like(gamma), torch.empty_like(gamma)]
        fused.batchnorm2d_backward(bn_x, dx, gamma, mean, inv_std, training=True, x_grad=grads[0],
                                   gamma_grad=grads[1], beta_grad=grads[2], accumulate=(False, False, False), gate=y)
        assert id(dx) not in native._PENDING_SPLITS
        if two_streams:
            native.stream_wait(native._stream(), side)
        results.append([host(t) for t in (dx, dw, db, *grads)])
    for name, a, e in zip(("dx", "dw", "db", "x_grad", "gamma_grad", "beta_grad"), results[1], results[0]):
        np.testing.assert_array_equal(a, e, err_msg=name)


def test_resnet_step_with_deferred_input_gradients_matches_the_plain_step():
    """ResNet18 at batch 64, 3x120x160 (the bench step), both streams: the Graph lets the batch-norm
    units of layer3 and layer4 form the split dX of the convolution they feed; one forward and
    backward with and without that give the same loss, output and gradients bit for bit."""
    from myflows_amd import ops_conv
    from tests.test_gpu_model import build_resnet
    print("deferred dx step", flush=True)
    formed = []
    take = native.take_pending_split

    def counting(y):
        entry = take(y)
        formed.append(entry is not None)
        return entry

    runs = []
    for defer in (True, False):
        model, graph, out, loss, _, _ = build_resnet(64, 120, 160, optimize=True)
        graph.forward()
        graph.backward()  # installs the plan's deferred dX pairs
        convs = [n for n in graph.nodes if type(n) is ops_conv.Conv2D_Op]
        assert sum(n._defer_dx is not None for n in convs) == 8  # each block's second convolution
        graph.forward()
        if not defer:  # the plan's pairs stay installed, so the next backward keeps these
            for n in convs:
                n._defer_dx = None
        native.take_pending_split = counting
        try:
            graph.backward()
        finally:
            native.take_pending_split = take
        assert not native._PENDING_SPLITS
        runs.append([host(loss.value), host(out.value)] + [host(p.grad) for p in model.params])
        if defer:
            print("dX formed by batch norms:", sum(formed), flush=True)
            assert sum(formed) >= 1  # layer3/layer4 second convolutions whose dX plans split K
        formed.clear()
    for a, b in zip(*runs):
        np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("shape", [(4, 2048, 56, 56), (256, 2048, 7, 7)], ids=str)
def test_batchnorm_of_a_wide_layer_with_many_positions_against_fp64(shape):
    """C >= 8 * CUs channels with more positions per channel than the one-launch channel kernels
    hold (8192): the pass splits each channel into slices (two launches) and every position is
    normalised: y and dx against the FP64 batch norm, as the operator test bounds them."""
    import myflows_amd as mf
    print("wide batch norm", shape, flush=True)
    eps32 = np.finfo(np.float32).eps
    rng = np.random.default_rng(31)
    x = rng.normal(0.5, 2.0, shape).astype(np.float32)
    dy = rng.standard_normal(shape).astype(np.float32)
    c = shape[1]
    gamma, beta = rng.uniform(0.5, 1.5, c).astype(np.float32), rng.standard_normal(c).astype(np.float32)
    nodes = [mf.Variable(gpu(a), trainable=True) for a in (x, gamma, beta)]
    rm, rv = np.zeros(c, np.float32), np.ones(c, np.float32)
    op = mf.BatchNorm2d_Op(*nodes, gpu(rm), gpu(rv), momentum=0.1, eps=1e-5, training=True)
    op.forward(*(n.value for n in nodes))
    op.grad = gpu(dy)
    op.backward()
    y, dx, dgamma, dbeta, _, _ = _bn_fp64(x, dy, gamma, beta, 1e-5, True, rm, rv)
    assert_near(host(op.value), y, 8 * eps32, "y")
    assert_near(host(nodes[0].grad), dx, 64 * eps32, "dx")
    assert_near(host(nodes[1].grad), dgamma, 4 * eps32, "dgamma")
    assert_near(host(nodes[2].grad), dbeta, 2 * eps32, "dbeta")
