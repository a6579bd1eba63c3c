"""The fused BN(+Add)+ReLU execution unit of Graph(optimize=True) against the separate nodes, after
the reference's tests/test_bn_activation_fusion.py:14-77: three passes with a train / eval / train
flip of the layer, residual None, of the BN's shape and a per-channel (C,) one (which the unit runs
as its chained route), with and without retain_grad of the hidden BN output and of the ReLU output.
Every value, running statistic and gradient equals the unfused graph's bit for bit, and the fused
unit leaves the hidden BN output unformed. Graph.materialize_intermediates keeps those values for
inspection with the same bits.
"""

import numpy as np
import pytest
import torch

import myflows_amd as mf
from myflows_amd.resnet import BatchNorm2d

pytestmark = pytest.mark.gpu


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def trajectory(optimized, residual_shape, retain):
    rng = np.random.default_rng(271)
    x = mf.Variable(torch.as_tensor(rng.normal(size=(2, 4, 3, 5)).astype(np.float32), device="cuda"), trainable=True)
    layer = BatchNorm2d(4, unbiased_running_var=True)
    base = layer(x)
    residual = None
    if residual_shape:
        residual = mf.Variable(torch.as_tensor(rng.normal(size=residual_shape).astype(np.float32), device="cuda"),
                               trainable=True)
    total = mf.Add(base, residual) if residual else base
    output = mf.ReLU(total)
    coeff = mf.Variable(torch.as_tensor(rng.normal(size=(2, 4, 3, 5)).astype(np.float32), device="cuda"),
                        requires_grad=False)
    graph = mf.Graph(mf.MSELoss(output, coeff), optimize=optimized)
    if retain:
        graph.retain_grad(base, output)
    assert len(graph._bn_groups) == int(optimized)
    states = []
    for training in (True, False, True):
        layer.train(training)
        graph.forward()
        graph.backward()
        values = [output.value, graph.target_node.value, layer.running_mean, layer.running_var, x.grad,
                  layer.gamma.grad, layer.beta.grad]
        if residual:
            values.append(residual.grad)
        if retain:
            values.extend((base.value, base.grad, output.grad))
        elif optimized and (residual_shape is None or residual_shape == (2, 4, 3, 5)):
            assert base.value is None  # the fused unit never forms the BN output
        states.extend(host(v).tobytes() for v in values)
    return states


@pytest.mark.parametrize("residual_shape", (None, (2, 4, 3, 5), (4,)), ids=("none", "same", "per-channel"))
@pytest.mark.parametrize("retain", (False, True), ids=("plain", "retained"))
def test_fused_unit_trajectory_equals_the_separate_nodes(residual_shape, retain):
    print("bn unit", residual_shape, retain, flush=True)
    assert trajectory(False, residual_shape, retain) == trajectory(True, residual_shape, retain)


def test_materialized_intermediates_keep_the_bn_output_for_one_pass():
    """materialize_intermediates(): the next forward forms the BN output (the separate node's
    value) and the ReLU output has the fused unit's bits; switched off, the BN output is left
    unformed again."""
    print("materialize intermediates", flush=True)
    rng = np.random.default_rng(5)
    x = mf.Variable(torch.as_tensor(rng.normal(size=(2, 3, 3, 3)).astype(np.float32), device="cuda"), trainable=True)
    layer = BatchNorm2d(3)
    bn = layer(x)
    relu = mf.ReLU(bn)
    graph = mf.Graph(relu, optimize=True)
    graph.forward()
    assert bn.value is None
    fused_out = host(relu.value)
    layer.running_mean.zero_()
    layer.running_var.fill_(1.0)
    graph.materialize_intermediates()
    graph.forward()
    assert bn.value is not None
    np.testing.assert_array_equal(host(relu.value), fused_out)
    np.testing.assert_array_equal(host(torch.clamp_min(bn.value, 0.0)), fused_out)
    graph.backward()
    assert x.grad is not None
    graph.materialize_intermediates(False)
    graph.forward()
    assert bn.value is None
