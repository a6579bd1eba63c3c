"""ResNet18's structure options, as the reference's ``layers/resnet.py:200-240`` defines them, and the
two device-arithmetic operators they add (``ops/pooling.py:65-87`` ChannelNormalize_Op,
``ops/dropout.py:12-40`` Dropout_Op). Graph building and host tensors only: runs on the CPU."""

import numpy as np
import pytest
import torch

import myflows_amd as mf
from myflows_amd import device


@pytest.fixture
def on_cpu():
    previous = device.get_device()
    device.set_device("cpu")
    try:
        yield
    finally:
        device.set_device(previous)


def _convs(model):
    layers = [model.stem_conv]
    for block in model.blocks():
        layers += [block.conv1, block.conv2] + ([block.downsample_conv] if block.downsample else [])
    return layers


def _bns(model):
    bns = [model.stem_bn]
    for block in model.blocks():
        bns += [block.bn1, block.bn2] + ([block.downsample_bn] if block.downsample else [])
    return bns


def test_torchvision_structure_and_argument_checks(on_cpu):
    default = mf.ResNet18(output_dim=2, base_width=8, initializer=mf.make_initializer(seed=0))
    assert all(conv.b is not None for conv in _convs(default))
    assert not any(bn.unbiased_running_var for bn in _bns(default))
    tv = mf.ResNet18(output_dim=2, compat="torchvision", initializer=mf.make_initializer(seed=0))
    assert all(conv.b is None for conv in _convs(tv)) and len(tv.params) == len(default.params) - 20
    assert all(bn.unbiased_running_var for bn in _bns(tv))
    # The stem pool pads by one in torchvision's structure.
    x = mf.Variable(torch.zeros((1, 3, 32, 32)), requires_grad=False)
    pools = [n for n in mf.Graph(tv.spatial_features(x)).nodes if isinstance(n, mf.MaxPool2d_Op)]
    assert [p.padding for p in pools] == [(1, 1)]
    for kwargs in ({"compat": "keras"}, {"compat": "torchvision", "stem": "cifar"},
                   {"compat": "torchvision", "base_width": 32}, {"compat": "torchvision", "in_channels": 1},
                   {"input_norm": "cifar"}, {"stem": "tiny"}):
        with pytest.raises(ValueError):
            mf.ResNet18(**kwargs)


def test_channel_normalize_and_its_gradient(on_cpu):
    rng = np.random.default_rng(1)
    x_np = rng.random((2, 3, 4, 5)).astype(np.float32)
    x = mf.Variable(torch.as_tensor(x_np), trainable=True)
    node = mf.ChannelNormalize_Op(x)
    node.forward(x.value)
    mean = np.array([0.485, 0.456, 0.406], np.float32).reshape(1, 3, 1, 1)
    std = np.array([0.229, 0.224, 0.225], np.float32).reshape(1, 3, 1, 1)
    np.testing.assert_array_equal(node.value.numpy(), (x_np - mean) / std)
    node.grad = torch.ones_like(node.value)
    node.backward()
    np.testing.assert_array_equal(x.grad.numpy(), np.broadcast_to(np.float32(1.0) / std, x_np.shape))
    with pytest.raises(ValueError):
        mf.ChannelNormalize_Op(x, std=(1.0, 0.0, 1.0))
    bad = mf.ChannelNormalize_Op(x)
    with pytest.raises(ValueError):
        bad.forward(torch.zeros((2, 4, 4, 5)))


def test_dropout_masks_follow_the_seed_and_eval_is_the_identity(on_cpu):
    x_np = np.random.default_rng(2).standard_normal((3, 16)).astype(np.float32)
    x = mf.Variable(torch.as_tensor(x_np), trainable=True)
    layer = mf.Dropout(0.25, seed=7)
    op = layer(x)
    op.forward(x.value)
    keep = 0.75
    mask = (np.random.default_rng(7).random(x_np.shape) < keep).astype(np.float32) / np.float32(keep)
    np.testing.assert_array_equal(op.value.numpy(), x_np * mask)
    op.grad = torch.ones_like(op.value)
    op.backward()
    np.testing.assert_array_equal(x.grad.numpy(), mask)
    layer.eval()
    op.forward(x.value)
    assert op.value is x.value
    with pytest.raises(ValueError):
        mf.Dropout(1.0)
    model = mf.ResNet18(output_dim=2, base_width=8, dropout=0.5, dropout_seed=3)
    assert model.dropout is not None and model.dropout in model.sub_layers
    model.eval()
    assert not model.dropout.training
    assert mf.ResNet18(output_dim=2, base_width=8).dropout is None
