"""Graph(optimize=True) fuses a BN(+Add)+ReLU chain only when the chain's values and the batch
norm's running statistics are private to it (the reference's
tests/test_bn_activation_fusion.py:71-77): a BN output that another node also reads, or running
statistics that a second BN shares, leave the chain unfused. Graph building only: runs on the CPU."""

import torch

import myflows_amd as mf
from myflows_amd import device
from myflows_amd.resnet import BatchNorm2d


def test_shared_bn_outputs_and_reused_running_statistics_are_not_fused():
    previous = device.get_device()
    device.set_device("cpu")
    try:
        x = mf.Variable(torch.ones((2, 3, 3, 3)), trainable=True)
        layer = BatchNorm2d(3)
        bn = layer(x)
        assert not mf.Graph(mf.Add(mf.ReLU(bn), bn), optimize=True)._bn_groups
        assert not mf.Graph(mf.Add(mf.ReLU(bn), mf.ReLU(layer(x))), optimize=True)._bn_groups
        # A private chain is fused.
        assert len(mf.Graph(mf.ReLU(BatchNorm2d(3)(x)), optimize=True)._bn_groups) == 1
    finally:
        device.set_device(previous)


def test_materialize_intermediates_drops_the_fused_units_from_the_plan():
    previous = device.get_device()
    device.set_device("cpu")
    try:
        x = mf.Variable(torch.ones((2, 3, 3, 3)), trainable=True)
        relu = mf.ReLU(BatchNorm2d(3)(x))
        graph = mf.Graph(relu, optimize=True)
        assert graph._plan().groups
        graph.materialize_intermediates()
        assert not graph._plan().groups
        graph.materialize_intermediates(False)
        assert graph._plan().groups
    finally:
        device.set_device(previous)
