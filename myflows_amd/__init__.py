"""myflows_amd: the MI355X (gfx950) ``hip_native`` backend of MyFlows' convolution / GEMM / max-pool
path, with the Variable / Graph / layer / optimiser API it plugs under.

The public names mirror the reference package (``Variable``, ``Graph``, ``Conv2D``, ``Dense``,
``MaxPool2d``, ``ResNet18``, ``Adam``, ...). Layers and operators take ``backend="hip_native"``
(``conv_backend=`` for ResNet18); the kernels live in ``libmfhip.so`` (``native`` and ``fused``).
"""

from . import fused, native
from .capture import CapturedStep, RecordedStep
from .device import cuda_available, get_device, set_device
from .fusion import apply_graph_optimizations
from .graph import GradientOp, Graph, Node, Variable
from .init import make_initializer
from .layers import Conv2D, Dense, Dropout, Flatten, Layer, MaxPool2d
from .ops_basic import LINEAR_BACKENDS, Add, ChannelNormalize_Op, Dropout_Op, LeakyReLU, Linear, MSELoss, ReLU
from .ops_conv import (BACKENDS, NATIVE_BACKENDS, Conv2D_AddReLU_Op, Conv2D_LeakyReLU_Op, Conv2D_Op, Conv2D_ReLU_Op,
                       Flatten_Op, MaxPool2d_Op)
from .ops_norm import BatchNorm2d_Op, BatchNormActivation, BatchNormReLUPool, GlobalAvgPool2d_Op
from .optim import MBGD, Adam, Optimizer, ParameterGroups
from .resnet import BasicBlock, BatchNorm2d, GlobalAvgPool2d, ResNet18

__all__ = [
    "Adam", "Add", "BACKENDS", "BasicBlock", "BatchNorm2d", "BatchNorm2d_Op", "BatchNormActivation",
    "BatchNormReLUPool", "CapturedStep", "ChannelNormalize_Op", "Conv2D", "Dropout", "Dropout_Op",
    "Conv2D_AddReLU_Op", "Conv2D_LeakyReLU_Op", "Conv2D_Op", "Conv2D_ReLU_Op", "Dense", "Flatten", "Flatten_Op",
    "GlobalAvgPool2d", "GlobalAvgPool2d_Op", "GradientOp", "Graph", "LINEAR_BACKENDS", "Layer", "LeakyReLU", "Linear", "MBGD",
    "MSELoss", "MaxPool2d", "MaxPool2d_Op", "NATIVE_BACKENDS", "Node", "Optimizer", "ParameterGroups",
    "RecordedStep", "ReLU", "ResNet18", "Variable",
    "apply_graph_optimizations", "cuda_available", "fused", "get_device", "make_initializer", "native",
    "set_device",
]
