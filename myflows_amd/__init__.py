"""myflows_amd: the MI355X (gfx950) hip_native backend of MyFlows' convolution / GEMM / max-pool path.

The public names mirror the reference package (``Variable``, ``Graph``, ``Conv2D``, ``Dense``,
``MaxPool2d``, ``ResNet18``, ``Adam``, ...). Layers and operators take ``backend="hip_native"``
(``conv_backend=`` for ResNet18); the kernels live in ``libmfhip.so`` (``native``).
"""

from .activation import MSELoss, ReLU
from .basic import Add, Linear
from .batchnorm import BatchNorm2d_Op, GlobalAvgPool2d_Op
from .convolution import (BACKENDS, NATIVE_BACKENDS, Conv2D_LeakyReLU_Op, Conv2D_Op, Conv2D_ReLU_Op, Flatten_Op,
                          MaxPool2d_Op)
from .core import GradientOp, Graph, Node, Variable
from .device import cuda_available, get_device, set_device
from .initializers import make_initializer
from .layers import Conv2D, Dense, Flatten, Layer, MaxPool2d
from .opt import MBGD, Adam, Optimizer
from .resnet import BasicBlock, BatchNorm2d, GlobalAvgPool2d, ResNet18
from . import native

__all__ = [
    "Add", "Adam", "BACKENDS", "BasicBlock", "BatchNorm2d", "BatchNorm2d_Op", "Conv2D", "Conv2D_LeakyReLU_Op",
    "Conv2D_Op", "Conv2D_ReLU_Op", "Dense", "Flatten", "Flatten_Op", "GlobalAvgPool2d", "GlobalAvgPool2d_Op",
    "GradientOp", "Graph", "Layer", "Linear", "MBGD", "MSELoss", "MaxPool2d", "MaxPool2d_Op", "NATIVE_BACKENDS",
    "Node", "Optimizer", "ReLU", "ResNet18", "Variable", "cuda_available", "get_device", "make_initializer",
    "native", "set_device",
]
