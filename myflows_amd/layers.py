"""Layers with the reference's constructor arguments (``layers/layer.py:36-425``): ``Dense``,
``Conv2D``, ``MaxPool2d`` and ``Flatten``, each taking ``backend=`` ("hip_native", or "auto", which
is hip_native on the GPU), and ``Dropout``. Parameters are drawn by the seeded initialiser in float64 and cast to
float32 on the active device, so a seeded model holds the reference model's weights.
"""

from __future__ import annotations

import weakref

import torch

from .device import asarray
from .graph import Variable
from .init import make_initializer
from .ops_basic import Dropout_Op, Linear, ReLU, _linear_backend
from .ops_conv import Conv2D_Op, Conv2D_ReLU_Op, Flatten_Op, MaxPool2d_Op, _backend_name, _int_pair


def _count(value, name):
    value = int(value)
    if value <= 0:
        raise ValueError(f"{name} must be positive, got {value}")
    return value


def _parameter(data, layer_name, suffix):
    return Variable(asarray(data), trainable=True, name=f"{layer_name}_{suffix}" if layer_name else suffix)


class Layer:
    """Builds graph nodes on call; ``params`` lists its trainable Variables."""

    def __init__(self, name=None):
        self.name = name
        self.params = []

    def __call__(self, *args, **kwargs):
        return self.forward(*args, **kwargs)


class Dense(Layer):
    """Z = X W + b, with W (input_dim, output_dim) and b (1, output_dim)."""

    def __init__(self, input_dim, output_dim, activation=None, name=None, initializer=None, dtype=None,
                 backend="auto"):
        super().__init__(name=name)
        self.backend = _linear_backend(backend)
        draw = make_initializer(initializer)
        self.W = _parameter(draw((input_dim, output_dim)), name, "W")
        self.b = _parameter(torch.zeros((1, output_dim), dtype=torch.float64), name, "b")
        self.params = [self.W, self.b]
        self.activation = activation

    def forward(self, input_node):
        z = Linear(input_node, self.W, self.b, backend=self.backend)
        return self.activation(z) if self.activation else z


class Conv2D(Layer):
    """2-D convolution, kernel (out, in, kh, kw) and optional bias (out,). With activation=ReLU and
    fuse_activation, the ReLU runs in the convolution's epilogue (Conv2D_ReLU_Op)."""

    def __init__(self, in_channels, out_channels, kernel_size=3, stride=1, padding=0, groups=1, dilation=1,
                 activation=None, fuse_activation=True, name=None, initializer=None, dtype=None, backend="auto",
                 bias=True, recompute_im2col=None):
        super().__init__(name=name)
        self.backend = _backend_name(backend)
        self.in_channels, self.out_channels = _count(in_channels, "in_channels"), _count(out_channels, "out_channels")
        self.groups = _count(groups, "groups")
        if self.in_channels % self.groups or self.out_channels % self.groups:
            raise ValueError("in_channels and out_channels must be divisible by groups")
        self.kernel_size = _int_pair(kernel_size, "kernel_size")
        self.stride = _int_pair(stride, "stride")
        self.padding = _int_pair(padding, "padding", minimum=0)
        self.dilation = _int_pair(dilation, "dilation")
        self.recompute_im2col = recompute_im2col
        draw = make_initializer(initializer)
        shape = (self.out_channels, self.in_channels // self.groups, *self.kernel_size)
        self.kernel = _parameter(draw(shape), name, "kernel")
        self.b = _parameter(torch.zeros(self.out_channels, dtype=torch.float64), name, "bias") if bias else None
        self.params = [self.kernel] if self.b is None else [self.kernel, self.b]
        self.activation = activation
        self.fuse_activation = bool(fuse_activation)

    def forward(self, input_node):
        options = dict(stride=self.stride, padding=self.padding, groups=self.groups, dilation=self.dilation,
                       bias=self.b, backend=self.backend, recompute_im2col=self.recompute_im2col)
        if self.fuse_activation and self.activation is ReLU:
            return Conv2D_ReLU_Op(input_node, self.kernel, **options)
        out = Conv2D_Op(input_node, self.kernel, **options)
        return self.activation(out) if self.activation else out


class MaxPool2d(Layer):
    def __init__(self, kernel_size=2, stride=2, name=None, backend="auto", padding=0):
        super().__init__(name=name)
        self.backend = _backend_name(backend)
        self.k, self.s = kernel_size, stride
        self.padding = _int_pair(padding, "padding", minimum=0)

    def forward(self, input_node):
        return MaxPool2d_Op(input_node, self.k, self.s, backend=self.backend, padding=self.padding)


class Flatten(Layer):
    def forward(self, input_node):
        return Flatten_Op(input_node)


class Dropout(Layer):
    """Inverted dropout (Dropout_Op): active in train mode, the identity in eval mode; ``train()`` /
    ``eval()`` switch every operator the layer has built. The reference's ``layers/layer.py:391-416``."""

    def __init__(self, p=0.5, seed=None, name=None):
        super().__init__(name=name)
        self.p = float(p)
        if self.p < 0.0 or self.p >= 1.0:
            raise ValueError("dropout p must be in [0, 1)")
        self.seed = seed
        self.training = True
        self._built = weakref.WeakSet()

    def forward(self, input_node):
        op = Dropout_Op(input_node, p=self.p, training=self.training, seed=self.seed, name=self.name)
        self._built.add(op)
        return op

    def train(self, mode=True):
        self.training = bool(mode)
        for op in self._built:
            op.training = self.training

    def eval(self):
        self.train(False)
