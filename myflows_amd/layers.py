"""Layers with the reference's constructor arguments (``layers/layer.py:36-383``): Dense, Conv2D,
MaxPool2d and Flatten, each taking ``backend=`` ("hip_native" or "auto", which is hip_native on the
GPU). Parameters are drawn with the seeded initialisers in float64 and cast to float32 on the
active device, so a seeded model matches the reference's weights."""

from __future__ import annotations

from .basic import Linear, _linear_backend
from .convolution import Conv2D_Op, Conv2D_ReLU_Op, Flatten_Op, MaxPool2d_Op, _backend_name, _normalize_pair
from .core import Variable
from .device import asarray
from .initializers import make_initializer


class Layer:
    def __init__(self, name=None):
        self.name = name
        self.params = []

    def __call__(self, *args, **kwargs):
        return self.forward(*args, **kwargs)


class Dense(Layer):
    """Z = X W + b (layers/layer.py:46-76)."""

    def __init__(self, input_dim, output_dim, activation=None, name=None, initializer=None, dtype=None,
                 backend="auto"):
        super().__init__(name=name)
        self.backend = _linear_backend(backend)
        init = make_initializer(initializer)
        self.W = Variable(asarray(init((input_dim, output_dim))), trainable=True, name=f"{name}_W" if name else "W")
        self.b = Variable(asarray([[0.0] * output_dim]), trainable=True, name=f"{name}_b" if name else "b")
        self.params = [self.W, self.b]
        self.activation = activation

    def forward(self, input_node):
        z = Linear(input_node, self.W, self.b, backend=self.backend)
        return self.activation(z) if self.activation else z


class Conv2D(Layer):
    """layers/layer.py:79-170; groups and dilation other than 1 are rejected by the native operator."""

    def __init__(self, in_channels, out_channels, kernel_size=3, stride=1, padding=0, groups=1, dilation=1,
                 activation=None, fuse_activation=True, name=None, initializer=None, dtype=None, backend="auto",
                 bias=True, recompute_im2col=None):
        super().__init__(name=name)
        self.backend = _backend_name(backend)
        self.recompute_im2col = recompute_im2col
        if int(in_channels) <= 0 or int(out_channels) <= 0 or int(groups) <= 0:
            raise ValueError("channel counts and groups must be positive")
        kh, kw = _normalize_pair(kernel_size, "kernel_size")
        self.stride = _normalize_pair(stride, "stride")
        self.padding = _normalize_pair(padding, "padding", allow_zero=True)
        self.dilation = _normalize_pair(dilation, "dilation")
        if in_channels % groups or out_channels % groups:
            raise ValueError("channels must be divisible by groups")
        init = make_initializer(initializer)
        self.kernel = Variable(asarray(init((out_channels, in_channels // groups, kh, kw))), trainable=True,
                               name=f"{name}_kernel" if name else "kernel")
        self.b = (Variable(asarray([0.0] * out_channels), trainable=True, name=f"{name}_bias" if name else "bias")
                  if bias else None)
        self.params = [self.kernel] if self.b is None else [self.kernel, self.b]
        self.in_channels, self.out_channels = in_channels, out_channels
        self.kernel_size = (kh, kw)
        self.groups = groups
        self.activation = activation
        self.fuse_activation = bool(fuse_activation)

    def forward(self, input_node):
        from .activation import ReLU

        kwargs = dict(stride=self.stride, padding=self.padding, groups=self.groups, dilation=self.dilation,
                      bias=self.b, backend=self.backend, recompute_im2col=self.recompute_im2col)
        if self.fuse_activation and self.activation is ReLU:
            return Conv2D_ReLU_Op(input_node, self.kernel, **kwargs)
        out = Conv2D_Op(input_node, self.kernel, **kwargs)
        return self.activation(out) if self.activation else out


class MaxPool2d(Layer):
    def __init__(self, kernel_size=2, stride=2, name=None, backend="auto", padding=0):
        super().__init__(name=name)
        self.backend = _backend_name(backend)
        self.k, self.s = kernel_size, stride
        self.padding = _normalize_pair(padding, "padding", allow_zero=True)

    def forward(self, input_node):
        return MaxPool2d_Op(input_node, self.k, self.s, backend=self.backend, padding=self.padding)


class Flatten(Layer):
    def forward(self, input_node):
        return Flatten_Op(input_node)
