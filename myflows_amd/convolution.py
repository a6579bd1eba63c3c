"""Convolution and pooling operators on the ``hip_native`` backend.

Restates the native branches of the reference's ``ops/convolution.py``: ``Conv2D_Op`` (:287-523,
native forward :347-360, native backward :446-457), ``Conv2D_ReLU_Op`` (:526-545),
``Conv2D_LeakyReLU_Op`` (:548-573), ``MaxPool2d_Op`` (:817-890) and ``Flatten_Op`` (:893-898).
The backend value ``hip_native`` selects libmfhip; ``auto`` means ``hip_native`` on the GPU. There is
no CPU path in this package: CPU arrays are rejected like the reference rejects a native backend on
the CPU device.
"""

from __future__ import annotations

import os

import torch

from .core import GradientOp
from . import native

# backend value -> GEMM engine of libmfhip
NATIVE_BACKENDS = {"hip_native": "mfma"}
BACKENDS = ("auto", *NATIVE_BACKENDS)


def _backend_name(backend):
    if backend not in BACKENDS:
        raise ValueError(f"unknown convolution backend: {backend}")
    return backend


def _resolve_backend(backend, *arrays):
    """``auto`` -> ``hip_native``; every array must be a GPU tensor on the current device
    (ops/convolution.py:20-30)."""
    actual = "hip_native" if backend == "auto" else backend
    for value in arrays:
        if value is None:
            continue
        if not isinstance(value, torch.Tensor):
            raise TypeError("operator arrays must be torch tensors")
        if value.device.type != "cuda":
            raise ValueError(f"backend={actual} is incompatible with device=cpu")
        if value.device.index != torch.cuda.current_device():
            raise ValueError("operator arrays must be on the current GPU")
    return actual


def _normalize_pair(value, name, allow_zero=False):
    if isinstance(value, int):
        pair = (value, value)
    elif isinstance(value, (tuple, list)) and len(value) == 2:
        pair = (int(value[0]), int(value[1]))
    else:
        raise TypeError(f"{name} must be an int or a pair of ints, got {value!r}")
    minimum = 0 if allow_zero else 1
    if pair[0] < minimum or pair[1] < minimum:
        relation = "non-negative" if allow_zero else "positive"
        raise ValueError(f"{name} must be {relation}, got {value!r}")
    return pair


class Conv2D_Op(GradientOp):
    def _fused_activation(self):
        return None

    def _activation_alpha(self):
        return 0.0

    def __init__(self, x, kernel, stride=1, padding=0, groups=1, dilation=1, bias=None, backend="auto",
                 recompute_im2col=None):
        if bias is None:
            super().__init__(x, kernel)
        else:
            super().__init__(x, kernel, bias)
        self.backend = _backend_name(backend)
        if int(groups) != 1 or _normalize_pair(dilation, "dilation") != (1, 1):
            raise ValueError(f"{backend} supports only groups=1 and dilation=1")
        self.bias = bias
        self.stride = _normalize_pair(stride, "stride")
        self.padding = _normalize_pair(padding, "padding", allow_zero=True)
        self.groups = 1
        self.dilation = (1, 1)
        self.recompute_im2col = (os.environ.get("MYFLOWS_RECOMPUTE_IM2COL") == "1"
                                 if recompute_im2col is None else bool(recompute_im2col))
        self._activation_fused = False

    def forward(self, x_val, kernel_val, bias_val=None):
        self.actual_backend = _resolve_backend(self.backend, x_val, kernel_val, bias_val)
        if self.bias is not None and bias_val is None:
            raise ValueError("bias value is missing")
        activation = self._fused_activation()
        self.value, cols = native.conv2d_forward(
            x_val, kernel_val, bias_val, stride=self.stride, padding=self.padding, activation=activation,
            alpha=self._activation_alpha(), engine=NATIVE_BACKENDS[self.actual_backend])
        self._activation_fused = activation is not None
        self._cols = cols if self.parents[1].requires_grad and not self.recompute_im2col else None
        self._inputs = (x_val, kernel_val) if self.requires_grad else None

    def backward(self):
        if not hasattr(self, "actual_backend"):
            raise RuntimeError("forward must run before backward")
        _resolve_backend(self.actual_backend, self.grad, *(p.value for p in self.parents))
        x_node, kernel_node = self.parents[:2]
        need_x, need_w = x_node.requires_grad, kernel_node.requires_grad
        need_b = self.bias is not None and self.bias.requires_grad
        if not (need_x or need_w or need_b):
            return
        grads = native.conv2d_backward(
            *self._inputs, self.grad, self._cols, stride=self.stride, padding=self.padding, need_bias_grad=need_b,
            need_weight_grad=need_w, need_input_grad=need_x,
            activation=self._fused_activation() if self._activation_fused else None,
            alpha=self._activation_alpha(), output=self.value, engine=NATIVE_BACKENDS[self.actual_backend],
            recompute_cols=self.recompute_im2col)
        for parent, grad in zip(self.parents, grads):
            if grad is not None:
                parent.accumulate_grad(grad, owned=True)


class Conv2D_ReLU_Op(Conv2D_Op):
    """Conv2D(+bias) followed by ReLU, applied in the convolution's epilogue and gated in the
    transposed-gradient kernel of the backward pass."""

    def _fused_activation(self):
        return "relu"


class Conv2D_LeakyReLU_Op(Conv2D_Op):
    """Conv2D(+bias) followed by LeakyReLU. Only alpha > 0 is fused (then y > 0 exactly where the
    pre-activation is > 0, so the output alone gates the backward pass)."""

    def __init__(self, *args, alpha=0.01, **kwargs):
        super().__init__(*args, **kwargs)
        self.alpha = float(alpha)

    def _fused_activation(self):
        return "leaky_relu" if self.alpha > 0 else None

    def _activation_alpha(self):
        return self.alpha

    def forward(self, x_val, kernel_val, bias_val=None):
        super().forward(x_val, kernel_val, bias_val=bias_val)
        if self._activation_fused:
            return
        mask = self.value > 0
        self.value = torch.where(mask, self.value, self.alpha * self.value)
        self._leaky_mask = mask if self.requires_grad else None

    def backward(self):
        if not self._activation_fused:
            self.grad = torch.where(self._leaky_mask, self.grad, self.alpha * self.grad)
        super().backward()


class MaxPool2d_Op(GradientOp):
    """Max pooling; ``padding`` pads with -inf (as torch.nn.MaxPool2d), after which the native path
    is the unpadded one and the input gradient is cropped back."""

    def __init__(self, x, kernel_size=2, stride=2, backend="auto", padding=0):
        super().__init__(x)
        self.backend = _backend_name(backend)
        self.kernel_size = _normalize_pair(kernel_size, "kernel_size")
        self.stride = _normalize_pair(stride, "stride")
        self.padding = _normalize_pair(padding, "padding", allow_zero=True)

    def forward(self, x_val):
        self.actual_backend = _resolve_backend(self.backend, x_val)
        ph, pw = self.padding
        if ph or pw:
            x_val = torch.nn.functional.pad(x_val, (pw, pw, ph, ph), value=float("-inf"))
        self.value, context = native.maxpool2d_forward(x_val, kernel_size=self.kernel_size, stride=self.stride)
        self._context = context if self.requires_grad else None

    def backward(self):
        if not hasattr(self, "actual_backend"):
            raise RuntimeError("forward must run before backward")
        _resolve_backend(self.actual_backend, self.grad, self.parents[0].value)
        dx = native.maxpool2d_backward(self.grad, self._context)
        self.parents[0].accumulate_grad(self._unpad(dx), owned=True)

    def _unpad(self, grad):
        ph, pw = self.padding
        if not (ph or pw):
            return grad
        return grad[:, :, ph:grad.shape[2] - ph, pw:grad.shape[3] - pw]


class Flatten_Op(GradientOp):
    def forward(self, x):
        self.in_shape = x.shape
        self.value = x.reshape(x.shape[0], -1)

    def backward(self):
        self.parents[0].accumulate_grad(self.grad.reshape(self.in_shape))
