"""Add, the fused Linear operator (y = x W + b), ReLU / LeakyReLU, MSELoss, the input channel
normalisation and dropout.

Operator API of the reference's ``ops/basic.py`` (``Add`` :5-35, ``Linear`` :76-164),
``ops/activation.py`` (``ReLU`` :43-52, ``LeakyReLU`` :67-80), ``ops/loss.py`` (``MSELoss``
:94-113), ``ops/pooling.py`` (``ChannelNormalize_Op`` :65-87) and ``ops/dropout.py``
(``Dropout_Op`` :12-40); the last two are device tensor arithmetic, off the kernel path.

* ``Linear`` on ``hip_native`` runs its three GEMMs on the MFMA engine: the forward with the bias
  in the epilogue, dX = g W^T and dW = x^T g reading the transposed operands in place;
  ``hip_native_kahan`` / ``hip_native_dot2`` use the compensated teaching kernels instead. db is an
  FP64 sum rounded once; an input with requires_grad=False skips the dX GEMM.
* ``ReLU`` / ``LeakyReLU`` run on libmfhip (forward, and a backward that gates and accumulates in
  one pass); they accept GPU tensors only.
* ``Add`` is device tensor arithmetic (torch): broadcast add with the reduction of the broadcast
  axes in backward. ``MSELoss`` (the FP64 mean of squared errors and its gradient) and a 2-D
  Linear's bias gradient run on libmfhip for float32 GPU tensors (torch on host tensors).
"""

from __future__ import annotations

import numpy as np
import torch

from . import fused, native
from .fused import on_libmfhip as _on_libmfhip
from .graph import GradientOp

LINEAR_BACKENDS = ("auto", "hip_native", "hip_native_kahan", "hip_native_dot2", "cuda_native_register",
                   "cuda_native_kahan", "cuda_native_dot2")
_LINEAR_KERNEL = {"auto": "mfma", "hip_native": "mfma", "cuda_native_register": "mfma", "hip_native_kahan": "kahan",
                  "cuda_native_kahan": "kahan", "hip_native_dot2": "dot2", "cuda_native_dot2": "dot2"}


def _linear_backend(backend):
    if backend not in LINEAR_BACKENDS:
        raise ValueError(f"backend must be one of {', '.join(LINEAR_BACKENDS)}")
    return backend


def _reduce_to(grad, shape):
    """Sum grad over the axes broadcast to reach it from ``shape``, in FP64, rounded once."""
    lead = grad.ndim - len(shape)
    axes = list(range(lead)) + [lead + i for i, (g, s) in enumerate(zip(grad.shape[lead:], shape)) if s == 1 and g != 1]
    if not axes:
        return grad.reshape(shape)
    return grad.sum(dim=axes, dtype=torch.float64).reshape(shape).to(grad.dtype)


def _sum_to(grad, shape):
    """Sum grad over the axes broadcast to reach it from ``shape`` (in grad's dtype)."""
    lead = grad.ndim - len(shape)
    if lead:
        grad = grad.sum(dim=tuple(range(lead)))
    axes = tuple(i for i, (g, s) in enumerate(zip(grad.shape, shape)) if s == 1 and g != 1)
    if axes:
        grad = grad.sum(dim=axes, keepdim=True)
    return grad.reshape(shape)


class Add(GradientOp):
    """a + b with broadcasting; a 1-D b added to a 4-D a is a per-channel (axis 1) bias."""

    def forward(self, a, b):
        self.a_shape, self.b_shape = tuple(a.shape), tuple(b.shape)
        if a.ndim == 4 and b.ndim == 1:
            b = b.reshape(1, -1, 1, 1)
            self._b_view = tuple(b.shape)
        else:
            self._b_view = self.b_shape
        self.value = a + b

    def backward(self):
        a, b = self.parents
        if a.requires_grad:
            a.accumulate_grad(_sum_to(self.grad, self.a_shape))
        if b.requires_grad:
            b.accumulate_grad(_sum_to(self.grad, self._b_view).reshape(self.b_shape))


class Linear(GradientOp):
    """y = x @ W + b for 2-D x."""

    def __init__(self, x, w, b, name=None, backend="auto"):
        super().__init__(x, w, b, name=name)
        self.backend = _linear_backend(backend)

    def _kernel(self):
        from .ops_conv import _resolve_backend
        _resolve_backend("hip_native", *(p.value for p in self.parents))
        return _LINEAR_KERNEL[self.backend]

    def _product(self, a, b, trans_a=False, trans_b=False):
        kernel = self._kernel()
        if kernel == "mfma":
            return native.gemm(a, b, trans_a=trans_a, trans_b=trans_b)
        return native.matmul((a.t() if trans_a else a).contiguous(), (b.t() if trans_b else b).contiguous(),
                             variant="register", accumulate=kernel)

    def forward(self, x, w, b):
        self.x_shape, self.w_shape, self.b_shape = tuple(x.shape), tuple(w.shape), tuple(b.shape)
        kernel = self._kernel()
        if x.ndim != 2:
            raise ValueError("Linear on hip_native expects a 2-D input")
        fused_bias = b.reshape(-1) if b.numel() == w.shape[1] else None
        if kernel == "mfma":
            out = native.gemm(x, w, fused_bias)
        else:
            out = native.matmul(x, w, fused_bias, variant="register", accumulate=kernel)
        self.value = out if fused_bias is not None else out + b

    def backward(self):
        x, w, b = self.parents
        g = self.grad
        if x.requires_grad:
            x.accumulate_grad(self._product(g, w.value, trans_b=True), owned=True)
        if w.requires_grad:
            w.accumulate_grad(self._product(x.value, g, trans_a=True), owned=True)
        if b.requires_grad:
            if _on_libmfhip(g) and g.ndim == 2 and b.value.numel() == g.shape[1]:
                b.accumulate_grad(fused.column_sums(g).reshape(b.value.shape), owned=True)
            else:
                b.accumulate_grad(_reduce_to(g, tuple(b.value.shape)))


def _gpu_only(value, op):
    if not (isinstance(value, torch.Tensor) and value.is_cuda):
        raise ValueError(f"{op} runs on libmfhip and needs a GPU tensor (device=cpu is not supported)")


class ReLU(GradientOp):
    """max(0, x); the backward adds grad where x > 0 into the parent's gradient in one pass."""

    def forward(self, x):
        _gpu_only(x, "ReLU")
        self.value = fused.relu_forward(x)

    def backward(self):
        x_node = self.parents[0]
        x_node.grad = fused.relu_backward_accumulate(x_node.value, self.grad, x_node.grad)


class LeakyReLU(GradientOp):
    """x if x > 0 else alpha * x."""

    def __init__(self, x, alpha=0.01, name=None):
        self.alpha = alpha
        super().__init__(x, name=name)

    def forward(self, x):
        _gpu_only(x, "LeakyReLU")
        self.value = torch.where(x > 0, x, self.alpha * x)

    def backward(self):
        x_node = self.parents[0]
        x_node.grad = fused.leaky_relu_backward_accumulate(x_node.value, self.grad, x_node.grad, self.alpha)


class MSELoss(GradientOp):
    """Mean squared error. The loss stays on the device: FP64 mean, rounded to the prediction dtype."""

    def __init__(self, y_pred, y_true, name="MSELoss"):
        super().__init__(y_pred, y_true, name=name)

    def forward(self, y_pred_val, y_true_val):
        if _on_libmfhip(y_pred_val) and _on_libmfhip(y_true_val) and y_pred_val.shape == y_true_val.shape:
            self.value = fused.mse_loss_forward(y_pred_val, y_true_val)
            return
        diff = y_pred_val - y_true_val
        self.value = torch.mean(diff * diff, dtype=torch.float64).to(diff.dtype)

    def backward(self):
        y_pred, y_true = self.parents
        if not y_pred.requires_grad:
            return
        if (_on_libmfhip(y_pred.value) and _on_libmfhip(y_true.value) and _on_libmfhip(self.grad)
                and y_pred.value.shape == y_true.value.shape and self.grad.numel() == 1):
            buffer, add = y_pred.grad_buffer()
            fused.mse_loss_backward(y_pred.value, y_true.value, self.grad, buffer, add)
            return
        count = max(y_pred.value.numel(), 1)
        y_pred.accumulate_grad(self.grad * (2.0 * (y_pred.value - y_true.value) / count), owned=True)


# ImageNet channel statistics of [0, 1] RGB inputs (torchvision's pretrained-weight convention).
IMAGENET_MEAN = (0.485, 0.456, 0.406)
IMAGENET_STD = (0.229, 0.224, 0.225)


class ChannelNormalize_Op(GradientOp):
    """y = (x - mean[c]) / std[c] over the channels of an NCHW tensor, in x's dtype (device tensor
    arithmetic); the gradient is dy / std[c]. The reference's ``ops/pooling.py:65-87``."""

    def __init__(self, x, mean=IMAGENET_MEAN, std=IMAGENET_STD, name=None):
        super().__init__(x, name=name)
        self.mean = tuple(float(v) for v in mean)
        self.std = tuple(float(v) for v in std)
        if len(self.mean) != len(self.std):
            raise ValueError("mean and std must have one value per channel")
        if any(v <= 0 for v in self.std):
            raise ValueError("std must be positive")

    def _channel(self, values, like):
        return torch.tensor(values, dtype=like.dtype, device=like.device).reshape(1, -1, 1, 1)

    def forward(self, x_val):
        if x_val.ndim != 4 or x_val.shape[1] != len(self.mean):
            raise ValueError(f"expected an NCHW tensor of {len(self.mean)} channels, got shape {tuple(x_val.shape)}")
        self.value = (x_val - self._channel(self.mean, x_val)) / self._channel(self.std, x_val)

    def backward(self):
        x_node = self.parents[0]
        if not getattr(x_node, "requires_grad", True):
            return
        x_node.accumulate_grad(self.grad / self._channel(self.std, self.grad), owned=True)


class Dropout_Op(GradientOp):
    """Inverted dropout: in training, y = x * mask with mask = (u < 1 - p) / (1 - p) in x's dtype,
    u uniform on [0, 1) drawn per element by NumPy's generator from ``seed`` (the reference's masks
    for a seed), or by torch's on x's device without one; identity when not training or p = 0.
    The reference's ``ops/dropout.py:12-40``."""

    def __init__(self, x, p=0.5, training=True, seed=None, name=None):
        self.p = float(p)
        if self.p < 0.0 or self.p >= 1.0:
            raise ValueError("dropout p must be in [0, 1)")
        self.training = bool(training)
        self.seed = seed
        self._rng = np.random.default_rng(int(seed)) if seed is not None else None
        self._mask = None
        super().__init__(x, name=name)

    def _uniform(self, like):
        if self._rng is not None:
            return torch.as_tensor(self._rng.random(tuple(like.shape)), device=like.device)
        return torch.rand(like.shape, dtype=torch.float64, device=like.device)

    def forward(self, x):
        if not self.training or self.p == 0.0:
            self._mask = torch.ones_like(x) if self.requires_grad else None
            self.value = x
            return
        keep = 1.0 - self.p
        self._mask = (self._uniform(x) < keep).to(x.dtype) / keep
        self.value = x * self._mask
        if not self.requires_grad:
            self._mask = None

    def backward(self):
        self.parents[0].accumulate_grad(self.grad * self._mask, owned=True)
