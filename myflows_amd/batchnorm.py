"""BatchNorm2d and GlobalAvgPool2d operators.

Restates ``ops/batchnorm.py:7-123`` and the arithmetic of ``ops/fused.py:250-387``: statistics in
FP64, the mean split into float32 hi + lo parts, inv_std = 1 / sqrt(var + eps) rounded once,
y = (((x - hi) - lo) * inv_std) * gamma + beta in float32, running statistics updated with
momentum; backward with FP64 channel sums. These are torch device operations (the model's
non-GEMM glue), not part of libmfhip.
"""

from __future__ import annotations

import torch

from .core import GradientOp


def _channel(a):
    return a.reshape(1, -1, 1, 1)


def batchnorm2d_forward(x, gamma, beta, running_mean, running_var, *, momentum, eps, training,
                        unbiased_running_var=False, relu=False, residual=None):
    n, c, h, w = x.shape
    count = n * h * w
    var_scale = count / (count - 1) if unbiased_running_var and count > 1 else 1.0
    if training:
        x64 = x.double()
        mean64 = x64.mean(dim=(0, 2, 3))
        centered = x64 - _channel(mean64)
        var64 = (centered * centered).mean(dim=(0, 2, 3))
        del x64, centered
        running_mean.copy_((1.0 - momentum) * running_mean.double() + momentum * mean64)
        running_var.copy_((1.0 - momentum) * running_var.double() + momentum * var64 * var_scale)
    else:
        mean64, var64 = running_mean.double(), running_var.double()
    hi = mean64.to(x.dtype)
    mean = torch.stack([hi, (mean64 - hi.double()).to(x.dtype)])
    inv_std = (1.0 / torch.sqrt(var64 + eps)).to(x.dtype)
    y = (((x - _channel(mean[0])) - _channel(mean[1])) * _channel(inv_std)) * _channel(gamma) + _channel(beta)
    if residual is not None:
        y = y + residual
    if relu:
        y = torch.clamp_min(y, 0)
    return y, mean, inv_std


def _store(out, value, add):
    if add:
        out += value
    else:
        out.copy_(value)


def batchnorm2d_backward(x, dy, gamma, mean, inv_std, *, training, x_grad, gamma_grad, beta_grad,
                         accumulate=(True, True, True)):
    if x_grad is None and gamma_grad is None and beta_grad is None:
        return
    n, c, h, w = x.shape
    count = n * h * w
    istd = inv_std.double()
    dy64 = dy.double()
    sdy = dy64.sum(dim=(0, 2, 3))
    if beta_grad is not None:
        _store(beta_grad, sdy.to(beta_grad.dtype), accumulate[2])
    centered = x.double() - _channel(mean[0].double() + mean[1].double())
    dgamma = istd * (dy64 * centered).sum(dim=(0, 2, 3))
    del centered, dy64
    if gamma_grad is not None:
        _store(gamma_grad, dgamma.to(gamma_grad.dtype), accumulate[1])
    if x_grad is None:
        return
    a = _channel((gamma.double() * istd).to(x.dtype))
    if training:
        k1 = _channel((sdy / count).to(x.dtype))
        k2 = _channel((istd * dgamma / count).to(x.dtype))
        dx = a * (dy - k1 - ((x - _channel(mean[0])) - _channel(mean[1])) * k2)
    else:
        dx = a * dy
    _store(x_grad, dx, accumulate[0])


class BatchNorm2d_Op(GradientOp):
    def __init__(self, x, gamma, beta, running_mean, running_var, momentum=0.1, eps=1e-5, training=True,
                 unbiased_running_var=False):
        super().__init__(x, gamma, beta)
        self.unbiased_running_var = bool(unbiased_running_var)
        self.running_mean = running_mean
        self.running_var = running_var
        self.momentum = float(momentum)
        self.eps = float(eps)
        self.training = bool(training)

    def forward(self, x_val, gamma_val, beta_val):
        c = x_val.shape[1]
        if tuple(gamma_val.shape) != (c,) or tuple(beta_val.shape) != (c,):
            raise ValueError("gamma/beta shape must be (C,)")
        self._training_used = self.training
        self.value, self._mean, self._inv_std = batchnorm2d_forward(
            x_val, gamma_val, beta_val, self.running_mean, self.running_var, momentum=self.momentum, eps=self.eps,
            training=self.training, unbiased_running_var=self.unbiased_running_var)
        if not self.requires_grad:
            self._mean = self._inv_std = None

    def backward(self):
        x_node, gamma_node, beta_node = self.parents
        outputs = [node.grad_buffer() if node.requires_grad else (None, False) for node in self.parents]
        batchnorm2d_backward(x_node.value, self.grad, gamma_node.value, self._mean, self._inv_std,
                             training=self._training_used, x_grad=outputs[0][0], gamma_grad=outputs[1][0],
                             beta_grad=outputs[2][0], accumulate=tuple(add for _, add in outputs))


class GlobalAvgPool2d_Op(GradientOp):
    """(N, C, H, W) -> (N, C), mean accumulated in FP64 and rounded once."""

    def forward(self, x_val):
        self._in_shape = tuple(x_val.shape)
        self.value = x_val.mean(dim=(2, 3), dtype=torch.float64).to(x_val.dtype)

    def backward(self):
        n, c, h, w = self._in_shape
        self.parents[0].accumulate_grad(self.grad.reshape(n, c, 1, 1) / (h * w))
