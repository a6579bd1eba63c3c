"""BatchNorm2d, the fused BatchNorm(+Add)+ReLU execution unit and GlobalAvgPool2d.

Operator API of the reference's ``ops/batchnorm.py``: ``BatchNorm2d_Op`` (:7-60),
``BatchNormActivation`` (:63-107) and ``GlobalAvgPool2d_Op`` (:110-123). The arithmetic is that of
``fused.batchnorm2d_forward`` / ``batchnorm2d_backward`` (libmfhip): FP64 statistics, the mean kept
as a float hi + lo pair, x_hat recomputed from x in the backward instead of being stored.
"""

from __future__ import annotations

import torch

from . import fused
from .fused import on_libmfhip as _on_libmfhip
from .graph import GradientOp


class BatchNorm2d_Op(GradientOp):
    """Batch norm of x (N, C, H, W) with parameters gamma, beta (C,) and external running statistics.

    training=True normalises with the batch statistics and updates the running ones with momentum;
    training=False uses the running statistics. The mode of the forward is the one its backward uses.
    """

    def __init__(self, x, gamma, beta, running_mean, running_var, momentum=0.1, eps=1e-5, training=True,
                 unbiased_running_var=False):
        super().__init__(x, gamma, beta)
        self.running_mean, self.running_var = running_mean, running_var
        self.momentum, self.eps = float(momentum), float(eps)
        self.training = bool(training)
        self.unbiased_running_var = bool(unbiased_running_var)
        self._stats = None

    def forward(self, x_val, gamma_val, beta_val):
        c = x_val.shape[1]
        if tuple(gamma_val.shape) != (c,) or tuple(beta_val.shape) != (c,):
            raise ValueError("gamma/beta shape must be (C,)")
        self._training_used = self.training
        self.value, mean, inv_std = fused.batchnorm2d_forward(
            x_val, gamma_val, beta_val, self.running_mean, self.running_var, momentum=self.momentum, eps=self.eps,
            training=self.training, unbiased_running_var=self.unbiased_running_var)
        self._stats = (mean, inv_std) if self.requires_grad else None

    def backward(self):
        x_node, gamma_node, beta_node = self.parents
        buffers = [node.grad_buffer() if node.requires_grad else (None, False) for node in self.parents]
        fused.batchnorm2d_backward(
            x_node.value, self.grad, gamma_node.value, *self._stats, training=self._training_used,
            x_grad=buffers[0][0], gamma_grad=buffers[1][0], beta_grad=buffers[2][0],
            accumulate=tuple(add for _, add in buffers))


class BatchNormActivation:
    """One execution unit for ReLU(BN(x) [+ residual]) that keeps the logical BN / Add / ReLU nodes
    addressable: the forward writes only the ReLU node's value, the backward gates by it and hands
    the gated gradient to the residual branch. A residual that needs broadcasting runs unfused."""

    def __init__(self, bn, add, output, residual):
        self.bn, self.add, self.output, self.residual = bn, add, output, residual
        self.hidden = (bn,) if add is None else (bn, add)
        self.parents = list(bn.parents) + ([residual] if residual is not None else [])
        self.name = "BatchNormReLU" if add is None else "BatchNormAddReLU"
        self._unfused = False

    def forward(self, x, gamma, beta, residual=None):
        bn = self.bn
        if tuple(gamma.shape) != (x.shape[1],) or beta.shape != gamma.shape:
            raise ValueError("gamma/beta shape must be (C,)")
        self._unfused = residual is not None and (residual.shape != x.shape or residual.dtype != x.dtype)
        if self._unfused:
            bn.forward(x, gamma, beta)
            self.add.forward(*(p.value for p in self.add.parents))
            self.output.forward(self.add.value)
            return
        self.training = bn.training
        self.output.value, mean, inv_std = fused.batchnorm2d_forward(
            x, gamma, beta, bn.running_mean, bn.running_var, momentum=bn.momentum, eps=bn.eps,
            training=self.training, unbiased_running_var=bn.unbiased_running_var, relu=True, residual=residual)
        for node in self.hidden:
            node.value = None
        self._stats = (mean, inv_std) if bn.requires_grad else None

    def backward(self):
        bn = self.bn
        if self._unfused:
            self.output.backward()
            self.add.backward()
            if bn.requires_grad:
                bn.backward()
            for node in self.hidden:
                node.grad = None
            return
        buffers = [p.grad_buffer() if p.requires_grad else (None, False) for p in self.parents]
        residual_grad, add_residual = buffers[3] if self.residual is not None else (None, False)
        if self._stats is None:  # only the residual branch needs a gradient
            if residual_grad is not None:
                gated = torch.where(self.output.value > 0, self.output.grad, torch.zeros_like(self.output.grad))
                residual_grad.add_(gated) if add_residual else residual_grad.copy_(gated)
            return
        fused.batchnorm2d_backward(
            bn.parents[0].value, self.output.grad, bn.parents[1].value, *self._stats, training=self.training,
            x_grad=buffers[0][0], gamma_grad=buffers[1][0], beta_grad=buffers[2][0],
            accumulate=tuple(add for _, add in buffers[:3]), gate=self.output.value, residual_grad=residual_grad,
            add_residual=add_residual)


class GlobalAvgPool2d_Op(GradientOp):
    """(N, C, H, W) -> (N, C): FP64 mean over H, W rounded once to the input dtype."""

    def forward(self, x_val):
        self._in_shape = tuple(x_val.shape)
        if _on_libmfhip(x_val):
            self.value = fused.global_avg_pool_forward(x_val)
        else:
            self.value = x_val.mean(dim=(2, 3), dtype=torch.float64).to(x_val.dtype)

    def backward(self):
        n, c, h, w = self._in_shape
        x = self.parents[0]
        if _on_libmfhip(x.value):
            buffer, add = x.grad_buffer()
            fused.global_avg_pool_backward(self.grad, self._in_shape, buffer, add)
        else:
            x.accumulate_grad(self.grad.reshape(n, c, 1, 1) / (h * w))
