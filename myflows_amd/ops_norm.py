"""BatchNorm2d, the fused BatchNorm(+Add)+ReLU execution unit and GlobalAvgPool2d.

Operator API of the reference's ``ops/batchnorm.py``: ``BatchNorm2d_Op`` (:7-60),
``BatchNormActivation`` (:63-107) and ``GlobalAvgPool2d_Op`` (:110-123). The arithmetic is that of
``fused.batchnorm2d_forward`` / ``batchnorm2d_backward`` (libmfhip): FP64 statistics, the mean kept
as a float hi + lo pair, x_hat recomputed from x in the backward instead of being stored.
``BatchNormReLUPool`` (BN, ReLU and an unpadded max-pool as one unit) has no counterpart in the
reference; it gives the separate nodes' bits.
"""

from __future__ import annotations

import torch

from . import fused, native
from .fused import on_libmfhip as _on_libmfhip
from .graph import GradientOp
from .ops_conv import _resolve_backend


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

    def forms_input_grad(self):
        """Whether the next backward can form its dy from a convolution's split-K dX slices (a
        training pass that sums over the channels)."""
        return self._stats is not None and self._training_used

    def backward(self):
        x_node, gamma_node, beta_node = self.parents
        buffers = [node.grad_buffer() if node.requires_grad else (None, False) for node in self.parents]
        fused.batchnorm2d_backward(
            x_node.value, self.grad, gamma_node.value, *self._stats, training=self._training_used,
            x_grad=buffers[0][0], gamma_grad=buffers[1][0], beta_grad=buffers[2][0],
            accumulate=tuple(add for _, add in buffers))


class BatchNormActivation:
    """The chain BN -> [Add(BN, residual)] -> ReLU of a Graph run as one execution unit.

    Contract with the executor (``graph.Graph``): the unit takes the place of the chain's last node,
    ``output`` (the ReLU), in the forward and backward orders; the executor skips the chain's other
    nodes (``hidden``), hands ``forward`` the values of ``parents`` (x, gamma, beta and, with an Add,
    the residual) and calls ``backward`` once ``output.grad`` is set. Afterwards ``output`` and the
    parents hold what the separate nodes would have given them.

    Route of a pass, chosen per forward:
      * fused: one libmfhip pass for BN, the residual add and the ReLU (the hidden nodes' values are
        never formed and are left empty), and one backward pass that gates dy by the output and
        writes the residual's gradient beside the BN gradients;
      * chained: a residual that the Add would broadcast or promote (another shape or dtype) runs
        the chain's own nodes one after the other, forward and backward.
    """

    def __init__(self, bn, add, output, residual):
        self.bn, self.add, self.output, self.residual = bn, add, output, residual
        self.chain = (bn, output) if add is None else (bn, add, output)
        self.hidden = self.chain[:-1]
        self.parents = list(bn.parents) + ([] if residual is None else [residual])
        self.name = "BatchNormReLU" if add is None else "BatchNormAddReLU"
        self.chained = False  # the route of the last forward
        self._stats = None    # (mean, inv_std, training) of the last fused forward, when BN needs gradients

    @staticmethod
    def _fusable(x, residual):
        return residual is None or (tuple(residual.shape) == tuple(x.shape) and residual.dtype == x.dtype)

    def forward(self, x, gamma, beta, residual=None):
        if tuple(gamma.shape) != (x.shape[1],) or tuple(beta.shape) != tuple(gamma.shape):
            raise ValueError("gamma/beta shape must be (C,)")
        self.chained = not self._fusable(x, residual)
        if self.chained:
            for node in self.chain:
                node.forward(*(parent.value for parent in node.parents))
            return
        bn = self.bn
        y, mean, inv_std = fused.batchnorm2d_forward(
            x, gamma, beta, bn.running_mean, bn.running_var, momentum=bn.momentum, eps=bn.eps, training=bn.training,
            unbiased_running_var=bn.unbiased_running_var, relu=True, residual=residual)
        self.output.value = y
        for node in self.hidden:
            node.value = None
        self._stats = (mean, inv_std, bn.training) if bn.requires_grad else None

    def forms_input_grad(self):
        """Whether the next backward can form its dy from a convolution's split-K dX slices: the
        fused route of a training pass whose batch norm needs gradients."""
        return not self.chained and self._stats is not None and self._stats[2]

    def backward(self):
        if self.chained:
            for node in reversed(self.chain):
                if node.requires_grad and node.grad is not None:
                    node.backward()
            for node in self.hidden:
                node.grad = None
            return
        dy, gate = self.output.grad, self.output.value
        wants_residual = self.residual is not None and self.residual.requires_grad
        if self._stats is None:
            # BN needs no gradient: the residual's is dy where the ReLU passed its input.
            if wants_residual:
                self.residual.accumulate_grad(torch.where(gate > 0, dy, torch.zeros_like(dy)), owned=True)
            return
        mean, inv_std, training = self._stats
        x_node, gamma_node, beta_node = self.bn.parents
        target = {role: node.grad_buffer() if node.requires_grad else (None, False)
                  for role, node in zip(("x", "gamma", "beta"), (x_node, gamma_node, beta_node))}
        residual_grad, add_residual = self.residual.grad_buffer() if wants_residual else (None, False)
        fused.batchnorm2d_backward(
            x_node.value, dy, gamma_node.value, mean, inv_std, training=training, x_grad=target["x"][0],
            gamma_grad=target["gamma"][0], beta_grad=target["beta"][0],
            accumulate=(target["x"][1], target["gamma"][1], target["beta"][1]), gate=gate,
            residual_grad=residual_grad, add_residual=add_residual)


class BatchNormReLUPool:
    """The chain BN -> ReLU -> MaxPool2d of a Graph (a network stem) run as one execution unit.

    Contract with the executor (``graph.Graph``), as ``BatchNormActivation``'s: the unit takes the
    place of the chain's last node, ``output`` (the max-pool), the executor skips ``hidden`` (the BN
    and the ReLU), hands ``forward`` the values of ``parents`` (x, gamma, beta) and calls
    ``backward`` once ``output.grad`` is set.

    Route of a pass, chosen per forward:
      * fused: libmfhip's BN + ReLU + max-pool launches. The ReLU output is never formed (the
        hidden nodes' values stay empty): the forward pools the normalised planes in LDS, and the
        backward takes the pooled gradient to x, gamma and beta, recomputing the ReLU gate from x.
        Bit for bit the separate nodes' results;
      * chained: the chain's own nodes one after the other, for a padded max-pool or a shape the
        fused kernels do not take.
    """

    def __init__(self, bn, relu, pool):
        self.bn, self.relu, self.output = bn, relu, pool
        self.chain = (bn, relu, pool)
        self.hidden = (bn, relu)
        self.parents = list(bn.parents)
        self.name = "BatchNormReLUPool"
        self.chained = False  # the route of the last forward
        self._saved = None    # (argmax, mean, inv_std, training) of the last fused forward, when BN needs gradients

    def _fusable(self, x):
        pool = self.output
        return (isinstance(x, torch.Tensor) and x.ndim == 4 and _on_libmfhip(x) and pool.padding == (0, 0)
                and fused.batchnorm_relu_pool_supported(x.shape, pool.kernel_size, pool.stride))

    def forward(self, x, gamma, beta):
        if tuple(gamma.shape) != (x.shape[1],) or tuple(beta.shape) != tuple(gamma.shape):
            raise ValueError("gamma/beta shape must be (C,)")
        self.chained = not self._fusable(x)
        if self.chained:
            for node in self.chain:
                node.forward(*(parent.value for parent in node.parents))
            return
        bn, pool = self.bn, self.output
        pool.actual_backend = _resolve_backend(pool.backend, x)
        pooled, argmax, mean, inv_std = fused.batchnorm2d_relu_pool_forward(
            x, gamma, beta, bn.running_mean, bn.running_var, momentum=bn.momentum, eps=bn.eps, training=bn.training,
            kernel_size=pool.kernel_size, stride=pool.stride, unbiased_running_var=bn.unbiased_running_var)
        pool.value = pooled
        # The max-pool node keeps the forward state it would have had (its window choices).
        pool._context = native.NativePoolContext(tuple(x.shape), tuple(pooled.shape), pool.kernel_size, pool.stride,
                                                 argmax, x.device.index) if pool.requires_grad else None
        for node in self.hidden:
            node.value = None
        self._saved = (argmax, mean, inv_std, bn.training) if bn.requires_grad else None

    def backward(self):
        if self.chained:
            for node in reversed(self.chain):
                if node.requires_grad and node.grad is not None:
                    node.backward()
            for node in self.hidden:
                node.grad = None
            return
        if self._saved is None:
            return
        argmax, mean, inv_std, training = self._saved
        pool = self.output
        x_node, gamma_node, beta_node = self.bn.parents
        target = [node.grad_buffer() if node.requires_grad else (None, False)
                  for node in (x_node, gamma_node, beta_node)]
        fused.batchnorm2d_relu_pool_backward(
            x_node.value, pool.grad, argmax, gamma_node.value, beta_node.value, mean, inv_std, training=training,
            kernel_size=pool.kernel_size, stride=pool.stride, x_grad=target[0][0], gamma_grad=target[1][0],
            beta_grad=target[2][0], accumulate=tuple(add for _, add in target))


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
