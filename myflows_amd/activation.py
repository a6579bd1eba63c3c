"""ReLU and MSELoss, restating ``ops/activation.py:43-52``, ``ops/fused.py:50-62`` and
``ops/loss.py:94-113`` of the reference."""

from __future__ import annotations

import torch

from .core import GradientOp


class ReLU(GradientOp):
    def forward(self, x):
        self.value = torch.clamp_min(x, 0)  # max(0, x); NaN stays NaN

    def backward(self):
        x_node = self.parents[0]
        gated = torch.where(x_node.value > 0, self.grad, torch.zeros((), dtype=self.grad.dtype, device=self.grad.device))
        if x_node.grad is None:
            x_node.grad = gated
        else:
            x_node.grad += gated


class MSELoss(GradientOp):
    """Mean squared error; the loss stays on the device (FP64 mean rounded to the prediction dtype)."""

    def __init__(self, y_pred, y_true, name="MSELoss"):
        super().__init__(y_pred, y_true, name=name)

    def forward(self, y_pred_val, y_true_val):
        diff = y_pred_val - y_true_val
        self.value = torch.mean(diff * diff, dtype=torch.float64).to(diff.dtype)

    def backward(self):
        y_pred, y_true = self.parents
        if not y_pred.requires_grad:
            return
        n = max(y_pred.value.numel(), 1)
        g = 2.0 * (y_pred.value - y_true.value) / n
        y_pred.accumulate_grad(self.grad * g, owned=True)
