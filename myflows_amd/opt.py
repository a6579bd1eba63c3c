"""Optimizer base and Adam, restating ``train/opt.py:11-281`` of the reference.

``one_step()`` runs forward and backward and accumulates the trainable gradients;
``update()`` applies the step and clears the accumulators. Adam keeps zero-initialised moments and
rounds every operation to float32 in the order of ``ops/fused.py:494-533``
(m = b1 m + (1 - b1) g; v = b2 v + (1 - b2) g^2; p -= (lr (m / bc1)) / (sqrt(v / bc2) + eps)).
"""

from __future__ import annotations

import torch

from .core import Variable


class Optimizer:
    def __init__(self, graph, learning_rate):
        self.graph = graph
        self.learning_rate = learning_rate
        self.acc_gradient = {}
        self.acc_no = 0

    def one_step(self):
        self.forward_backward()
        self.acc_no += 1

    def get_gradient(self, node):
        if node not in self.acc_gradient:
            return None
        if self.acc_no in (0, 1):
            return self.acc_gradient[node]
        return self.acc_gradient[node] / self.acc_no

    def _update(self):
        raise NotImplementedError

    def update(self, var_gradients=None):
        if var_gradients is not None:
            for node, gradient in var_gradients.items():
                self.acc_gradient[node] = gradient
        self._update()
        self.acc_gradient.clear()
        self.acc_no = 0

    def forward_backward(self):
        self.graph.forward()
        self.graph.backward()
        self._accumulate_gradients()

    def _accumulate_gradients(self):
        for node in self.graph.nodes:
            if node.trainable is True and node.grad is not None:
                if node in self.acc_gradient:
                    self.acc_gradient[node] += node.grad
                else:
                    self.acc_gradient[node] = node.grad


class MBGD(Optimizer):
    def __init__(self, graph, learning_rate=0.01):
        super().__init__(graph, learning_rate)

    def _update(self):
        for node in list(self.acc_gradient):
            grad = self.get_gradient(node)
            if getattr(node, "trainable", False) and grad is not None:
                node.value -= self.learning_rate * grad


def adam_update(param, grad, m, v, *, lr, beta1, beta2, eps, step, grad_scale=1.0):
    """One textbook Adam step applied in place, each operation rounded to float32 in the reference's order."""
    bc1, bc2 = 1.0 - beta1 ** step, 1.0 - beta2 ** step
    f32 = lambda value: float(torch.tensor(value, dtype=torch.float32))
    scale, b1, omb1, b2, omb2, bc1, bc2, lr, eps = map(f32, (grad_scale, beta1, 1.0 - beta1, beta2, 1.0 - beta2,
                                                             bc1, bc2, lr, eps))
    gs = grad if scale == 1.0 else grad * scale
    m.mul_(b1)
    m.add_(omb1 * gs)
    v.mul_(b2)
    v.add_(omb2 * (gs * gs))
    denom = torch.sqrt(v / bc2)
    denom += eps
    param.sub_((lr * (m / bc1)) / denom)


class Adam(Optimizer):
    def __init__(self, graph, learning_rate=0.01, beta_1=0.9, beta_2=0.999, eps=1e-8):
        super().__init__(graph, learning_rate)
        self.beta_1, self.beta_2, self.eps = beta_1, beta_2, eps
        self.v, self.s = {}, {}
        self.t = 0
        self.parameter_steps = {}

    def _update(self):
        self.t += 1
        scale = 1.0 if self.acc_no in (0, 1) else 1.0 / self.acc_no
        for node in self.graph.nodes:
            if isinstance(node, Variable) and node.trainable:
                grad = self.acc_gradient.get(node)
                if grad is None:
                    continue
                if node not in self.s:
                    self.v[node] = torch.zeros_like(node.value)
                    self.s[node] = torch.zeros_like(node.value)
                    self.parameter_steps[node] = 0
                step = self.parameter_steps.get(node, self.t - 1) + 1
                self.parameter_steps[node] = step
                adam_update(node.value, grad, self.v[node], self.s[node], lr=self.learning_rate, beta1=self.beta_1,
                            beta2=self.beta_2, eps=self.eps, step=step, grad_scale=scale)
