"""Optimisers over a Graph: the accumulate-then-update protocol and Adam, as in the reference's
``train/opt.py:11-281``.

``one_step()`` runs forward and backward and adds the trainable gradients into ``acc_gradient``;
``update()`` applies the step with the accumulated gradient averaged over the steps taken, then
clears the accumulators. Adam keeps zero-initialised moments and a step count per parameter and
runs as one multi-tensor libmfhip launch (per 16 tensors) with the reference's float32 rounding
order (``fused.adam_update_many``).
"""

from __future__ import annotations

from .fused import adam_update, adam_update_many
from .graph import Variable


class Optimizer:
    def __init__(self, graph, learning_rate):
        self.graph = graph
        self.learning_rate = learning_rate
        self.acc_gradient = {}
        self.acc_no = 0

    def one_step(self):
        self.forward_backward()
        self.acc_no += 1

    def forward_backward(self):
        self.graph.forward()
        self.graph.backward()
        self._accumulate_gradients()

    def _accumulate_gradients(self):
        for node in self.graph.nodes:
            if node.trainable is True and node.grad is not None:
                held = self.acc_gradient.get(node)
                if held is None:
                    self.acc_gradient[node] = node.grad
                else:
                    held += node.grad

    def get_gradient(self, node):
        """The accumulated gradient of node averaged over the steps since the last update."""
        if node not in self.acc_gradient:
            return None
        held = self.acc_gradient[node]
        return held if self.acc_no in (0, 1) else held / self.acc_no

    def apply_gradients(self, gradients, summarize=False):
        """Set (or, with summarize, add to) the accumulated gradients from a {node: gradient} map."""
        for node, gradient in gradients.items():
            if not summarize:
                self.acc_gradient[node] = gradient
            elif gradient is not None:
                if node in self.acc_gradient:
                    self.acc_gradient[node] += gradient
                else:
                    self.acc_gradient[node] = gradient

    def update(self, var_gradients=None):
        if var_gradients is not None:
            self.apply_gradients(var_gradients)
        self._update()
        self.acc_gradient.clear()
        self.acc_no = 0

    def _update(self):
        raise NotImplementedError


class MBGD(Optimizer):
    """Plain gradient descent with the averaged gradient."""

    def __init__(self, graph, learning_rate=0.01):
        super().__init__(graph, learning_rate)

    def _update(self):
        for node in list(self.acc_gradient):
            gradient = self.get_gradient(node)
            if getattr(node, "trainable", False) and gradient is not None:
                node.value -= self.learning_rate * gradient


class Adam(Optimizer):
    """Adam (Kingma and Ba, 2015) with bias correction: m = b1 m + (1 - b1) g,
    v = b2 v + (1 - b2) g^2, p -= lr (m / (1 - b1^t)) / (sqrt(v / (1 - b2^t)) + eps)."""

    def __init__(self, graph, learning_rate=0.01, beta_1=0.9, beta_2=0.999, eps=1e-8, multi_tensor=True):
        super().__init__(graph, learning_rate)
        self.beta_1, self.beta_2, self.eps = beta_1, beta_2, eps
        self.v, self.s = {}, {}  # first and second moments
        self.t = 0
        self.parameter_steps = {}
        self.multi_tensor = bool(multi_tensor)

    def _update(self):
        import torch

        self.t += 1
        scale = 1.0 if self.acc_no in (0, 1) else 1.0 / self.acc_no
        batch = []
        acc, moments, steps, lr = self.acc_gradient, self.s, self.parameter_steps, self.learning_rate
        for node in self.graph.nodes:
            gradient = acc.get(node)
            if gradient is None or not (isinstance(node, Variable) and node.trainable):
                continue
            if node not in moments:
                self.v[node] = torch.zeros_like(node.value)
                moments[node] = torch.zeros_like(node.value)
                steps[node] = 0
            step = steps.get(node, self.t - 1) + 1
            steps[node] = step
            batch.append((node.value, gradient, self.v[node], moments[node], lr, 0.0, step))
        if self.multi_tensor:
            adam_update_many(batch, beta1=self.beta_1, beta2=self.beta_2, eps=self.eps, grad_scale=scale)
        else:
            for p, g, m, v, lr, decay, step in batch:
                adam_update(p, g, m, v, lr=lr, beta1=self.beta_1, beta2=self.beta_2, eps=self.eps, step=step,
                            grad_scale=scale, weight_decay=decay)
