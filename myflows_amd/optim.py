"""Optimisers over a Graph: the accumulate-then-update protocol, parameter groups and Adam, with
the interface of the reference's ``train/opt.py:11-281`` and ``train/param_groups.py``.

``one_step()`` runs forward and backward and adds the trainable gradients into ``acc_gradient``;
``update()`` applies the step with the accumulated gradient averaged over the steps taken, then
clears the accumulators. Parameter groups give their parameters an absolute learning rate or a
multiple of the optimiser's, and a weight decay. Adam keeps zero-initialised moments and a step
count per parameter and runs as one multi-tensor libmfhip launch per 48 tensors with the
reference's float32 rounding order (``fused.adam_update_many``).
"""

from __future__ import annotations

import math
import os

from .fused import adam_update, adam_update_many
from .graph import Variable


def _non_negative(value, field):
    number = float(value)
    if not math.isfinite(number) or number < 0:
        raise ValueError(f"{field} must be finite and nonnegative")
    return number


class ParameterGroups:
    """Validated parameter groups: each a dict with ``params`` (Variables of the graph, in no other
    group), an optional unique ``name``, ``weight_decay`` (default 0) and either ``lr`` (absolute)
    or ``lr_mult`` (a multiple of the optimiser's rate, default 1). Parameters in no group take the
    optimiser's rate and no decay."""

    def __init__(self, groups, nodes):
        known = set(nodes)
        self.groups, self.by_node = [], {}
        for index, spec in enumerate(groups or ()):
            name = str(spec.get("name", f"group{index}"))
            if not name or any(g["name"] == name for g in self.groups):
                raise ValueError("parameter group names must be unique and nonempty")
            if "lr" in spec and "lr_mult" in spec:
                raise ValueError("a parameter group must choose lr or lr_mult")
            params = tuple(spec["params"])
            bad = (not params or len(set(params)) != len(params)
                   or any(not isinstance(p, Variable) or p not in known or p in self.by_node for p in params))
            if bad:
                raise ValueError(f"group {name} has empty, duplicate or unknown parameters")
            group = {"name": name, "params": params,
                     "weight_decay": _non_negative(spec.get("weight_decay", 0.0), "weight_decay")}
            if "lr" in spec:
                group["lr"] = _non_negative(spec["lr"], "group lr")
            else:
                group["lr_mult"] = _non_negative(spec.get("lr_mult", 1.0), "lr_mult")
            self.groups.append(group)
            for param in params:
                self.by_node[param] = group

    @staticmethod
    def _rate(group, base_lr):
        return group["lr"] if "lr" in group else base_lr * group["lr_mult"]

    def options(self, node, base_lr):
        """(learning rate, weight decay) of a parameter."""
        group = self.by_node.get(node)
        return (base_lr, 0.0) if group is None else (self._rate(group, base_lr), group["weight_decay"])

    def rates(self, base_lr):
        return {group["name"]: self._rate(group, base_lr) for group in self.groups}


class Optimizer:
    def __init__(self, graph, learning_rate, param_groups=None):
        self.graph = graph
        self.learning_rate = learning_rate
        self.acc_gradient = {}
        self.acc_no = 0
        self.groups = ParameterGroups(param_groups, graph.nodes)

    def set_param_groups(self, groups):
        self.groups = ParameterGroups(groups, self.graph.nodes)

    def group_learning_rates(self):
        return self.groups.rates(self.learning_rate)

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

    def _group_gradient(self, node):
        """(averaged gradient plus the group's weight decay times the value, the group's rate)."""
        gradient = self.get_gradient(node)
        lr, decay = self.groups.options(node, self.learning_rate)
        if gradient is not None and decay:
            gradient = gradient + decay * node.value
        return gradient, lr

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
    """Plain gradient descent with the averaged gradient (plus the group's weight decay)."""

    def __init__(self, graph, learning_rate=0.01, *, param_groups=None):
        super().__init__(graph, learning_rate, param_groups)

    def _update(self):
        for node in list(self.acc_gradient):
            if not getattr(node, "trainable", False):
                continue
            gradient, lr = self._group_gradient(node)
            if gradient is not None:
                node.value -= lr * gradient


class Adam(Optimizer):
    """Adam (Kingma and Ba, 2015) with bias correction: m = b1 m + (1 - b1) g,
    v = b2 v + (1 - b2) g^2, p -= lr (m / (1 - b1^t)) / (sqrt(v / (1 - b2^t)) + eps), where g is the
    averaged gradient (plus the group's weight decay times p) and t counts this parameter's own
    updates: a parameter frozen for a while, or without a gradient at some update, starts at t = 1
    when it is first updated. ``v`` and ``s`` hold the first and second moments, ``parameter_steps``
    each parameter's t, ``t`` the optimiser's update count."""

    def __init__(self, graph, learning_rate=0.01, beta_1=0.9, beta_2=0.999, eps=1e-8, *, param_groups=None,
                 multi_tensor=None):
        super().__init__(graph, learning_rate, param_groups)
        self.beta_1, self.beta_2, self.eps = beta_1, beta_2, eps
        self.v, self.s = {}, {}
        self.t = 0
        self.parameter_steps = {}
        if multi_tensor is None:
            multi_tensor = os.environ.get("MYFLOWS_MULTI_ADAM", "1") == "1"
        self.multi_tensor = bool(multi_tensor)

    def _state_of(self, node):
        """(first moment, second moment, step) of node for this update: zero moments on its first
        update, and its step count advanced by one."""
        if node not in self.parameter_steps:
            import torch
            self.v[node], self.s[node] = torch.zeros_like(node.value), torch.zeros_like(node.value)
            self.parameter_steps[node] = 0
        self.parameter_steps[node] += 1
        return self.v[node], self.s[node], self.parameter_steps[node]

    def _update(self):
        self.t += 1
        # The averaging over the accumulated steps rides in the kernel as a gradient scale.
        scale = 1.0 if self.acc_no in (0, 1) else 1.0 / self.acc_no
        updates = []
        for node in self.graph.nodes:
            if not (isinstance(node, Variable) and node.trainable):
                continue
            gradient = self.acc_gradient.get(node)
            if gradient is not None:
                lr, decay = self.groups.options(node, self.learning_rate)
                first, second, step = self._state_of(node)
                updates.append((node.value, gradient, first, second, lr, decay, step))
        options = dict(beta1=self.beta_1, beta2=self.beta_2, eps=self.eps)
        if self.multi_tensor:
            adam_update_many(updates, grad_scale=scale, **options)
            return
        for param, gradient, first, second, lr, decay, step in updates:
            adam_update(param, gradient, first, second, lr=lr, step=step, grad_scale=scale, weight_decay=decay,
                        **options)
