"""Dynamic-graph core: Node, GradientOp, Variable and Graph over torch device tensors.

Restates the reference's ``core/node.py:5-123`` and ``core/graph.py:5-162`` with the same
semantics, so that the ``hip_native`` operators plug in under an unchanged Variable/Graph API:

* ``Variable(value, trainable, name, constant, requires_grad)``: trainable parameters always need a
  gradient; a leaf with ``requires_grad=False`` (input images, labels) lets operators skip the
  gradient GEMMs for it;
* ``accumulate_grad(contribution, owned=...)``: the first contribution becomes the gradient buffer
  (without a copy only when the caller owns it), later ones are added in place;
* ``Graph(target)``: topological order, a cached plan of which nodes need gradients (invalidated
  when leaf flags change), ``forward()`` in order and ``backward()`` in reverse order seeded with
  ones.
"""

from __future__ import annotations

import torch


class Node:
    requires_grad = True

    def __init__(self, *parents, trainable=False, name=None):
        self.parents = list(parents)
        self.children = []
        for p in parents:
            p.children.append(self)
        self.value = None
        self.grad = None
        self.trainable = trainable
        self.name = name if name else self.__class__.__name__

    def forward(self, *inputs):
        raise NotImplementedError

    def backward(self):
        raise NotImplementedError

    def clear_grad(self):
        self.grad = None if self.value is None else torch.zeros_like(self.value)

    def accumulate_grad(self, contribution, *, owned=False):
        """Write the first contribution, then sum. Only freshly allocated results may transfer ownership."""
        value = self.value
        if not isinstance(contribution, torch.Tensor):
            contribution = torch.as_tensor(contribution, device=value.device)
        if self.grad is not None:
            self.grad += contribution.to(value.dtype)
            return
        if tuple(contribution.shape) != tuple(value.shape):
            contribution = contribution.expand(value.shape)
            owned = False
        contribution = contribution.to(value.dtype)
        if owned and contribution.is_contiguous():
            self.grad = contribution
        else:
            self.grad = contribution.clone(memory_format=torch.contiguous_format)

    def grad_buffer(self):
        """Return a writable gradient and whether the caller must add to its existing contents."""
        add = self.grad is not None
        if not add:
            self.grad = torch.empty_like(self.value)
        return self.grad, add


class GradientOp(Node):
    """Operator whose backward handles the first write to each parent's gradient."""


class Variable(Node):
    def __init__(self, value=None, trainable=False, name=None, constant=False, requires_grad=True):
        self._is_parameter = False
        super().__init__(trainable=trainable, name=name)
        self.value = value
        self.constant = bool(constant)
        self.requires_grad = requires_grad

    @property
    def trainable(self):
        return self._trainable

    @trainable.setter
    def trainable(self, value):
        self._trainable = bool(value)
        if self._trainable:
            self._is_parameter = True

    @property
    def requires_grad(self):
        return self._trainable if self._is_parameter else self._leaf_requires_grad

    @requires_grad.setter
    def requires_grad(self, value):
        self._leaf_requires_grad = bool(value)

    def forward(self):
        pass

    def backward(self):
        pass


class Graph:
    _active_plan = None

    def __init__(self, target_node, optimize=False, fold_constants=False, fuse_linear=True, fuse_activations=True):
        self._opt_stats = None
        if optimize:
            from .graph_opt import apply_graph_optimizations
            self.target_node, self._opt_stats = apply_graph_optimizations(
                target_node, fold_constants=fold_constants, fuse_linear=fuse_linear, fuse_activations=fuse_activations)
        else:
            self.target_node = target_node
        self.sorted_nodes = self._build_topo_sort(self.target_node)
        self.nodes = self.sorted_nodes
        if optimize and fuse_activations:
            from .graph_opt import batchnorm_activation_groups
            self._bn_groups = batchnorm_activation_groups(self.nodes)
        else:
            self._bn_groups = {}
        if self._opt_stats is not None:
            self._opt_stats["bn_activation_fusions"] = len(self._bn_groups)
        self._leaves = [node for node in self.nodes if not node.parents]
        self._retained = set()
        self._signature = None
        self._forward_active = None
        self._forward_groups = None
        self._refresh_gradients()

    def retain_grad(self, *nodes):
        for node in nodes:
            if node not in self.nodes or (not node.parents and not node.requires_grad):
                raise ValueError("retain_grad expects a graph intermediate or a differentiable leaf")
        self._retained.update(node for node in nodes if node.parents)
        self._signature = None

    def _refresh_gradients(self):
        """Cache a topological plan; changing leaf flags or retained targets invalidates it
        (core/graph.py:63-100)."""
        signature = tuple(node.requires_grad for node in self._leaves)
        if signature != self._signature:
            needed = dict(zip(self._leaves, signature))
            propagate = []
            for node in self.nodes:
                if node.parents:
                    parents_need_grad = any(needed[p] for p in node.parents)
                    needed[node] = parents_need_grad or node in self._retained
                    if parents_need_grad:
                        propagate.append(node)
            self._active = frozenset(node for node, required in needed.items() if required)
            self._flags = tuple(needed.items())
            groups = {n: g for n, g in self._bn_groups.items() if self._retained.isdisjoint(g.hidden)}
            hidden = {node for group in groups.values() for node in group.hidden}
            self._group_signature = frozenset(groups)
            self._execution_nodes = tuple(groups.get(n, n) for n in self.nodes if n not in hidden)
            self._backward_nodes = tuple((groups.get(n, n), n) for n in reversed(propagate) if n not in hidden)
            self._keep_grads = tuple(n for n in self.nodes if needed[n] and (not n.parents or n in self._retained))
            self._clear_nodes = tuple(node for node in self.nodes if node in self._active)
            self._signature = signature
            self._plan = object()
        if Graph._active_plan is not self._plan:
            for node, required in self._flags:
                if node.parents:
                    node.requires_grad = required
                if not required:
                    node.grad = None
            Graph._active_plan = self._plan

    @staticmethod
    def _build_topo_sort(target_node):
        visited, order = set(), []
        stack = [(target_node, False)]
        while stack:
            node, expanded = stack.pop()
            if expanded:
                order.append(node)
                continue
            if node in visited:
                continue
            visited.add(node)
            stack.append((node, True))
            for p in reversed(getattr(node, "parents", [])):
                if p not in visited:
                    stack.append((p, False))
        return order

    def forward(self):
        self._refresh_gradients()
        self._forward_active = self._active
        self._forward_groups = self._group_signature
        for node in self._execution_nodes:
            if node.parents:
                node.forward(*[p.value for p in node.parents])
            elif isinstance(node, Variable):
                continue

    def backward(self, loss_scale=1.0):
        self._refresh_gradients()
        if self._forward_active is not None and self._forward_active is not self._active:
            if not self._active.issubset(self._forward_active) or self._forward_groups != self._group_signature:
                raise RuntimeError("new gradients requested after forward; run forward again to rebuild saved tensors")
        if self.target_node not in self._active:
            return
        for n in self._clear_nodes:
            n.grad = None
        value = self.target_node.value
        self.target_node.grad = torch.ones_like(value) if loss_scale == 1.0 else torch.full_like(value, loss_scale)
        for node, output in self._backward_nodes:
            if output.grad is None:
                continue
            saved = output.grad if output in self._retained else None
            node.backward()
            # An intermediate adjoint is released as soon as its node has consumed it, unless retained.
            output.grad = saved
        for node in self._keep_grads:
            if node.grad is None:
                node.clear_grad()
