"""The dynamic graph: nodes, leaves and the executor that runs them over torch GPU tensors.

Keeps the semantics of the reference's ``core/node.py:5-123`` and ``core/graph.py:5-162``, so the
``hip_native`` operators plug in under an unchanged Variable/Graph API:

* ``Variable(value, trainable, name, constant, requires_grad)``: a trainable leaf always needs a
  gradient; another leaf with ``requires_grad=False`` (input images, labels) lets the operators
  skip the gradient work for it (e.g. the dX GEMMs of the stem convolution);
* ``accumulate_grad(contribution, owned=...)``: the first contribution becomes the gradient (kept
  without a copy only when its producer hands it over), later ones are added in place, each
  rounded to the value's dtype;
* ``Graph(target)``: topological order; for each combination of leaf flags (and retained
  intermediates) an execution plan of which nodes need gradients; ``forward()`` in order,
  ``backward()`` in reverse seeded with ones; intermediate gradients are released as soon as their
  node has consumed them. Before each pass, the kernel reorders that the pass's implicit-GEMM
  convolutions read are made by one native launch for all of them (``weight_orders``), and the
  convolutions' dW products run on a second stream beside their dX products (``streams.py``).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import streams


class Node:
    """A vertex of the graph: parents in, one value out, one gradient back."""

    # Set per node by the executing Graph; a standalone operator behaves as if it needs gradients.
    requires_grad = True

    def __init__(self, *parents, trainable=False, name=None):
        self.parents = list(parents)
        self.children = []
        for parent in self.parents:
            parent.children.append(self)
        self.value = None
        self.grad = None
        self.trainable = trainable
        self.name = name or type(self).__name__

    def forward(self, *inputs):
        raise NotImplementedError

    def backward(self):
        raise NotImplementedError

    def clear_grad(self):
        """Zero gradient of the value's shape (None before the first forward)."""
        self.grad = None if self.value is None else torch.zeros_like(self.value)

    def accumulate_grad(self, contribution, *, owned=False):
        """Add a gradient contribution. The first one becomes the gradient: as is when the caller
        owns a fresh contiguous tensor of the value's shape (owned=True), otherwise as a copy."""
        target = self.value
        if not isinstance(contribution, torch.Tensor):
            contribution = torch.as_tensor(contribution, device=target.device)
        if self.grad is not None:
            self.grad += contribution.to(target.dtype)
            return
        if contribution.shape != target.shape:
            contribution, owned = contribution.expand(target.shape), False
        contribution = contribution.to(target.dtype)
        if owned and contribution.is_contiguous():
            self.grad = contribution
        else:
            self.grad = contribution.clone(memory_format=torch.contiguous_format)

    def grad_buffer(self):
        """(tensor, add): where to write this node's gradient, and whether to add to what is
        there (True) or overwrite a fresh, uninitialised buffer (False)."""
        if self.grad is not None:
            return self.grad, True
        self.grad = torch.empty_like(self.value)
        return self.grad, False


class GradientOp(Node):
    """An operator whose backward writes its parents' gradients itself (first write included)."""


class Variable(Node):
    """A leaf: parameter (trainable), input or constant."""

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
    def trainable(self, flag):
        self._trainable = bool(flag)
        self._is_parameter = self._is_parameter or self._trainable

    @property
    def requires_grad(self):
        # Once a parameter, the trainable flag decides; other leaves keep their own flag.
        return self._trainable if self._is_parameter else self._wants_grad

    @requires_grad.setter
    def requires_grad(self, flag):
        self._wants_grad = bool(flag)

    def forward(self):
        pass

    def backward(self):
        pass


def topological_order(root):
    """Post-order of a depth-first walk over parents (parents in order), iteratively."""
    order, seen = [], set()
    stack = [(root, False)]
    while stack:
        node, done = stack.pop()
        if done:
            order.append(node)
            continue
        if node in seen:
            continue
        seen.add(node)
        stack.append((node, True))
        for parent in reversed(node.parents):
            if parent not in seen:
                stack.append((parent, False))
    return order


def _prepare_weight_orders(units, phase):
    """Batch the kernel reorders of every unit that asks for some in this pass (a convolution's
    ``weight_orders(phase)``) into one native launch and hand each unit its results. Returns the
    units served, whose unused results the caller drops after the pass."""
    pending = []
    for unit in units:
        wants = getattr(unit, "weight_orders", None)
        requests = wants(phase) if wants is not None else None
        if requests:
            pending.append((unit, requests))
    if not pending:
        return ()
    from . import native
    made = native.conv_weight_orders([r for _, requests in pending for r in requests])
    first = 0
    for unit, requests in pending:
        unit.take_weight_orders(phase, made[first:first + len(requests)])
        first += len(requests)
    return tuple(unit for unit, _ in pending)


def _next_on_stream(steps):
    """For a sequence of (unit, kind) forward steps: unit -> the next unit issued on the same stream
    (MAIN units on the current stream, SIDE units on the side stream)."""
    after, last = {}, {}
    for unit, kind in steps:
        if kind in (FORK, JOIN) or unit is None or not unit.parents:
            continue
        stream = SIDE if kind == SIDE else MAIN
        if stream in last:
            after[last[stream]] = unit
        last[stream] = unit
    return after


@dataclass(frozen=True)
class _Plan:
    """What one combination of leaf flags and retained nodes asks of a graph."""
    needs: tuple            # (node, needs a gradient) for every node, in topological order
    active: frozenset       # nodes that need a gradient
    forward_units: tuple    # nodes (or fused groups) to run forward, in order
    backward_units: tuple   # (unit, node whose gradient the unit consumes), in reverse order
    pre_clear: dict         # non-GradientOp unit -> its parents that need a zero gradient first
    keep: tuple             # nodes whose gradient survives backward (leaves, retained nodes)
    groups: frozenset       # fused groups in use
    forward_steps: tuple    # forward_units with shortcut branches on the side stream: (unit, step kind)
    deferred: tuple         # per forward order (one stream, branches on the side stream): convolution ->
                            # the batch norm, its only consumer and next on its stream, that may form its output
    deferred_dx: dict       # convolution -> the batch-norm unit, next in the backward order, whose output
                            # is the convolution's input and has no other consumer: it may form the dX


# Kinds of a forward step: a unit on the current stream, the fork of a branch (the side stream waits
# for the current one), a unit of that branch (issued on the side stream), the join before the
# branch's consumer (the current stream waits for the side stream).
MAIN, FORK, SIDE, JOIN = 0, 1, 2, 3


class Graph:
    """Forward and backward over the subgraph that produces ``target_node``."""

    _installed = None  # the plan whose per-node flags are written into the (possibly shared) nodes
    _deferred_installed = None  # (plan, forward order) whose deferred pairs the nodes hold
    _deferred_dx_installed = None  # the plan whose deferred dX pairs the nodes hold

    def __init__(self, target_node, optimize=False, fold_constants=False, fuse_linear=True, fuse_activations=True):
        self._opt_stats = None
        if optimize:
            from .fusion import apply_graph_optimizations
            target_node, self._opt_stats = apply_graph_optimizations(
                target_node, fold_constants=fold_constants, fuse_linear=fuse_linear,
                fuse_activations=fuse_activations)
        self.target_node = target_node
        self.sorted_nodes = topological_order(target_node)
        self.nodes = self.sorted_nodes
        self._bn_groups = {}
        if optimize and fuse_activations:
            from .fusion import batchnorm_activation_groups
            self._bn_groups = batchnorm_activation_groups(self.nodes)
        if self._opt_stats is not None:
            self._opt_stats["bn_activation_fusions"] = len(self._bn_groups)
        self.profiler = None
        # Whether backward() runs the convolutions' dW products on the weight-gradient stream
        # (streams.py) beside their dX products; the gradients are the same either way.
        self.overlap_weight_grads = True
        # Whether forward() runs convolution + batch-norm shortcut branches (a ResNet downsample) on
        # the side stream beside the main path; the values are the same either way.
        self.overlap_branches = True
        self._leaves = tuple(node for node in self.nodes if not node.parents)
        self._retained = set()
        self._materialize = False
        self._plans = {}
        self._forward_plan = None

    def materialize_intermediates(self, enabled=True):
        """Run the fused units' nodes one by one from the next forward on (while enabled), so that
        the batch-norm and residual-add values a fused unit never forms are there to inspect; the
        results are the same bits either way."""
        if self._materialize != bool(enabled):
            self._materialize = bool(enabled)
            self._plans.clear()

    def retain_grad(self, *nodes):
        """Keep the gradients of these intermediates (or differentiable leaves) after backward."""
        for node in nodes:
            if node not in self.nodes or (not node.parents and not node.requires_grad):
                raise ValueError("retain_grad expects a graph intermediate or a differentiable leaf")
        self._retained.update(node for node in nodes if node.parents)
        self._plans.clear()

    def _make_plan(self, flags):
        needs = dict(zip(self._leaves, flags))
        propagating = []
        for node in self.nodes:
            if node.parents:
                from_parents = any(needs[p] for p in node.parents)
                needs[node] = from_parents or node in self._retained
                if from_parents:
                    propagating.append(node)
        groups = {} if self._materialize else {
            out: g for out, g in self._bn_groups.items() if self._retained.isdisjoint(g.hidden)}
        hidden = {node for g in groups.values() for node in g.hidden}
        forward_units = tuple(groups.get(n, n) for n in self.nodes if n not in hidden)
        backward_units = tuple((groups.get(n, n), n) for n in reversed(propagating) if n not in hidden)
        pre_clear = {n: tuple(p for p in n.parents if needs[p]) for n in propagating if not isinstance(n, GradientOp)}
        keep = tuple(n for n in self.nodes if needs[n] and (not n.parents or n in self._retained))
        forward_steps = self._forward_steps(forward_units, groups)
        return _Plan(tuple(needs.items()), frozenset(n for n, need in needs.items() if need), forward_units,
                     backward_units, pre_clear, keep, frozenset(groups), forward_steps,
                     self._deferred_splits(groups, forward_units, forward_steps),
                     self._deferred_input_grads(backward_units))

    def _deferred_splits(self, groups, forward_units, forward_steps):
        """Plain convolutions (no fused activation) whose only consumer is a batch norm
        that runs alone or as the BN of a BN(+Add)+ReLU unit: a training batch norm of few enough
        positions forms such a convolution's output from the product's split-K slices itself
        (Conv2D_Op.forward, fused.batchnorm2d_forward). The slices wait in the stream's convolution
        workspace, so a pair is kept only when the batch norm's unit is the next unit issued on the
        convolution's stream, and no other product on that stream runs between. Returns the pairs
        of each forward order: (forward_units on one stream, forward_steps with the shortcut
        branches on the side stream)."""
        from .ops_conv import Conv2D_Op
        from .ops_norm import BatchNorm2d_Op, BatchNormActivation
        consumers = {}
        for node in self.nodes:
            for parent in node.parents:
                consumers.setdefault(parent, set()).add(node)
        in_unit = {g.bn: g for g in groups.values()}
        pairs = {}
        for node in self.nodes:
            if type(node) is not Conv2D_Op or node is self.target_node:
                continue
            users = consumers.get(node, ())
            bn = next(iter(users)) if len(users) == 1 else None
            if (isinstance(bn, BatchNorm2d_Op) and bn.parents[0] is node and node not in self._retained
                    and (bn not in in_unit or isinstance(in_unit[bn], BatchNormActivation))):
                pairs[node] = bn
        if not pairs:
            return {}, {}
        unit_of = {g.bn: g for g in groups.values()}
        orders = (_next_on_stream((unit, MAIN) for unit in forward_units), _next_on_stream(forward_steps))
        return tuple({conv: bn for conv, bn in pairs.items() if after.get(conv) is unit_of.get(bn, bn)}
                     for after in orders)

    def _deferred_input_grads(self, backward_units):
        """Convolutions whose input is the output of a batch norm (alone, or the end of a
        BN(+Add)+ReLU unit) with no other consumer, that unit being the next in the backward order:
        a training batch norm of few enough positions forms such a convolution's dX from the dX
        product's split-K slices itself (Conv2D_Op.backward, fused.batchnorm2d_backward). The
        gradient is then the dX alone (no other consumer adds to it) and nothing runs between the
        product and the batch norm. A retained input keeps its gradient formed."""
        from .ops_conv import Conv2D_Op
        from .ops_norm import BatchNorm2d_Op, BatchNormActivation
        consumers = {}
        for node in self.nodes:
            for parent in node.parents:
                consumers.setdefault(parent, set()).add(node)
        pairs = {}
        for (unit, _), (after, after_output) in zip(backward_units, backward_units[1:]):
            if not isinstance(unit, Conv2D_Op):
                continue
            x_node = unit.parents[0]
            if (x_node is after_output and consumers.get(x_node) == {unit} and x_node not in self._retained
                    and x_node is not self.target_node
                    and (isinstance(after, BatchNormActivation) or isinstance(after, BatchNorm2d_Op))):
                pairs[unit] = after
        return pairs

    def _install_deferred_dx(self, plan):
        """Write this plan's deferred dX pairs into the convolution nodes (which another graph may
        have set otherwise)."""
        if Graph._deferred_dx_installed is plan:
            return
        for node, _ in plan.needs:
            if hasattr(node, "_defer_dx"):
                node._defer_dx = plan.deferred_dx.get(node)
        Graph._deferred_dx_installed = plan

    def _forward_steps(self, forward_units, groups):
        """forward_units with every convolution + batch-norm shortcut (a ResNet downsample: a Conv2D
        whose only consumer is a BatchNorm2d whose only consumer is the residual Add of a fused
        BN+Add+ReLU unit) moved up to just after the unit that makes the convolution's input and
        issued on the side stream, so that it runs beside the main path's convolutions; the fused
        unit waits for it. Each node still runs after its parents and before its consumers."""
        from .ops_conv import Conv2D_Op
        from .ops_norm import BatchNorm2d_Op, BatchNormActivation
        consumers = {}
        for node in self.nodes:
            for parent in node.parents:
                consumers.setdefault(parent, set()).add(node)
        units = list(forward_units)
        producer = {}
        for unit in units:
            producer[getattr(unit, "output", unit)] = unit
        branches = []
        for consumer in units:
            if not isinstance(consumer, BatchNormActivation) or consumer.residual is None or consumer.add is None:
                continue
            bn = consumer.residual
            conv = bn.parents[0] if isinstance(bn, BatchNorm2d_Op) else None
            if (not isinstance(conv, Conv2D_Op) or bn not in units or conv not in units
                    or consumers.get(bn) != {consumer.add} or consumers.get(conv) != {bn}
                    or any(p.parents for p in conv.parents[1:] + bn.parents[1:])):
                continue
            branches.append((conv, bn, consumer))
        if not branches:
            return tuple((unit, MAIN) for unit in units)
        for conv, bn, _ in branches:
            units.remove(conv)
            units.remove(bn)
        steps = [(unit, MAIN) for unit in units]
        for conv, bn, consumer in branches:
            anchor = producer.get(conv.parents[0])
            at = 0 if anchor is None else next(i for i, (u, _) in enumerate(steps) if u is anchor) + 1
            steps[at:at] = [(None, FORK), (conv, SIDE), (bn, SIDE)]
            join = next(i for i, (u, _) in enumerate(steps) if u is consumer)
            steps.insert(join, (None, JOIN))
        return tuple(steps)

    def _plan(self):
        flags = tuple(leaf.requires_grad for leaf in self._leaves)
        plan = self._plans.get(flags)
        if plan is None:
            plan = self._plans[flags] = self._make_plan(flags)
        if Graph._installed is not plan:
            # Another graph may share these nodes with other needs: write this plan's flags back.
            for node, need in plan.needs:
                if node.parents:
                    node.requires_grad = need
                if not need:
                    node.grad = None
            Graph._installed = plan
        return plan

    def _install_deferred(self, plan, overlapped):
        """Write the deferred convolution -> batch norm pairs of this plan's forward order into the
        convolution nodes (which another graph or order may have set otherwise)."""
        key = (plan, overlapped)
        if Graph._deferred_installed == key:
            return
        pairs = plan.deferred[1 if overlapped else 0]
        for node, _ in plan.needs:
            if hasattr(node, "_defer_bn"):
                node._defer_bn = pairs.get(node)
        Graph._deferred_installed = key

    def forward(self):
        plan = self._plan()
        self._forward_plan = plan
        profiler = self.profiler
        overlapped = profiler is None and self.overlap_branches
        from . import native
        native.drop_pending_splits()  # outputs a failed earlier forward left unformed
        self._install_deferred(plan, overlapped)
        served = _prepare_weight_orders((u for u in plan.forward_units if u.parents), "forward")
        if overlapped:
            self._run_steps(plan.forward_steps)
        else:
            for unit in plan.forward_units:
                if not unit.parents:
                    continue
                inputs = [p.value for p in unit.parents]
                if profiler is None:
                    unit.forward(*inputs)
                else:
                    with profiler.node(unit, "forward"):
                        unit.forward(*inputs)
        for unit in served:
            unit.drop_weight_orders("forward")

    @staticmethod
    def _run_steps(steps):
        """Run forward steps (see _forward_steps). A branch takes the side stream only when its input
        is a GPU tensor; otherwise its units run in place, in the same order."""
        from . import native
        side = main = None
        for unit, kind in steps:
            if kind == FORK:
                side = main = None
                continue
            if kind == JOIN:
                if side is not None:
                    native.stream_wait(main, side)
                side = main = None
                continue
            if not unit.parents:
                continue
            inputs = [p.value for p in unit.parents]
            if kind == SIDE:
                if side is None and main is None:
                    x = inputs[0]
                    if isinstance(x, torch.Tensor) and x.is_cuda:
                        main = native._stream()
                        side = streams.side_stream(native.current_device_index()).cuda_stream
                        native.stream_wait(side, main)
                    else:
                        main = False  # no side stream for this branch
                if side is not None:
                    with native.launch_stream(side):
                        unit.forward(*inputs)
                    continue
            unit.forward(*inputs)

    def backward(self, loss_scale=1.0):
        plan = self._plan()
        ran = self._forward_plan
        if ran is not None and ran is not plan and (not plan.active <= ran.active or plan.groups != ran.groups):
            raise RuntimeError("new gradients requested after forward; run forward again to rebuild saved tensors")
        if self.target_node not in plan.active:
            return
        for node in plan.active:
            node.grad = None
        seed = self.target_node.value
        if isinstance(seed, torch.Tensor) and seed.is_cuda and seed.dtype == torch.float32:
            from . import native  # a library launch, so that a recorded program seeds its backward too
            self.target_node.grad = native.fill_(torch.empty_like(seed, memory_format=torch.contiguous_format),
                                                 loss_scale)
        else:
            self.target_node.grad = (torch.ones_like(seed) if loss_scale == 1.0
                                     else torch.full_like(seed, loss_scale))
        profiler = self.profiler
        self._install_deferred_dx(plan)
        served = _prepare_weight_orders((unit for unit, _ in plan.backward_units), "backward")
        overlap = self.overlap_weight_grads and isinstance(seed, torch.Tensor) and seed.is_cuda
        with streams.weight_grad_overlap(overlap):
            for unit, output in plan.backward_units:
                if output.grad is None:
                    continue
                for parent in plan.pre_clear.get(unit, ()):
                    if parent.grad is None:  # a plain Node may add into parent.grad directly
                        parent.clear_grad()
                retained = output.grad if output in self._retained else None
                if profiler is None:
                    unit.backward()
                else:
                    with profiler.node(unit, "backward"):
                        unit.backward()
                output.grad = retained  # release the consumed intermediate gradient unless retained
        for unit in served:
            unit.drop_weight_orders("backward")
        for node in plan.keep:
            if node.grad is None:
                node.clear_grad()
