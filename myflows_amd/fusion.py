"""Build-time graph rewrites used by ``Graph(optimize=True)`` and ``apply_graph_optimizations``.

The passes of the reference's ``core/graph_opt.py``:

* ``fold_constant_adds`` (:60-103): Add(constant Variable, constant Variable) -> one constant;
* ``fuse_conv_activation_ops`` (:295-349): ReLU / LeakyReLU of a plain Conv2D_Op -> the fused
  Conv2D_ReLU_Op / Conv2D_LeakyReLU_Op (activation in the GEMM epilogue);
* ``fold_bn_into_conv`` (:114-190): eval-mode BatchNorm of a Conv2D_Op used only by it -> the
  convolution with copies of its kernel and bias scaled by gamma / sqrt(var + eps) (the model's own
  parameters are left untouched);
* ``batchnorm_activation_groups`` (:231-257): ReLU(BN(x)) and ReLU(BN(x) + residual) whose
  intermediates nobody else reads -> one BatchNormActivation unit; MaxPool(ReLU(BN(x))) whose ReLU
  output only the max-pool reads -> one BatchNormReLUPool unit (no counterpart in the reference);
* ``fuse_conv_add_relu`` (inference, after the BN fold; no counterpart in the reference):
  ReLU(Conv2D_Op + residual) whose convolution and Add outputs nobody else reads -> one
  Conv2D_AddReLU_Op, the residual add and the ReLU in the GEMM epilogue.

As in the reference, ``mode="inference"`` turns on the BN fold, and activation fusion runs before
it within one call, so a ReLU whose parent becomes a convolution only through folding is fused by a
second pass (``Graph(root, optimize=True)`` on the folded root).
"""

from __future__ import annotations

from collections import Counter

import torch

from .graph import Variable, topological_order


def replace_node(old, new):
    """Rewire every child of ``old`` to ``new`` and detach ``old`` from its parents."""
    for parent in old.parents:
        if old in parent.children:
            parent.children.remove(old)
    for child in old.children:
        child.parents = [new if p is old else p for p in child.parents]
        if child not in new.children:
            new.children.append(child)
    old.children = []


def _swap_parent(node, index, new_parent):
    old = node.parents[index]
    node.parents[index] = new_parent
    if node in old.children:
        old.children.remove(node)
    if node not in new_parent.children:
        new_parent.children.append(node)


def fold_constant_adds(root):
    from .ops_basic import Add

    total = 0
    while True:
        folded = 0
        for node in topological_order(root):
            if type(node) is not Add or len(node.parents) != 2:
                continue
            a, b = node.parents
            if not all(isinstance(v, Variable) and v.constant for v in (a, b)):
                continue
            bv = b.value.reshape(1, -1, 1, 1) if a.value.ndim == 4 and b.value.ndim == 1 else b.value
            constant = Variable(a.value + bv, trainable=False, name=f"{node.name}_folded", constant=True)
            if node is root:
                root = constant
            replace_node(node, constant)
            folded += 1
        total += folded
        if not folded:
            return root, total


def fuse_conv_activation_ops(root):
    from .ops_basic import LeakyReLU, ReLU
    from .ops_conv import Conv2D_LeakyReLU_Op, Conv2D_Op, Conv2D_ReLU_Op

    fused = 0
    for node in topological_order(root):
        if type(node) not in (ReLU, LeakyReLU) or len(node.parents) != 1:
            continue
        conv = node.parents[0]
        if type(conv) is not Conv2D_Op:
            continue
        bias = conv.parents[2] if len(conv.parents) == 3 else None
        options = dict(stride=conv.stride, padding=conv.padding, bias=bias, backend=conv.backend,
                       recompute_im2col=conv.recompute_im2col)
        if type(node) is ReLU:
            replacement = Conv2D_ReLU_Op(conv.parents[0], conv.parents[1], **options)
        else:
            replacement = Conv2D_LeakyReLU_Op(conv.parents[0], conv.parents[1], alpha=node.alpha, **options)
        if node is root:
            root = replacement
        replace_node(node, replacement)
        fused += 1
    return root, fused


def _folded_parameters(conv, bn):
    """Kernel and bias of conv followed by eval-mode bn, computed in FP64 and rounded once."""
    kernel = conv.parents[1].value.double()
    scale = bn.parents[1].value.double() / torch.sqrt(bn.running_var.double() + bn.eps)
    bias = conv.parents[2].value.double() if conv.bias is not None else torch.zeros_like(scale)
    folded_bias = (bias - bn.running_mean.double()) * scale + bn.parents[2].value.double()
    return (kernel * scale.reshape(-1, 1, 1, 1)).float(), folded_bias.float()


def fold_bn_into_conv(root):
    from .ops_conv import Conv2D_Op
    from .ops_norm import BatchNorm2d_Op

    folded = 0
    for node in topological_order(root):
        if not isinstance(node, BatchNorm2d_Op) or node.training:
            continue
        conv = node.parents[0]
        if type(conv) is not Conv2D_Op or any(child is not node for child in conv.children):
            continue
        kernel, bias = _folded_parameters(conv, node)
        old_kernel = conv.parents[1]
        _swap_parent(conv, 1, Variable(kernel, trainable=old_kernel.trainable, name=f"{old_kernel.name}_bn_folded"))
        if conv.bias is not None:
            old_bias = conv.parents[2]
            new_bias = Variable(bias, trainable=old_bias.trainable, name=f"{old_bias.name}_bn_folded")
            _swap_parent(conv, 2, new_bias)
        else:
            new_bias = Variable(bias, trainable=True, name=f"{conv.name}_folded_bias")
            conv.parents.append(new_bias)
            new_bias.children.append(conv)
        conv.bias = new_bias
        if node is root:
            root = conv
        replace_node(node, conv)
        folded += 1
    return root, folded


def apply_graph_optimizations(root, *, mode="train", fold_constants=True, fuse_linear=True, fuse_activations=True,
                              fold_bn=None):
    """(new root, statistics). ``fuse_linear`` is accepted for interface parity: this package builds
    Linear directly and has no separate MatMul + Add to fuse."""
    if fold_bn is None:
        fold_bn = str(mode).lower() == "inference"
    stats = {"constant_folds": 0, "linear_fusions": 0, "conv_act_fusions": 0, "bn_folds": 0,
             "conv_add_act_fusions": 0}
    if fold_constants:
        root, stats["constant_folds"] = fold_constant_adds(root)
    if fuse_activations:
        root, stats["conv_act_fusions"] = fuse_conv_activation_ops(root)
    if fold_bn:
        root, stats["bn_folds"] = fold_bn_into_conv(root)
        if fuse_activations:
            root, stats["conv_add_act_fusions"] = fuse_conv_add_relu(root)
        mark_inference_pools(root)
    return root, stats


def mark_inference_pools(root):
    """Max-pools of an inference graph (batch norms folded) do not store their window indices: no
    backward reads them (MaxPool2d_Op.backward then raises)."""
    from .ops_conv import MaxPool2d_Op

    for node in topological_order(root):
        if isinstance(node, MaxPool2d_Op):
            node.inference = True


def fuse_conv_add_relu(root):
    """ReLU(Add(Conv2D_Op, residual)) -> Conv2D_AddReLU_Op when the convolution and the Add have no
    other reader (a residual block's second convolution once its BN is folded). For graphs that take
    no gradient: the fused operator has no backward."""
    from .ops_basic import Add, ReLU
    from .ops_conv import Conv2D_AddReLU_Op, Conv2D_Op

    fused = 0
    for node in topological_order(root):
        if type(node) is not ReLU or len(node.parents) != 1:
            continue
        add = node.parents[0]
        if type(add) is not Add or len(add.parents) != 2 or add.children != [node]:
            continue
        pick = None
        for k in (0, 1):
            conv, residual = add.parents[k], add.parents[1 - k]
            if type(conv) is Conv2D_Op and conv.children == [add] and residual is not conv:
                pick = (conv, residual)
                break
        if pick is None:
            continue
        conv, residual = pick
        bias = conv.parents[2] if len(conv.parents) == 3 else None
        replacement = Conv2D_AddReLU_Op(conv.parents[0], conv.parents[1], residual, stride=conv.stride,
                                        padding=conv.padding, bias=bias, backend=conv.backend,
                                        recompute_im2col=conv.recompute_im2col,
                                        residual_first=add.parents[0] is residual)
        if node is root:
            root = replacement
        replace_node(node, replacement)
        for stale in (add, conv):  # the replaced nodes leave their parents' children lists
            for parent in stale.parents:
                if stale in parent.children:
                    parent.children.remove(stale)
            stale.children = []
        fused += 1
    return root, fused


def batchnorm_activation_groups(nodes):
    """{output node: unit} for the BN(+Add)+ReLU chains whose BN and Add outputs (and BN parameters
    and running statistics) no other node uses (BatchNormActivation, keyed by the ReLU), and for the
    BN+ReLU chains read only by an unpadded max-pool (BatchNormReLUPool, keyed by the max-pool: the
    ReLU output then never reaches memory)."""
    from .ops_basic import Add, ReLU
    from .ops_conv import MaxPool2d_Op
    from .ops_norm import BatchNorm2d_Op, BatchNormActivation, BatchNormReLUPool

    readers = Counter(p for n in nodes for p in n.parents)
    stat_owners = Counter(id(n.running_mean) for n in nodes if type(n) is BatchNorm2d_Op)

    def private(bn):
        return (type(bn) is BatchNorm2d_Op and readers[bn] == 1 and stat_owners[id(bn.running_mean)] == 1
                and all(readers[p] == 1 for p in bn.parents[1:]))

    groups = {}
    pooled = set()
    for pool in nodes:
        if type(pool) is not MaxPool2d_Op or pool.padding != (0, 0):
            continue
        relu = pool.parents[0]
        if type(relu) is not ReLU or readers[relu] != 1 or not private(relu.parents[0]):
            continue
        groups[pool] = BatchNormReLUPool(relu.parents[0], relu, pool)
        pooled.add(relu)
    for relu in nodes:
        if type(relu) is not ReLU or relu in pooled:
            continue
        parent = relu.parents[0]
        add = parent if type(parent) is Add else None
        if add is not None and readers[add] != 1:
            continue
        for bn in (add.parents if add is not None else (parent,)):
            if not private(bn):
                continue
            residual = None if add is None else next((p for p in add.parents if p is not bn), None)
            if residual in bn.parents:
                continue
            groups[relu] = BatchNormActivation(bn, add, relu, residual)
            break
    return groups
